// Persistent BiGEMM forward for d = 64, rd = 128 and contiguous channel groups with C = q_c * 64,
// q_c in {1, 4} (the 28x28x256 stage of OmniWeave-T at radix level 0), one (pair, channel group)
// unit per wave at a time.  q_c = 2 (56x56x128) takes bigemm_fwd_wave16.hip.
//
// Same math and operand packing as the other forward kernels (reference
// omniweave/ops/reference.py:147-171; operand scheme in ow_device.h).  Organisation:
//   * a workgroup of eight waves (one per CU) owns one channel group g: its 48 KB of packed
//     weights (4 chunks of the expanded dimension) are copied to LDS once and read from there by
//     all eight waves;
//   * each wave processes whole units: the 32 tokens of a pair of token groups against all
//     128 expanded rows of group g, so the token side is computed once per unit and no partial
//     sums cross waves — no workgroup barrier after the weight copy;
//   * the q_c workgroups of a team (logical ids q_c m .. q_c m + q_c - 1, one per channel group,
//     placed on one XCD) walk the same contiguous range of pairs, each wave drawing its next pair
//     from its workgroup's LDS counter, so the two waves of a SIMD stay busy to the end whatever
//     their issue priority (the hardware issues from the older wave first: under a fixed split
//     one wave of each SIMD finished its share long before the other);
//   * each wave reads its pair's whole rows (the RMSNorm statistics need all C channels) a pair
//     ahead in the 32x32x16 operand layout (lane = token, 8 channels per 16-byte piece), at
//     q_c = 4 in four batches of one group each during the chunk loop, sums the squares with
//     v_dot2_f32 and writes only its group's columns to its own LDS tile; the other groups'
//     waves read the same rows, which their XCD's L2 serves;
//   * the residual round(x + round(delta)) is written into the tile, which the wave then stores
//     as whole 16-byte row pieces of its group's columns.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "ow_device.h"

namespace ow {
namespace {

constexpr int kD = 64;
constexpr int kRD = 128;
constexpr int kKS = kD / 16;                  // 16-deep K steps over a channel group
constexpr int kMB = kD / 32;                  // 32-channel blocks of the group
constexpr int kNCH = kRD / 32;                // 32-row chunks of the expanded dimension
constexpr int kFrCh = 2 * kKS + 2 * kMB;      // fragments per chunk (B_u'^T, B_v'^T, B_o)
constexpr int kGroupFrags = kNCH * kFrCh;     // 48 fragments = 48 KB per channel group
constexpr int kLdt = kD + 8;                  // tile row stride (elements)
constexpr int kWaves = 8;

struct WaveLds {
  u32x4 w[kGroupFrags][64];        // the group's packed weights
  u32x4 tok_ops[3][64];            // token-side operand rows A_u, A_v, A_o (read per unit)
  uint16_t tile[kWaves][32 * kLdt];  // per wave: the pair's rows, group columns
  float rsc[kWaves][32];           // per wave: RMSNorm scale of each token of the pair
  int32_t rows[kWaves][32];        // per wave: output row of each token (-1: not stored)
  int32_t next_pair;               // the next pair of the team's range
};

// Logical workgroup id such that ids q_c m .. q_c m + q_c - 1 run on one XCD (workgroups are
// dispatched round-robin over the 8 XCDs).
__device__ __forceinline__ int wave_xcd_remap(int bid, int nwg) {
  const int xcd = bid & 7, slot = bid >> 3;
  const int per = nwg >> 3, rem = nwg & 7;
  return (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + slot;
}

// Buffer descriptor of a tensor (raw, no stride): loads past num_records return zero and
// stores there are dropped, so pad rows need no branches; the launcher keeps tensors below
// 2 GiB.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tensor_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, static_cast<int>(bytes), 0x00020000);
}
constexpr uint32_t kOutOfRange = 0x80000000u;  // a byte offset past every buffer

// Position of a pair's first token group 2 pair = b q_s + s (image b, group s of the image).
struct PairPos {
  int32_t b, s;
};

// Position of pair p (wave-uniform).
__device__ __forceinline__ PairPos pair_pos(int32_t p, int32_t q_s) {
  const int32_t t = 2 * p, b = t / q_s;
  return PairPos{b, t - b * q_s};
}

// One pair index of the workgroup's counter, taken by lane 0 (the value is read a unit later,
// through readfirstlane, so the LDS atomic's latency is not waited on).
__device__ __forceinline__ int32_t take_pair(int32_t* counter, int lane) {
  int32_t v = 0;
  if (lane == 0) v = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  return v;
}

// Token-table entries of this lane's token (lane % 32) for the pair at `pos`: only loads here;
// the values are examined a pair later (unit_row), so the loads are not waited on meanwhile.
struct TokEntry {
  int32_t tk, to, b;
};

template <bool OM>
__device__ __forceinline__ TokEntry tok_entry(const ResidentArgs& a, PairPos pos, bool live, int l32) {
  // The pair's second token group (lanes 16..31) is the next group; selects, no branch.
  const int32_t s1 = pos.s + 1;
  const bool wrap = s1 == a.q_s;
  const int32_t s = l32 >= 16 ? (wrap ? 0 : s1) : pos.s;
  const int32_t b = (l32 >= 16 && wrap) ? pos.b + 1 : pos.b;
  TokEntry e;
  e.b = live ? b : a.batch;
  e.tk = a.tok[s * kG + (l32 & 15)];  // s < q_s: in bounds for every pair
  e.to = OM ? a.out_tok[s * kG + (l32 & 15)] : 0;
  return e;
}

// Input row of the entry's token (-1: pad token or past the end), and its output row.
template <bool OM>
__device__ __forceinline__ void unit_row(const ResidentArgs& a, const TokEntry& e, int32_t& in, int32_t& out) {
  // Bitwise conditions and selects: a branch here would make the compiler wait for every
  // outstanding memory operation before reading e.tk.
  const bool ok = (e.b < a.batch) & (e.tk >= 0) & (e.tk < a.n_tok);
  const int32_t base = e.b * a.n_tok;
  in = ok ? base + e.tk : -1;
  out = in;
  if (OM) out = (ok & (e.to >= 0) & (e.to < a.n_tok)) ? base + e.to : -1;
}

// The 16-byte pieces 2 ks + hh (channels 16 ks + 8 hh ..) of this lane's token row, ks < C / 16;
// zeros for row -1.
template <int NV>
__device__ __forceinline__ void load_pieces(__amdgpu_buffer_rsrc_t rx, int32_t row, int channels, int hh,
                                            u32x4 (&v)[NV]) {
  const uint32_t base = row >= 0 ? static_cast<uint32_t>(row) * static_cast<uint32_t>(channels * 2) + 16u * hh
                                 : kOutOfRange;
#pragma unroll
  for (int k = 0; k < NV; ++k) v[k] = __builtin_amdgcn_raw_buffer_load_b128(rx, base + 32u * k, 0, 0);
}

// Pieces 2 (k0 + k) + hh, k < 4, of this lane's token row (one channel group of a d = 64 row):
// one batch of the streamed row read.
__device__ __forceinline__ void load_batch(__amdgpu_buffer_rsrc_t rx, int32_t row, int channels, int hh, int k0,
                                           u32x4 (&v)[4]) {
  const uint32_t base = row >= 0 ? static_cast<uint32_t>(row) * static_cast<uint32_t>(channels * 2) + 16u * hh
                                 : kOutOfRange;
#pragma unroll
  for (int k = 0; k < 4; ++k) v[k] = __builtin_amdgcn_raw_buffer_load_b128(rx, base + 32u * (k0 + k), 0, 0);
}

template <class Ty, int QC, bool OM, bool DROP>
__global__ void __attribute__((amdgpu_flat_work_group_size(64 * kWaves, 64 * kWaves), amdgpu_waves_per_eu(2, 2)))
bigemm_fwd_wave_kernel(ResidentArgs a, int32_t n_pairs) {
  constexpr int C = QC * kD;
  constexpr int NV = C / 16;  // row pieces per lane
  // q_c = 4: the next pair's rows are streamed in four batches (one channel group each) during
  // the chunk loop, reduced to this lane's sum of squares and its group's pieces, instead of
  // being held whole (64 registers) for a unit.
  constexpr bool STREAM = QC == 4;
  constexpr int NX = STREAM ? 4 : NV;  // pieces carried from one unit to the next
  __shared__ __attribute__((aligned(16))) WaveLds sh;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int hh = lane >> 5, l32 = lane & 31;
  const int lid = wave_xcd_remap(blockIdx.x, gridDim.x);
  const int g = lid % QC, team = lid / QC, n_team = static_cast<int>(gridDim.x) / QC;
  const int32_t lo = static_cast<int32_t>(static_cast<int64_t>(team) * n_pairs / n_team);
  const int32_t hi = static_cast<int32_t>(static_cast<int64_t>(team + 1) * n_pairs / n_team);

  // The group's weights into LDS (1 KB per wave and copy), the token operands into LDS.
  {
    const uint16_t* src = a.packed + kHeadElems + static_cast<size_t>(g) * kGroupFrags * kFragElems;
    for (int f = wave; f < kGroupFrags; f += kWaves)
      __builtin_amdgcn_global_load_lds(
          (const __attribute__((address_space(1))) void*)(src + static_cast<size_t>(f) * kFragElems + lane * 8),
          (__attribute__((address_space(3))) void*)(&sh.w[f][0]), 16, 0, 0);
  }
  if (wave < 3) sh.tok_ops[wave][lane] = reinterpret_cast<const u32x4*>(a.packed)[wave * 64 + lane];
  if (threadIdx.x == 0) sh.next_pair = lo;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (lo >= hi) return;

  uint16_t* tile = sh.tile[wave];
  float* rsc = sh.rsc[wave];
  int32_t* rows = sh.rows[wave];
  const uint32_t bytes = static_cast<uint32_t>(static_cast<int64_t>(a.batch) * a.n_tok * C * 2);
  const __amdgpu_buffer_rsrc_t rx = tensor_rsrc(a.x, bytes), ro = tensor_rsrc(a.out, bytes);

  // Drawn pairs: `pend` (lane 0) holds the index taken a unit before it is read; p_ent is the
  // pair whose table entries next_entry returned last.
  int32_t pend = take_pair(&sh.next_pair, lane), p_ent = 0;
  auto next_entry = [&]() {
    p_ent = __builtin_amdgcn_readfirstlane(pend);
    pend = take_pair(&sh.next_pair, lane);
    return tok_entry<OM>(a, pair_pos(p_ent, a.q_s), p_ent < hi, l32);
  };

  // One unit: pair p from xc (this lane's pieces, loaded a unit ago), output row out_c of this
  // lane's token.  `ent` holds the table entries of the next pair (read a unit ago): once xc
  // is in the tile, the next pair's pieces are loaded into xc, and ent takes the entries of
  // the pair after that.
  auto unit = [&](int64_t p, u32x4 (&xc)[NX], float& ssq, TokEntry& ent, int32_t& out_c) {
    int32_t in_n, out_n;
    unit_row<OM>(a, ent, in_n, out_n);

    // RMSNorm scale of this lane's token: its half of the row here (streamed: summed as the
    // batches arrived), the other half in lane l ^ 32.
    float acc = 0.0f;
    if (a.norm) {
      if constexpr (STREAM) {
        acc = ssq;
      } else {
#pragma unroll
        for (int k = 0; k < NV; ++k)
#pragma unroll
          for (int e = 0; e < 4; ++e) acc = Ty::dot2sq(xc[k][e], acc);
      }
      acc += __shfl_xor(acc, 32);
    }
    // The group's columns into the tile (q_c = 1: the row; q_c = 4: the streamed batch of group
    // g, xc[0..3]); the row scale (0 for pad tokens) and output row.
#pragma unroll
    for (int k = 0; k < 4; ++k) *reinterpret_cast<u32x4*>(&tile[l32 * kLdt + 16 * k + 8 * hh]) = xc[k];
    if (hh == 0) {
      const float sc = a.norm ? rms_scale<Ty>(acc / static_cast<float>(C), a.eps) : 1.0f;
      rsc[l32] = sc;
      rows[l32] = out_c;
      // The row scales for the backward: every group's waves form the same value, group 0's
      // write it (out_c is the input row without an output-row table).
      if (a.rs_out && g == 0 && out_c >= 0) a.rs_out[out_c] = sc;
    }
    if constexpr (STREAM)
      ssq = 0.0f;  // the next pair's batches are read during the chunk loop
    else
      load_pieces<NV>(rx, in_n, C, hh, xc);  // the next pair, a unit ahead of its use
    ent = next_entry();
    wave_lds_sync();

    // Token side.  Lane slots j of the token operand are tokens 16 tg + kord(j, hh) of its
    // group tg: two runs of four scales.
    // The token operands are read per unit from LDS rather than kept live through the loop.
    const u32x4 fAu = sh.tok_ops[0][lane], fAv = sh.tok_ops[1][lane];
    u32x4 bu = fAu, bv = fAv;
    if (a.norm) {
      const float* r8 = &rsc[16 * ((lane >> 4) & 1) + 4 * hh];
      bu = scale8<Ty>(fAu, r8);
      bv = scale8<Ty>(fAv, r8);
    }
    u32x4 Pu[kKS], Pv[kKS];
    {
      u32x4 xk[kKS / 2][2];  // X^T operands by transposed reads
      const uint32_t tb = lds_addr(tile);
      pair_xt_tr<kKS>([&](int r, int c) { return tb + 2u * static_cast<uint32_t>(r * kLdt + c); }, lane, xk);
      pair_token_side_mma<Ty, kKS>(xk, bu, bv, lane, Pu, Pv);
    }

    // Channel side over the four chunks of the expanded dimension, software-pipelined: step e
    // issues chunk e + 1's U'/V' products with two of chunk e's gate values after each of them
    // (the gate's VALU work runs while the products execute), then chunk e's W += Z B_o
    // products.  The weight fragments come from LDS DEPTH reads ahead of their MFMAs
    // (lds_read_async: no compiler wait per read; lds_wait before each use).
    f32x16 W[kMB] = {};
    const uint32_t wbase = lds_addr(&sh.w[0][lane]);
    constexpr int DEPTH = 4;
    u32x4 vb[4];  // streamed batch in flight
    auto step = [&](auto e_tag, f32x16& Un, f32x16& Vn, const f32x16& Uc, const f32x16& Vc) {
      constexpr int E = decltype(e_tag)::value;      // chunk of the gate and B_o products; -1: none
      if constexpr (STREAM) {
        // Step E + 1 takes in batch E (channel group E of the next pair's rows, read a step ago)
        // and reads batch E + 1.
        constexpr int T = E + 1;
        if constexpr (T >= 1) {
#pragma unroll
          for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int e = 0; e < 4; ++e) ssq = Ty::dot2sq(vb[k][e], ssq);
          if (T - 1 == g) {
#pragma unroll
            for (int k = 0; k < 4; ++k) xc[k] = vb[k];
          }
        }
        // (the reads after the batch is consumed: one batch of registers in flight)
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (T < QC) load_batch(rx, in_n, C, hh, 4 * T, vb);
      }
      constexpr int NU = E + 1 < kNCH ? 2 * kKS : 0;  // U'/V' products of chunk E + 1 (U, V alternate)
      constexpr int NO = E >= 0 ? 2 * kMB : 0;        // B_o products of chunk E
      constexpr int NF = NU + NO;
      static_assert(NU == 0 || NO == 0 || 2 * NU == 16, "two gate values per U'/V' product");
      auto read = [&](auto ic) -> u32x4 {
        constexpr int i = decltype(ic)::value;
        // B_o products in the order (block 0, K step 0), (block 1, 0), (0, 1), (1, 1): the two
        // accumulators alternate, so no product waits on the one issued right before it.
        constexpr int j = i - NU;
        constexpr int f = i < NU ? (E + 1) * kFrCh + ((i & 1) ? kKS + i / 2 : i / 2)
                                 : E * kFrCh + 2 * kKS + 2 * (j % kMB) + j / kMB;
        return lds_read_async<f * kFragElems * 2>(wbase);
      };
      u32x4 fr[DEPTH];
      static_for<0, DEPTH>([&](auto ic) {
        if constexpr (decltype(ic)::value < NF) fr[decltype(ic)::value] = read(ic);
      });
      // Gate values k = 8 s + 2 q + h of chunk E -> Z[s] word q, half h.
      u32x4 Z[2];
      float zl = 0.0f;
      auto gate = [&](auto kc) {
        constexpr int k = decltype(kc)::value;
        const float z = silu_gate(Uc[k], Vc[k]);
        if constexpr (k % 2 == 0)
          zl = z;
        else
          Z[k / 8][(k % 8) / 2] = Ty::pack2(zl, z);
      };
      if constexpr (NO > 0 && NU == 0) static_for<0, 16>(gate);
      if constexpr (NU > 0) {
        Un = f32x16{};
        Vn = f32x16{};
      }
      static_for<0, NF>([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        constexpr int after = NF - 1 - i < DEPTH - 1 ? NF - 1 - i : DEPTH - 1;
        lds_wait<after>(fr[i % DEPTH]);
        if constexpr (i < NU) {
          if constexpr (i % 2 == 0)
            Un = Ty::mma32(fr[i % DEPTH], Pu[i / 2], Un);
          else
            Vn = Ty::mma32(fr[i % DEPTH], Pv[i / 2], Vn);
        } else {
          constexpr int j = i - NU;
          W[j % kMB] = Ty::mma32(Z[j / kMB], fr[i % DEPTH], W[j % kMB]);
        }
        if constexpr (i + DEPTH < NF) fr[i % DEPTH] = read(std::integral_constant<int, i + DEPTH>{});
        if constexpr (NO > 0 && i < NU) {
          gate(std::integral_constant<int, 2 * i>{});
          gate(std::integral_constant<int, 2 * i + 1>{});
        }
      });
    };
    f32x16 Ua, Va, Ub = {}, Vb = {};
    step(std::integral_constant<int, -1>{}, Ua, Va, Ub, Vb);
    step(std::integral_constant<int, 0>{}, Ub, Vb, Ua, Va);
    step(std::integral_constant<int, 1>{}, Ua, Va, Ub, Vb);
    step(std::integral_constant<int, 2>{}, Ub, Vb, Ua, Va);
    step(std::integral_constant<int, 3>{}, Ua, Va, Ub, Vb);
    static_assert(kNCH == 4, "four chunks: the step sequence above");

    // delta^T = W^T A_o^T (lane = token row), rounded, plus x (and the drop-path scale), into
    // the tile in place as 8-byte pieces: the token side has read it.
    f32x16 dl[kMB];
    mfma_drain();
    pair_output_t<Ty, kMB>(W, sh.tok_ops[2][lane], lane, dl);
    mfma_drain();
    float sc = 1.0f;
    if constexpr (DROP) {
      const int64_t tg = 2 * p + ((lane >> 4) & 1);  // the lane's token group
      const int64_t b = tg / a.q_s;
      sc = a.drop_scale[b < a.batch ? b : a.batch - 1];
    }
#pragma unroll
    for (int mb = 0; mb < kMB; ++mb) {
      auto at = [&](int q) { return &tile[l32 * kLdt + 32 * mb + 8 * q + 4 * hh]; };
      if (a.residual)
        pair_store_block_t<Ty, true, DROP>(dl[mb], at, sc);
      else
        pair_store_block_t<Ty, false, DROP>(dl[mb], at, sc);
    }
    wave_lds_sync();

    // The tile's rows to memory: 32 rows x 8 pieces of the group's columns, 4 per lane; pad
    // rows go past the buffer.
    u32x4 ov[4];
    int32_t orow[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = (lane >> 3) + 8 * j;
      orow[j] = rows[r];
      ov[j] = *reinterpret_cast<const u32x4*>(&tile[r * kLdt + (lane & 7) * 8]);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t rb = orow[j] >= 0 ? static_cast<uint32_t>(orow[j]) * static_cast<uint32_t>(C * 2) : kOutOfRange;
      __builtin_amdgcn_raw_buffer_store_b128(ov[j], ro, rb + 2u * (kD * g + (lane & 7) * 8), 0, 0);
    }
    // The next unit overwrites the tile and the row table: every lane's reads above are done.
    wave_lds_sync();
    out_c = out_n;
  };

  u32x4 x[NX];
  float ssq = 0.0f;
  TokEntry ent = next_entry();
  const int32_t p_first = p_ent;
  int32_t in0, out_c;
  unit_row<OM>(a, ent, in0, out_c);
  if constexpr (STREAM) {
#pragma unroll
    for (int t = 0; t < QC; ++t) {
      u32x4 v[4];
      load_batch(rx, in0, C, hh, 4 * t, v);
#pragma unroll
      for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int e = 0; e < 4; ++e) ssq = Ty::dot2sq(v[k][e], ssq);
      if (t == g) {
#pragma unroll
        for (int k = 0; k < 4; ++k) x[k] = v[k];
      }
    }
  } else {
    load_pieces<NV>(rx, in0, C, hh, x);
  }
  ent = next_entry();
  // ent holds the entries of the pair after the current one; the unit reads its rows and draws
  // the next.
  int32_t p = p_first;
#pragma unroll 1
  while (p < hi) {
    const int32_t following = p_ent;
    unit(p, x, ssq, ent, out_c);
    p = following;
  }
}

template <class Ty, int QC>
int launch_qc(const ResidentArgs& a, hipStream_t stream) {
  // One workgroup of eight waves per CU (~89 KB of LDS): whole teams of QC workgroups, each team
  // a contiguous pair range of at least eight pairs where the batch allows.
  const int32_t n_pairs = a.n_pairs;
  const int64_t teams_needed = (static_cast<int64_t>(n_pairs) + kWaves - 1) / kWaves;
  int64_t grid = static_cast<int64_t>(device_cus());
  if (grid / QC > teams_needed) grid = teams_needed * QC;
  grid -= grid % QC;
  if (grid <= 0) return OW_OK;
  const dim3 g(static_cast<unsigned>(grid)), b(64 * kWaves);
  if (a.out_tok && a.drop_scale) return fail(OW_ERR_UNSUPPORTED, "an output-row table with a drop-path scale");
  if (a.out_tok)
    hipLaunchKernelGGL((bigemm_fwd_wave_kernel<Ty, QC, true, false>), g, b, 0, stream, a, n_pairs);
  else if (a.drop_scale)
    hipLaunchKernelGGL((bigemm_fwd_wave_kernel<Ty, QC, false, true>), g, b, 0, stream, a, n_pairs);
  else
    hipLaunchKernelGGL((bigemm_fwd_wave_kernel<Ty, QC, false, false>), g, b, 0, stream, a, n_pairs);
  return hip_status(hipGetLastError(), "bigemm_fwd_wave_kernel launch");
}

template <class Ty>
int launch_ty(const ResidentArgs& a, hipStream_t stream) {
  switch (a.q_c) {
    case 1: return launch_qc<Ty, 1>(a, stream);
    case 4: return launch_qc<Ty, 4>(a, stream);
    default: return fail(OW_ERR_UNSUPPORTED, "wave-unit forward needs q_c in {1, 4} (got %d)", a.q_c);
  }
}

}  // namespace

bool wave_supported(int32_t d, int32_t rd, int32_t channels, int32_t q_c, int32_t radix_level, int64_t x_elems) {
  // Byte offsets are 32-bit and kOutOfRange (2^31) must lie past x and out.  q_c = 2 runs on
  // bigemm_fwd_wave16.hip; interleaved q_c = 4 groups (radix levels >= 1) on the resident kernel.
  return d == kD && rd == kRD && (q_c == 1 || (q_c == 4 && radix_level == 0)) && channels == q_c * kD &&
         x_elems * 2 < (int64_t(1) << 31);
}

int launch_fwd_wave(const ResidentArgs& a, int32_t dtype, hipStream_t stream) {
  if (dtype == OW_DTYPE_BF16) return launch_ty<BF16>(a, stream);
  if (dtype == OW_DTYPE_F16) return launch_ty<F16>(a, stream);
  return fail(OW_ERR_UNSUPPORTED, "unsupported dtype %d", dtype);
}

}  // namespace ow
