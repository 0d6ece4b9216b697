// Forward for d = 64, rd = 128, C = 64 q_c with q_c in {2, 4} (the 56x56x128 and 28x28x256
// stages of OmniWeave-T), with contiguous channel groups or the interleaved groups of radix
// levels >= 1, on 16x16 MFMAs.
//
// Same math as the other forward kernels (reference omniweave/ops/reference.py:147-171, the
// block's RMSNorm and residual omniweave/models/block.py:83-108); the folded operands are those
// of ow_device.h (U' = -log2(e) w U, V' = -ln(2) w V, SiLU(U) V = U' V' / (1 + 2^U')).
// Organisation:
//   * a unit is one 16-token group of one image and two channel groups (q_c = 2: both): a wave
//     reads the unit's 16 rows once (four rows per 16-byte-per-lane load, so every load covers
//     four whole rows, or their halves), forms the RMSNorm scales from them and writes its two
//     groups' columns into its LDS tile, group-major (interleaved groups are split with
//     v_perm_b32);
//   * q_c = 4: the workgroups come in pairs on one XCD, blocks 16 m + x and 16 m + 8 + x (the
//     dispatcher places block b on XCD b % 8), which walk the same unit range: half ph = 0 of the
//     pair computes the groups of channels 0 .. 127 (contiguous) or of residues 0, 1 mod 4
//     (interleaved), half 1 the others.  Each reads whole rows for the RMSNorm sums; the
//     second read of a row comes from the XCD's L2.  Interleaved halves store 4-byte words
//     (the two residues of a word are the half's two groups), one row per store instruction;
//   * per group: the token side P^T = X^T (A diag r)^T on v_mfma_f32_16x16x16 (A operand by
//     transposed LDS reads of the tile), the channel side on v_mfma_f32_16x16x32 over four
//     32-row chunks of the expanded dimension (U'^T, V'^T, the gate, W += Z B_o), the output
//     delta^T = W^T A_o^T on v_mfma_f32_16x16x16, lane = token, four consecutive channels per
//     register quad; rounded, plus x, written back into the tile;
//   * the tile's rows then leave as 16-byte row pieces (q_c = 2 interleaved groups re-joined with
//     v_perm_b32): four stores of four rows each;
//   * the accumulator of each 16x16 product is, pair of accumulators by pair, the next product's
//     operand: its rows 4h + i (h = lane / 16) are the K slots kord16(j, h) = 16 (j / 4) + 4h +
//     j % 4 of the next 16x16x32 operand, the order the packed weights use (pack16_kernel);
//   * twelve waves (three per SIMD) per CU, two groups' packed weights (96 KB) in LDS, units
//     drawn one at a time from the workgroup's range through an LDS counter.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "ow_device.h"

namespace ow {
namespace {

constexpr int kD = 64;
constexpr int kRD = 128;
constexpr int kC = 2 * kD;              // tile width: the two groups a workgroup computes
constexpr int kNCH = kRD / 32;          // 4 chunks of 32 expanded rows
constexpr int kFr = 12;                 // 16x16x32 fragments per chunk: BU(eb, s) x4, BV(eb, s) x4, BO(cb) x4
constexpr int kGroupFr = kNCH * kFr;    // 48 fragments (48 KB) per channel group
constexpr int kWaves = 12;
constexpr int kThreads = 64 * kWaves;
// Elements of the packed weights' 32x32x16 part, before the second section.
constexpr int main_elems(int q_c) { return kHeadElems + q_c * kNCH * 12 * kFragElems; }

struct Wave16Lds {
  u32x4 w[2 * kGroupFr][64];       // the two groups' 16x16x32 fragments
  u32x2 tok_ops[3][64];            // A_u, A_v, A_o: lane l holds A[l % 16][4 (l / 16) .. + 3]
  uint16_t tile[kWaves][16 * kC];  // per wave: the unit's 16 rows, group-major columns
  float rsc[kWaves][16];           // RMSNorm scale of each token of the unit
  int32_t rows[kWaves][16];        // output row of each token (-1: not stored)
  int32_t next_unit;               // the next unit of the workgroup's range
};

// Element offset of (row r, column c) in a tile: 16-byte pieces swizzled by the row, so the four
// rows of a transposed read and the sixteen rows of a residual column hit different banks.
__device__ __forceinline__ int toff(int r, int c) { return r * kC + ((((c >> 3) ^ (r & 7))) << 3) + (c & 7); }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t tensor_rsrc16(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, static_cast<int>(bytes), 0x00020000);
}
constexpr uint32_t kOutOfRange = 0x80000000u;  // a byte offset past every buffer below 2 GiB

template <class Ty>
__device__ __forceinline__ u32x2 scale4(u32x2 a, float4 r) {
  return u32x2{Ty::pack2(Ty::to_f32(lo16(a[0])) * r.x, Ty::to_f32(hi16(a[0])) * r.y),
               Ty::pack2(Ty::to_f32(lo16(a[1])) * r.z, Ty::to_f32(hi16(a[1])) * r.w)};
}

// Two 16x16 accumulators (rows 4h + i of blocks b0 and b1) as one 16x16x32 operand.
template <class Ty>
__device__ __forceinline__ u32x4 join16(const f32x4& b0, const f32x4& b1) {
  return u32x4{Ty::pack2(b0[0], b0[1]), Ty::pack2(b0[2], b0[3]), Ty::pack2(b1[0], b1[1]), Ty::pack2(b1[2], b1[3])};
}

// The chunk loop's MFMAs in issue order: step E = -1 .. 3 issues the 8 U'/V' products of chunk
// E + 1 (U(eb, s) and V(eb, s) in the order (0, 0), (1, 0), (0, 1), (1, 1): each accumulator's
// second product comes four after its first), then the 4 B_o products of chunk E.
constexpr int w16_nu(int e) { return e + 1 < kNCH ? 8 : 0; }
constexpr int w16_no(int e) { return e >= 0 ? 4 : 0; }
constexpr int w16_first(int e) { return e <= -1 ? 0 : w16_first(e - 1) + w16_nu(e - 1) + w16_no(e - 1); }
constexpr int kLoop16 = w16_first(kNCH);
// Fragment of the m-th MFMA within the group's 48.
constexpr int w16_frag(int m, int e = -1) {
  return m < w16_nu(e) + w16_no(e)
             ? (m < w16_nu(e) ? (e + 1) * kFr + ((m & 1) ? 4 : 0) + 2 * ((m >> 1) & 1) + (m >> 2)
                              : e * kFr + 8 + (m - w16_nu(e)))
             : w16_frag(m - w16_nu(e) - w16_no(e), e + 1);
}
static_assert(kLoop16 == 48, "chunk-loop MFMAs");
constexpr int kDepth16 = 4;  // fragment reads in flight ahead of their MFMAs

// Token-table entry of token l16 of unit (b, s).
struct UnitEntry {
  int32_t tk, to, b;
};

template <class Ty, int QC, bool SG, bool OM, bool DROP>
__global__ void __attribute__((amdgpu_flat_work_group_size(kThreads, kThreads), amdgpu_waves_per_eu(3, 3)))
bigemm_fwd_wave16_kernel(ResidentArgs a, int32_t n_units) {
  static_assert(QC == 2 || QC == 4, "two or four channel groups");
  constexpr int kCT = QC * kD;  // channels of a row of x and out
  __shared__ __attribute__((aligned(16))) Wave16Lds sh;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int h = lane >> 4, l16 = lane & 15;
  // q_c = 4: half ph of the XCD pair (see above) and the pair's unit range rb of gridDim / 2.
  const int ph = QC == 4 ? static_cast<int>((blockIdx.x >> 3) & 1) : 0;
  const int64_t n_ranges = QC == 4 ? gridDim.x / 2 : gridDim.x;
  const int64_t rb = QC == 4 ? ((blockIdx.x & 7) | ((blockIdx.x >> 4) << 3)) : blockIdx.x;
  const int32_t lo = static_cast<int32_t>(rb * n_units / n_ranges);
  const int32_t hi = static_cast<int32_t>((rb + 1) * n_units / n_ranges);
  // q_c = 2 interleaved groups (group q = channels res_q + 2 t): the region holding the even channels.
  const int q_even = (QC == 2 && SG) ? (__builtin_amdgcn_readfirstlane(a.chan[0]) & 1) : 0;
  // The channel groups of the tile's two regions: q_c = 2 both, in order; q_c = 4 contiguous
  // groups 2 ph, 2 ph + 1; q_c = 4 interleaved (group q = channels (rot + q) % 4 + 4 t) the
  // groups of residues 2 ph and 2 ph + 1.
  int q0 = 0;
  if constexpr (QC == 4) {
    const int rot = SG ? (__builtin_amdgcn_readfirstlane(a.chan[0]) & 3) : 0;
    q0 = (2 * ph - rot) & 3;
  }
  const int q1 = QC == 4 ? ((q0 + 1) & 3) : 1;

  {
    const uint16_t* src = a.packed + main_elems(QC);
    for (int f = wave; f < 2 * kGroupFr; f += kWaves) {
      const int q = f < kGroupFr ? q0 : q1;
      const int ff = f < kGroupFr ? f : f - kGroupFr;
      __builtin_amdgcn_global_load_lds(
          (const __attribute__((address_space(1))) void*)(src + static_cast<size_t>(q * kGroupFr + ff) * kFragElems +
                                                          lane * 8),
          (__attribute__((address_space(3))) void*)(&sh.w[f][0]), 16, 0, 0);
    }
  }
  if (wave < 3) {
    // The 32x32x16 head row of lane l16 + 32 (h & 1) holds A[l16][4 (h & 1) + 8 (j / 4) + j % 4].
    const int src_lane = l16 + 32 * (h & 1);
    sh.tok_ops[wave][lane] = *reinterpret_cast<const u32x2*>(a.packed + wave * kFragElems + src_lane * 8 + 4 * (h >> 1));
  }
  if (threadIdx.x == 0) sh.next_unit = lo;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (lo >= hi) return;

  uint16_t* tile = sh.tile[wave];
  const uint32_t bytes = static_cast<uint32_t>(static_cast<int64_t>(a.batch) * a.n_tok * kCT * 2);
  const __amdgpu_buffer_rsrc_t rx = tensor_rsrc16(a.x, bytes), ro = tensor_rsrc16(a.out, bytes);

  // Units are drawn one at a time, the next one while the current one's first group is computed
  // (its rows are read during the second group): a wave holds at most one unit it has not
  // started, so at the end of the range no wave sits on units that idle waves could take.
  int32_t u_ent = 0;
  auto next_entry = [&]() {
    int32_t t = 0;
    if (lane == 0) t = __hip_atomic_fetch_add(&sh.next_unit, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    u_ent = __builtin_amdgcn_readfirstlane(t);
    const int32_t b = u_ent / a.q_s, s = u_ent - b * a.q_s;  // s < q_s for any unit index
    UnitEntry e;
    e.b = u_ent < hi ? b : a.batch;
    e.tk = a.tok[s * kG + l16];
    e.to = OM ? a.out_tok[s * kG + l16] : 0;
    return e;
  };
  // Input and output row of token l16 (-1: pad token or past the end).
  auto unit_row = [&](const UnitEntry& e, int32_t& in, int32_t& out) {
    const bool ok = (e.b < a.batch) & (e.tk >= 0) & (e.tk < a.n_tok);
    const int32_t base = e.b * a.n_tok;
    in = ok ? base + e.tk : -1;
    out = in;
    if (OM) out = (ok & (e.to >= 0) & (e.to < a.n_tok)) ? base + e.to : -1;
  };
  // Rows of the unit whose token-l16 input row is `in`: load k holds token 4k + h, piece l16
  // (q_c = 4: xr the piece of the 256-byte half at byte own_off, xo of the other half).
  const uint32_t own_off = (QC == 4 && !SG) ? 256u * ph : 0u;
  u32x4 xr[4], xo[QC == 4 ? 4 : 1];
  auto load_rows = [&](int32_t in) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int32_t row = __shfl(in, 4 * k + h, 16);
      const uint32_t off = row >= 0 ? static_cast<uint32_t>(row) * (kCT * 2u) + 16u * l16 : kOutOfRange;
      xr[k] = __builtin_amdgcn_raw_buffer_load_b128(rx, off + own_off, 0, 0);
      if constexpr (QC == 4) xo[k] = __builtin_amdgcn_raw_buffer_load_b128(rx, off + (256u - own_off), 0, 0);
    }
  };

  const uint32_t tile_base = lds_addr(tile);
  f32x4 W[4];
  u32x4 fr[kDepth16];
  u32x4 Pu[2], Pv[2];

  // Channel side of group g (fragments from w[48 g ..]): software-pipelined chunk loop, the
  // weight fragments read kDepth16 ahead of their MFMAs.
  auto channel_side = [&](int g) {
    const uint32_t wbase = lds_addr(&sh.w[g * kGroupFr][lane]);
    auto frag_read = [&](auto mc) -> u32x4 {
      return lds_read_async<w16_frag(decltype(mc)::value) * kFragElems * 2>(wbase);
    };
    static_for<0, kDepth16>([&](auto mc) { fr[decltype(mc)::value] = frag_read(mc); });
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) W[cb] = f32x4{};
    auto step = [&](auto e_tag, f32x4 (&Un)[2], f32x4 (&Vn)[2], const f32x4 (&Uc)[2], const f32x4 (&Vc)[2]) {
      constexpr int E = decltype(e_tag)::value;
      constexpr int NU = w16_nu(E), NO = w16_no(E), NF = NU + NO, M0 = w16_first(E);
      float z[8];
      auto gate = [&](auto kc) {
        constexpr int k = decltype(kc)::value;
        z[k] = silu_gate(Uc[k >> 2][k & 3], Vc[k >> 2][k & 3]);
      };
      if constexpr (NO > 0 && NU == 0) static_for<0, 8>(gate);
      if constexpr (NU > 0) {
        Un[0] = Un[1] = Vn[0] = Vn[1] = f32x4{};
      }
      u32x4 Z = {};
      static_for<0, NF>([&](auto ic) {
        constexpr int i = decltype(ic)::value, m = M0 + i;
        constexpr int after = kLoop16 - 1 - m < kDepth16 - 1 ? kLoop16 - 1 - m : kDepth16 - 1;
        if constexpr (i == NU && NO > 0) Z = u32x4{Ty::pack2(z[0], z[1]), Ty::pack2(z[2], z[3]), Ty::pack2(z[4], z[5]),
                                                  Ty::pack2(z[6], z[7])};
        lds_wait<after>(fr[m % kDepth16]);
        if constexpr (i < NU) {
          constexpr int eb = (i >> 1) & 1, sk = i >> 2;
          if constexpr (i & 1)
            Vn[eb] = Ty::mma16k32(fr[m % kDepth16], Pv[sk], Vn[eb]);
          else
            Un[eb] = Ty::mma16k32(fr[m % kDepth16], Pu[sk], Un[eb]);
        } else {
          constexpr int cb = i - NU;
          W[cb] = Ty::mma16k32(Z, fr[m % kDepth16], W[cb]);
        }
        if constexpr (m + kDepth16 < kLoop16) fr[m % kDepth16] = frag_read(std::integral_constant<int, m + kDepth16>{});
        if constexpr (NO > 0 && i < NU) gate(std::integral_constant<int, i>{});
      });
    };
    f32x4 Ua[2], Va[2], Ub[2] = {}, Vb[2] = {};
    step(std::integral_constant<int, -1>{}, Ua, Va, Ub, Vb);
    step(std::integral_constant<int, 0>{}, Ub, Vb, Ua, Va);
    step(std::integral_constant<int, 1>{}, Ua, Va, Ub, Vb);
    step(std::integral_constant<int, 2>{}, Ub, Vb, Ua, Va);
    step(std::integral_constant<int, 3>{}, Ua, Va, Ub, Vb);
    static_assert(kNCH == 4, "four chunks: the step sequence above");
  };

  // Prologue: the first unit's entries and rows.
  UnitEntry ent = next_entry();
  int32_t u_cur = u_ent;
  int32_t in_c, out_c, in_n = -1, out_n = -1;
  unit_row(ent, in_c, out_c);
  load_rows(in_c);

#pragma unroll 1
  while (u_cur < hi) {
    // RMSNorm scales of the unit's tokens, one per lane: row 4 (l16 % 4) + h.  part[k] is the
    // lane's partial sum of squares of row 4 k + h; a transposed reduction keeps, across lane
    // bit 0 and then bit 1, the partials of the rows whose k matches the lane's bits, then adds
    // the four quads of the 16-lane row (rotations by 4 and 8).
    float part[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (a.norm) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
#pragma unroll
        for (int e = 0; e < 4; ++e) part[k] = Ty::dot2sq(xr[k][e], part[k]);
        if constexpr (QC == 4) {
#pragma unroll
          for (int e = 0; e < 4; ++e) part[k] = Ty::dot2sq(xo[k][e], part[k]);
        }
      }
    }
    const bool b0 = (lane & 1) != 0, b1 = (lane & 2) != 0;
    const float q0 = (b0 ? part[1] : part[0]) + dpp_f32<0xb1, 0xf>(b0 ? part[0] : part[1]);  // quad_perm 1,0,3,2
    const float q1 = (b0 ? part[3] : part[2]) + dpp_f32<0xb1, 0xf>(b0 ? part[2] : part[3]);
    float mine = (b1 ? q1 : q0) + dpp_f32<0x4e, 0xf>(b1 ? q0 : q1);  // quad_perm 2,3,0,1
    mine += dpp_f32<0x124, 0xf>(mine);  // row_ror:4
    mine += dpp_f32<0x128, 0xf>(mine);  // row_ror:8
    const float sc = a.norm ? rms_scale<Ty>(mine / static_cast<float>(kCT), a.eps) : 1.0f;
    if (l16 < 4) sh.rsc[wave][4 * l16 + h] = sc;
    // The rows into the tile, group-major; scales and output rows into LDS.
    if constexpr (QC == 4 && SG) {
      // Piece p (channels 8 p .. 8 p + 7): residue 2 ph + j holds channels 8 p + 2 ph + j and
      // 8 p + 2 ph + j + 4, i.e. columns 2 p, 2 p + 1 of region j, the halves j of words ph and
      // ph + 2.  Row t = 4 k + h: toff(t, 2 p) = 512 k + o[k % 2][p / 16], with the lane's four
      // offsets o formed once (t & 7 = 4 (k % 2) + h); region 1 is 64 elements further.
      int pl = l16;
      asm volatile("" : "+v"(pl));
      int o[2][2];
#pragma unroll
      for (int kp = 0; kp < 2; ++kp)
#pragma unroll
        for (int j = 0; j < 2; ++j) o[kp][j] = h * kC + ((((2 * (16 * j + pl)) >> 3) ^ (4 * kp + h)) << 3) + ((2 * pl) & 7);
      // Word ph of a word pair by one v_perm_b32 (byte selector in a scalar register; a plain
      // ph ? a : b would become a dynamic vector index and a chain of selects).
      uint32_t wsel = ph ? 0x07060504u : 0x03020100u;
      asm volatile("" : "+s"(wsel));
#pragma unroll
      for (int k = 0; k < 4; ++k) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const u32x4& v = j == 0 ? xr[k] : xo[k];
          const uint32_t wl = __builtin_amdgcn_perm(v[1], v[0], wsel), wh = __builtin_amdgcn_perm(v[3], v[2], wsel);
          uint16_t* dst = tile + 4 * k * kC + o[k & 1][j];
          *reinterpret_cast<uint32_t*>(dst) = __builtin_amdgcn_perm(wh, wl, 0x05040100u);
          *reinterpret_cast<uint32_t*>(dst + 64) = __builtin_amdgcn_perm(wh, wl, 0x07060302u);
        }
      }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int t = 4 * k + h;
      if constexpr (QC == 4 && SG) {
        // (written above)
      } else if constexpr (SG) {
        *reinterpret_cast<u32x2*>(&tile[toff(t, 64 * q_even + 4 * l16)]) = strided_pack<4>(xr[k], 0);
        *reinterpret_cast<u32x2*>(&tile[toff(t, 64 * (q_even ^ 1) + 4 * l16)]) = strided_pack<4>(xr[k], 1);
      } else {
        *reinterpret_cast<u32x4*>(&tile[toff(t, 8 * l16)]) = xr[k];
      }
    }
    if (h == 0) sh.rows[wave][l16] = out_c;
    wave_lds_sync();
    // The row scales for the backward (out_c is the input row without an output-row table);
    // q_c = 4: half 0 of the pair writes them.
    if (a.rs_out && ph == 0 && h == 0 && out_c >= 0) a.rs_out[out_c] = sh.rsc[wave][l16];

    // Token-side operands: lane l holds (A diag r)^T column l16, rows 4h .. 4h + 3.
    const float4 r4 = *reinterpret_cast<const float4*>(&sh.rsc[wave][4 * h]);
    const u32x2 bu = a.norm ? scale4<Ty>(sh.tok_ops[0][lane], r4) : sh.tok_ops[0][lane];
    const u32x2 bv = a.norm ? scale4<Ty>(sh.tok_ops[1][lane], r4) : sh.tok_ops[1][lane];
    float dsc = 1.0f;
    if constexpr (DROP) {
      const int32_t b = u_cur / a.q_s;
      dsc = a.drop_scale[b < a.batch ? b : a.batch - 1];
    }

#pragma unroll 1
    for (int g = 0; g < 2; ++g) {
      // Token side: P^T block b (16 channels) = X^T (A diag r)^T on 16x16x16 products.
      {
        f32x4 pu[4], pv[4];
        const f32x4 zero = {};
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const u32x2 xt = lds_read_tr16(tile_base + 2u * toff(4 * h + (l16 >> 2), 64 * g + 16 * b + 4 * (l16 & 3)));
          pu[b] = Ty::mma16(xt, bu, zero);
          pv[b] = Ty::mma16(xt, bv, zero);
        }
#pragma unroll
        for (int sk = 0; sk < 2; ++sk) {
          Pu[sk] = join16<Ty>(pu[2 * sk], pu[2 * sk + 1]);
          Pv[sk] = join16<Ty>(pv[2 * sk], pv[2 * sk + 1]);
        }
      }
      if (g == 0) ent = next_entry();  // the next unit, read during the first group's channel side
      channel_side(g);
      // delta^T block cb = W^T A_o^T (lane = token l16, channels 16 cb + 4h + i), rounded, times
      // the drop-path scale, plus x, back into the tile.
      mfma_drain();
      f32x4 dl[4];
      {
        const u32x2 ao = sh.tok_ops[2][lane];
        const f32x4 zero = {};
#pragma unroll
        for (int cb = 0; cb < 4; ++cb)
          dl[cb] = Ty::mma16(u32x2{Ty::pack2(W[cb][0], W[cb][1]), Ty::pack2(W[cb][2], W[cb][3])}, ao, zero);
      }
      mfma_drain();
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) {
        uint32_t v0 = Ty::pack2(dl[cb][0], dl[cb][1]), v1 = Ty::pack2(dl[cb][2], dl[cb][3]);
        if constexpr (DROP) {
          v0 = Ty::pack2(Ty::to_f32(lo16(v0)) * dsc, Ty::to_f32(hi16(v0)) * dsc);
          v1 = Ty::pack2(Ty::to_f32(lo16(v1)) * dsc, Ty::to_f32(hi16(v1)) * dsc);
        }
        u32x2* p = reinterpret_cast<u32x2*>(&tile[toff(l16, 64 * g + 16 * cb + 4 * h)]);
        if (a.residual) {
          const u32x2 x = *p;
          v0 = add_residual2<Ty>(x[0], v0);
          v1 = add_residual2<Ty>(x[1], v1);
        }
        *p = u32x2{v0, v1};
      }
      if (g == 0) {  // the next unit's rows, read during the second group
        unit_row(ent, in_n, out_n);
        load_rows(in_n);
      }
    }

    // The tile's rows to memory; pad rows go past the buffer.
    wave_lds_sync();
    if constexpr (QC == 4 && SG) {
      // Store r writes row r's words of this half: lane l the residues 2 ph, 2 ph + 1 of
      // channel block 4 l, i.e. columns l of both regions, at byte 8 l + 4 ph of the row.
      // (The lane id passes through an empty asm, so that the compiler forms these addresses
      // here instead of keeping 32 of them live across the loop.)
      int ln = lane;
      asm volatile("" : "+v"(ln));
      const int32_t my_row = sh.rows[wave][ln & 15];
      // toff(r, ln) = 128 r + cb[r & 7], toff(r, 64 + ln) = toff(r, ln) + 64.
      int cb[8];
#pragma unroll
      for (int m = 0; m < 8; ++m) cb[m] = ((((ln >> 3) ^ m)) << 3) + (ln & 7);
      const uint32_t vb = 8u * ln + 4u * ph;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int32_t orow = __builtin_amdgcn_readlane(my_row, r);
        const uint16_t* tr = tile + r * kC + cb[r & 7];
        const uint32_t v = static_cast<uint32_t>(tr[0]) | (static_cast<uint32_t>(tr[64]) << 16);
        const uint32_t off = (orow >= 0 ? static_cast<uint32_t>(orow) * (kCT * 2u) : kOutOfRange) + vb;
        __builtin_amdgcn_raw_buffer_store_b32(v, ro, off, 0, 0);
      }
    }
#pragma unroll
    for (int k = 0; k < (QC == 4 && SG ? 0 : 4); ++k) {
      const int t = 4 * k + h;
      const int32_t orow = sh.rows[wave][t];
      u32x4 ov;
      if constexpr (SG) {
        const u32x2 e = *reinterpret_cast<const u32x2*>(&tile[toff(t, 64 * q_even + 4 * l16)]);
        const u32x2 o = *reinterpret_cast<const u32x2*>(&tile[toff(t, 64 * (q_even ^ 1) + 4 * l16)]);
        ov = u32x4{__builtin_amdgcn_perm(o[0], e[0], 0x05040100u), __builtin_amdgcn_perm(o[0], e[0], 0x07060302u),
                   __builtin_amdgcn_perm(o[1], e[1], 0x05040100u), __builtin_amdgcn_perm(o[1], e[1], 0x07060302u)};
      } else {
        ov = *reinterpret_cast<const u32x4*>(&tile[toff(t, 8 * l16)]);
      }
      const uint32_t off =
          orow >= 0 ? static_cast<uint32_t>(orow) * (kCT * 2u) + own_off + 16u * l16 : kOutOfRange;
      __builtin_amdgcn_raw_buffer_store_b128(ov, ro, off, 0, 0);
    }
    // The next unit overwrites the tile and the tables: every lane's reads above are done.
    wave_lds_sync();
    out_c = out_n;
    u_cur = u_ent;
  }
}

template <class Ty, int QC, bool SG>
int launch_sg(const ResidentArgs& a, hipStream_t stream) {
  const int32_t n_units = static_cast<int32_t>(static_cast<int64_t>(a.batch) * a.q_s);
  const int64_t want = (static_cast<int64_t>(n_units) + kWaves - 1) / kWaves;  // unit ranges
  if (want <= 0) return OW_OK;
  int64_t grid;
  if constexpr (QC == 4) {
    // Ranges in multiples of 8 (one per XCD), each computed by two workgroups.
    int64_t ranges = static_cast<int64_t>(device_cus()) / 16 * 8;
    if (ranges > (want + 7) / 8 * 8) ranges = (want + 7) / 8 * 8;
    if (ranges < 8) ranges = 8;
    grid = 2 * ranges;
  } else {
    grid = static_cast<int64_t>(device_cus());
    if (grid > want) grid = want;
  }
  if (a.out_tok && a.drop_scale) return fail(OW_ERR_UNSUPPORTED, "an output-row table with a drop-path scale");
  const dim3 g(static_cast<unsigned>(grid)), b(kThreads);
  if (a.out_tok)
    hipLaunchKernelGGL((bigemm_fwd_wave16_kernel<Ty, QC, SG, true, false>), g, b, 0, stream, a, n_units);
  else if (a.drop_scale)
    hipLaunchKernelGGL((bigemm_fwd_wave16_kernel<Ty, QC, SG, false, true>), g, b, 0, stream, a, n_units);
  else
    hipLaunchKernelGGL((bigemm_fwd_wave16_kernel<Ty, QC, SG, false, false>), g, b, 0, stream, a, n_units);
  return hip_status(hipGetLastError(), "bigemm_fwd_wave16_kernel launch");
}

template <class Ty>
int launch_ty(const ResidentArgs& a, bool interleaved, hipStream_t stream) {
  if (a.q_c == 4) return interleaved ? launch_sg<Ty, 4, true>(a, stream) : launch_sg<Ty, 4, false>(a, stream);
  return interleaved ? launch_sg<Ty, 2, true>(a, stream) : launch_sg<Ty, 2, false>(a, stream);
}

}  // namespace

bool wave16_supported(int32_t d, int32_t rd, int32_t channels, int32_t q_c, int64_t x_elems) {
  // Byte offsets are 32-bit and kOutOfRange (2^31) must lie past x and out.
  return d == kD && rd == kRD && (q_c == 2 || q_c == 4) && channels == q_c * kD && x_elems * 2 < (int64_t(1) << 31);
}

int launch_fwd_wave16(const ResidentArgs& a, int32_t radix_level, int32_t dtype, hipStream_t stream) {
  // routing.py:107-121: at radix levels >= 1 group q holds the channels of one residue mod q_c.
  const bool interleaved = radix_level != 0;
  if (dtype == OW_DTYPE_BF16) return launch_ty<BF16>(a, interleaved, stream);
  if (dtype == OW_DTYPE_F16) return launch_ty<F16>(a, interleaved, stream);
  return fail(OW_ERR_UNSUPPORTED, "unsupported dtype %d", dtype);
}

}  // namespace ow
