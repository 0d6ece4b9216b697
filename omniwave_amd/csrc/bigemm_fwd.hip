// Fused BiGEMM forward for gfx950 (CDNA4): RMSNorm row statistics, weight packing, the tile
// kernel and the C-ABI launchers.
//
// Math per tile (omniweave/ops/reference.py:147-171): for the 16 routed tokens of a token
// group and the d routed channels of a channel group,
//     delta = A_o . (SiLU(A_u . T . B_u) * (A_v . T . B_v)) . B_o      scaled per column by gamma
// evaluated with the cheapest association, P = A.T first and Z.B_o before A_o.  With the
// block's RMSNorm fused, T = diag(r) X diag(w) (r = per-token rsqrt scale, w = norm weight),
// so P^T = diag(w) X^T (A diag(r))^T: r scales the token operand of each token group and w is
// folded into the packed B_u / B_v rows, gamma into the packed B_o columns.  SiLU's exponent
// base is folded into the weights too: B_u' = -log2(e) B_u, B_v' = -ln(2) B_v give
// U' = -log2(e) U, V' = -ln(2) V and
//     SiLU(U) V = U V / (1 + e^-U) = U' V' / (1 + 2^U').
//
// Every product is a 32x32x16 MFMA over a pair of token groups (32 tokens), with operand
// orders chosen so that each accumulator is the next product's operand (ow_device.h):
//     P^T  = X^T . (A diag r)^T  block-diagonal token matrix, X^T read from the LDS tile
//     U'^T = B_u'^T . P_u^T      K = channels, weights from LDS
//     Z    = U'V' / (1 + 2^U')   registers
//     W    = Z . B_o             K = expanded dim, weights from LDS
//     delta = A_o . W            block-diagonal token matrix
// Weights are pre-packed (ow_pack_weights) so each MFMA operand is one 16-byte LDS read per
// lane, and each chunk of weights is copied global -> LDS directly (global_load_lds).
#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "ow_device.h"

namespace ow {
namespace {

constexpr int kWaves = 4;     // waves per workgroup
constexpr int kThreads = 256;

// ---------------------------------------------------------------------------------------
// RMSNorm row scales: scale[row] = rsqrt(mean(x[row]^2) + eps) in the reference's dtype
// sequence, one fp32 value per token.  Vector path: VPRW = C/8 16-byte vectors per row,
// LPR = min(64, VPRW) lanes per row, 8 rows per wave.

struct RmsArgs {
  const uint16_t* x;
  float* scale;
  int64_t rows;
  int32_t channels;
  float eps;
};

template <class Ty, int VPRW>
__global__ void __launch_bounds__(kThreads) rms_rows_kernel(RmsArgs a) {
  constexpr int LPR = VPRW < 64 ? VPRW : 64;
  constexpr int RPI = 64 / LPR;   // rows per wave instruction
  constexpr int NR = 8 / RPI;     // rows per lane
  constexpr int VPL = VPRW / LPR; // vectors per lane per row
  static_assert(RPI <= 8, "at least 8 lanes per row");
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int sub = lane % LPR;
  const int64_t base = (static_cast<int64_t>(blockIdx.x) * kWaves + wave) * 8;
  u32x4 v[NR][VPL];
#pragma unroll
  for (int rr = 0; rr < NR; ++rr) {
    const int64_t row = base + rr * RPI + lane / LPR;
#pragma unroll
    for (int q = 0; q < VPL; ++q) {
      v[rr][q] = u32x4{0u, 0u, 0u, 0u};
      if (row < a.rows)
        v[rr][q] = *reinterpret_cast<const u32x4*>(a.x + row * a.channels + (sub + q * LPR) * 8);
    }
  }
#pragma unroll
  for (int rr = 0; rr < NR; ++rr) {
    float acc = 0.0f;
#pragma unroll
    for (int q = 0; q < VPL; ++q)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc = Ty::dot2sq(v[rr][q][e], acc);
#pragma unroll
    for (int m = LPR >> 1; m > 0; m >>= 1) acc += __shfl_xor(acc, m);
    const int64_t row = base + rr * RPI + lane / LPR;
    if (sub == 0 && row < a.rows) a.scale[row] = rms_scale<Ty>(acc / static_cast<float>(a.channels), a.eps);
  }
}

// C = 128 J (J in {1, 2, 4, 8}): 16 lanes per row, lane l16 reads vectors l16 + 16 j of its row,
// 4 rows per wave instruction, NP passes per wave (16 loads in flight per lane), sums over the
// 16 lanes with DPP.
template <class Ty, int J>
__global__ void __launch_bounds__(kThreads) rms_rows16_kernel(RmsArgs a) {
  constexpr int NP = J < 16 ? 16 / J : 1;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t base = (static_cast<int64_t>(blockIdx.x) * kWaves + wave) * (4 * NP);
  u32x4 v[NP][J];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int64_t row = base + 4 * p + (lane >> 4);
#pragma unroll
    for (int j = 0; j < J; ++j) {
      v[p][j] = u32x4{0u, 0u, 0u, 0u};
      if (row < a.rows) v[p][j] = *reinterpret_cast<const u32x4*>(a.x + row * a.channels + ((lane & 15) + 16 * j) * 8);
    }
  }
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc = Ty::dot2sq(v[p][j][e], acc);
    acc = group_sum<16>(acc);
    const int64_t row = base + 4 * p + (lane >> 4);
    if ((lane & 15) == 15 && row < a.rows) a.scale[row] = rms_scale<Ty>(acc / static_cast<float>(a.channels), a.eps);
  }
}

// Any C: one wave per row, element loads.
template <class Ty>
__global__ void __launch_bounds__(kThreads) rms_rows_generic_kernel(RmsArgs a) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kWaves + wave;
  if (row >= a.rows) return;
  float acc = 0.0f;
  for (int c = lane; c < a.channels; c += 64) {
    const float v = Ty::to_f32(a.x[row * a.channels + c]);
    acc = fmaf(v, v, acc);
  }
  for (int m = 32; m > 0; m >>= 1) acc += __shfl_xor(acc, m);
  if (lane == 0) a.scale[row] = rms_scale<Ty>(acc / static_cast<float>(a.channels), a.eps);
}

// ---------------------------------------------------------------------------------------
// Tile kernel.

struct FwdArgs {
  const uint16_t* x;
  uint16_t* out;
  const float* row_scale;  // [batch * n_tok] RMSNorm scale per token (norm == kNormBuffer)
  const uint16_t* packed;
  const int32_t* tok;
  const int32_t* chan;
  const int32_t* out_tok;  // [q_s * 16] output row of each token slot; NULL: the token table
  int32_t batch, n_tok, channels, q_s, q_c;
  int32_t n_chunks;  // ceil(batch * q_s / token groups per workgroup)
  int32_t residual;  // write x + delta instead of delta
  int32_t mode;      // channel-group access, one of the kMode* values
  int32_t stride;    // kModeStrided: channel stride n of a group (= q_c)
  int32_t norm;      // RMSNorm row scales: one of the kNorm* values
  float eps;         // kNormInline / kNormPartials: RMSNorm epsilon
  int32_t parts;     // kNormPartials: partial sums per row in row_scale ([batch * n_tok, parts])
  float* stats_out;  // NULL, or [batch * n_tok, q_c]: sum of squares of each stored row's group columns
  const float* drop_scale;  // NULL, or [batch]: per-image multiplier of the rounded delta (drop-path)
};

// Where the RMSNorm row scales come from.
//   kNormBuffer  row_scale, computed by a statistics pass before the launch
//   kNormInline  the tile load reads whole rows (C / 8 16-byte vectors, 16 lanes per row) and
//                sums the squares itself; the other channel groups' workgroups of the same
//                tokens read the same rows, mostly from L2 (they run on the same XCD)
//   kNormPartials row_scale holds `parts` partial sums of squares per row, written by the
//                previous block's launch (stats_out); the tile load reads only the group's
//                columns
// (kNormNone, kNormBuffer, kNormInline, kNormPartials: ow_device.h)

// Channel-group access modes.
//   kModeContig   group qc is columns [qc*d, qc*d + d): 16-byte row vectors (radix level 0)
//   kModeStrided  group qc is columns res + k*n, k < d, n = q_c in {2, 4, 8}, C = n*d (radix
//                 levels >= 1, omniweave/models/routing.py:107-121): every 16-byte vector of
//                 a row holds 8/n consecutive tile columns of the group
//   kModeElement  anything else (padded groups, unaligned or ragged rows): element access
// (kModeContig, kModeStrided, kModeElement: ow_device.h)
constexpr int kBatch = 16;  // global loads kept in flight per thread by the gather / scatter loops

// Maps the hardware workgroup id to a logical id so that the q_c workgroups of one row chunk
// run on the same XCD (workgroups are dispatched round-robin over the 8 XCDs): their gathers
// and scatters touch the same cache lines of x and out, which then meet in one L2.
__device__ __forceinline__ int xcd_remap(int bid, int nwg) {
  const int xcd = bid & 7, slot = bid >> 3;
  const int per = nwg >> 3, rem = nwg & 7;
  return (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + slot;
}



// One workgroup: 4 waves x TPW token groups (TPW/2 pairs of 16 tokens per wave) x one channel
// group q_c.
template <class Ty, int D, int RD, int TPW, int OCC, bool F8>
__global__ void __attribute__((amdgpu_flat_work_group_size(kThreads, kThreads), amdgpu_waves_per_eu(OCC)))
bigemm_fwd_kernel(FwdArgs a) {
  constexpr int NP = TPW / 2;      // token-group pairs per wave (32-token MFMA N blocks)
  constexpr int R = kWaves * TPW;  // token groups per workgroup
  constexpr int ROWS = R * kG;
  constexpr int LDX = D + 8;       // padded LDS row stride (elements): conflict-free column reads
  constexpr int KS = D / 16;       // 16-deep K steps over the channel tile (= 16-channel blocks)
  constexpr int MB = D / 32;       // 32-channel output blocks of W^T
  constexpr int NCH = RD / 32;     // 32-row chunks of the expanded dimension
  constexpr int FR_U = KS;         // B_u'^T fragments per chunk (B_v'^T the same)
  constexpr int FR_O = 2 * MB;     // B_o^T fragments per chunk (MB blocks x 2 K steps)
  constexpr int FR_CH = 2 * FR_U + FR_O;
  // 1 KB copy units per chunk (fp8: KS Ty B_u'^T, KS / 4 two-unit fp8 B_v'^T and FR_O Ty B_o
  // fragments, padded to whole copy rounds).
  constexpr int CH_UNITS = F8 ? f8_chunk_units(D) : FR_CH;
  constexpr int F8_BV = FR_U;               // fp8: first unit of the B_v'^T K64 fragments
  constexpr int F8_BO = FR_U + 2 * (D / 64);  // fp8: first unit of the B_o fragments
  constexpr int CH_ELEMS = CH_UNITS * kFragElems;
  constexpr int HEAD = F8 ? kF8HeadBytes / 2 : kHeadElems;  // packed head, in 16-bit elements
  static_assert(TPW % 2 == 0, "token groups come in pairs");
  static_assert(CH_ELEMS <= ROWS * LDX, "a weight chunk must fit in the x-tile region");
  // Weight-chunk copies per wave and chunk (every wave issues the same number).
  constexpr int DPW = CH_UNITS / kWaves;
  static_assert(CH_UNITS % kWaves == 0, "chunk copy units split evenly over the waves");
  // Software-pipelined chunk loop (d = 128, one pair per wave): chunk
  // ec + 1's U'/V' MFMAs are issued before chunk ec's gate, so chunks ec and ec + 1 are resident
  // while ec + 2 is copied — three chunk buffers.  (The d = 64 instance runs at 3 waves per SIMD,
  // where the second set of U'/V' accumulators would spill.)
  constexpr bool PIPE = NP == 1 && NCH % 2 == 0 && D == 128;
  constexpr int XS_ELEMS = (PIPE && 2 * CH_ELEMS > ROWS * LDX) ? 2 * CH_ELEMS : ROWS * LDX;

  // LDS regions.  xs: the x tile until the token side has read it; then weight chunks (PIPE:
  // chunks 3k + 1 at xs and 3k + 2 at xs + CH_ELEMS; otherwise the odd chunks); after the
  // chunk loop, each wave's rows of the output tile.  wb: chunks 3k (PIPE) or the even chunks.
  __shared__ __attribute__((aligned(16))) uint16_t xs[XS_ELEMS];
  __shared__ __attribute__((aligned(16))) uint16_t wb[CH_ELEMS];
  __shared__ int32_t rowid[ROWS];   // b * n_tok + token, -1 for pad rows
  __shared__ int32_t rowout[ROWS];  // output row of each tile row, -1 for pad rows
  __shared__ float rsc[ROWS];      // RMSNorm scale of each row (1 without norm)
  __shared__ float dsc[R];         // drop-path scale of each token group's image (1 without)
  __shared__ int32_t chx[D];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;

  const int bid = xcd_remap(blockIdx.x, a.n_chunks * a.q_c);
  const int qc = bid % a.q_c, chunk = bid / a.q_c;

  const uint16_t* wsrc = a.packed + HEAD + static_cast<size_t>(qc) * NCH * CH_ELEMS;
  auto chunk_buf = [&](int ec) -> uint16_t* {
    if constexpr (PIPE) {
      const int k = ec % 3;
      return k == 0 ? wb : xs + (k - 1) * CH_ELEMS;
    } else {
      return (ec & 1) ? xs : wb;
    }
  };
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  auto issue_chunk = [&](int ec) {
    const uint16_t* src = wsrc + static_cast<size_t>(ec) * CH_ELEMS;
    uint16_t* dst = chunk_buf(ec);
#pragma unroll
    for (int i = 0; i < DPW; ++i) {
      const int f = wave_u + i * kWaves;
      copy_frag_to_lds(src + f * kFragElems, dst + f * kFragElems, 16u * lane);
    }
  };
  issue_chunk(0);

  static_assert(ROWS <= kThreads, "one row id per thread");
  if (tid < ROWS) {
    const int64_t tg = static_cast<int64_t>(chunk) * R + tid / kG;
    int32_t id = -1, od = -1;
    if (tg < static_cast<int64_t>(a.batch) * a.q_s) {
      const int32_t b = static_cast<int32_t>(tg / a.q_s);
      const int32_t s = static_cast<int32_t>(tg - static_cast<int64_t>(b) * a.q_s);
      const int32_t t = a.tok[s * kG + (tid % kG)];
      if (t >= 0 && t < a.n_tok) {
        id = b * a.n_tok + t;
        od = id;
        if (a.out_tok) {
          const int32_t to = a.out_tok[s * kG + (tid % kG)];
          od = (to >= 0 && to < a.n_tok) ? b * a.n_tok + to : -1;
        }
      }
    }
    rowid[tid] = id;
    rowout[tid] = od;
    if (tid % kG == 0) {
      float ds = 1.0f;
      if (a.drop_scale && tg < static_cast<int64_t>(a.batch) * a.q_s) ds = a.drop_scale[tg / a.q_s];
      dsc[tid / kG] = ds;
    }
  }
  for (int k = tid; k < D; k += kThreads) {
    const int c = a.chan[qc * D + k];
    chx[k] = (c >= 0 && c < a.channels) ? c : -1;
  }
  __syncthreads();

  // Row scales and the x tile [ROWS x D] into LDS (pad rows / columns read as zero); the
  // row-scale loads are in flight together with the tile loads.
  const int strided_res = __builtin_amdgcn_readfirstlane(chx[0]) & (a.stride - 1);
  float my_rsc = 1.0f;
  if (tid < ROWS && a.norm == kNormBuffer) {
    const int64_t id = rowid[tid];
    if (id >= 0) my_rsc = a.row_scale[id];
  } else if (tid < ROWS && a.norm == kNormPartials) {
    const int64_t id = rowid[tid];
    if (id >= 0) {
      float acc = 0.0f;
      for (int q = 0; q < a.parts; ++q) acc += a.row_scale[id * a.parts + q];
      my_rsc = rms_scale<Ty>(acc / static_cast<float>(a.channels), a.eps);
    }
  }
  // Whole rows, 16 lanes per row: lane l16 reads vectors l16 + 16 j (j < J = C / 128) of its
  // row, sums their squares for the row scale and keeps this group's tile columns: with M = 0
  // the group is contiguous (vector v holds columns 8 (v - qc D / 8) .. + 8 when it belongs
  // to group qc), with M > 0 strided (vector v holds tile columns M v .. M v + M).
  auto gather_rows = [&](auto j_tag, auto m_tag) {
    constexpr int J = decltype(j_tag)::value;
    constexpr int M = decltype(m_tag)::value;
    constexpr int RS = kThreads / 16;         // rows per pass
    constexpr int NI = ROWS / RS;             // passes
    constexpr int IB = J <= 4 ? NI : NI / 2;  // passes whose loads are in flight together
    static_assert(NI % IB == 0, "whole batches");
    const int l16 = tid & 15, rs = tid >> 4;
#pragma unroll 1
    for (int i0 = 0; i0 < NI; i0 += IB) {
      u32x4 v[IB][J];
#pragma unroll
      for (int i = 0; i < IB; ++i) {
        const int64_t id = rowid[rs + RS * (i0 + i)];
#pragma unroll
        for (int j = 0; j < J; ++j) {
          v[i][j] = u32x4{0u, 0u, 0u, 0u};
          if (id >= 0) v[i][j] = *reinterpret_cast<const u32x4*>(a.x + id * a.channels + (l16 + 16 * j) * 8);
        }
      }
#pragma unroll
      for (int i = 0; i < IB; ++i) {
        const int r = rs + RS * (i0 + i);
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < J; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) acc = Ty::dot2sq(v[i][j][e], acc);
        acc = group_sum<16>(acc);
        if (l16 == 0) rsc[r] = rms_scale<Ty>(acc / static_cast<float>(a.channels), a.eps);
#pragma unroll
        for (int j = 0; j < J; ++j) {
          const int vv = l16 + 16 * j;
          if constexpr (M == 0) {
            if (vv / (D / 8) == qc) *reinterpret_cast<u32x4*>(&xs[r * LDX + (vv % (D / 8)) * 8]) = v[i][j];
          } else {
            const StridedPack<M> e = strided_pack<M>(v[i][j], strided_res);
            uint16_t* dst = &xs[r * LDX + vv * M];
            if constexpr (M == 1)
              *dst = static_cast<uint16_t>(e);
            else
              *reinterpret_cast<StridedPack<M>*>(dst) = e;
          }
        }
      }
    }
  };
  auto gather_rows_m = [&](auto m_tag) {
    switch (a.channels / 128) {
      case 1: gather_rows(std::integral_constant<int, 1>{}, m_tag); break;
      case 2: gather_rows(std::integral_constant<int, 2>{}, m_tag); break;
      case 4: gather_rows(std::integral_constant<int, 4>{}, m_tag); break;
      default: gather_rows(std::integral_constant<int, 8>{}, m_tag); break;
    }
  };
  if (a.norm == kNormInline) {
    if (a.mode == kModeContig) gather_rows_m(std::integral_constant<int, 0>{});
    else if (a.stride == 2) gather_rows_m(std::integral_constant<int, 4>{});
    else if (a.stride == 4) gather_rows_m(std::integral_constant<int, 2>{});
    else gather_rows_m(std::integral_constant<int, 1>{});
  } else if (a.mode == kModeContig) {
    constexpr int VPR = D / 8;
    constexpr int NV = ROWS * VPR / kThreads;
    u32x4 v[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int idx = tid + i * kThreads;
      const int64_t id = rowid[idx / VPR];
      v[i] = u32x4{0u, 0u, 0u, 0u};
      if (id >= 0) v[i] = *reinterpret_cast<const u32x4*>(a.x + id * a.channels + qc * D + (idx % VPR) * 8);
    }
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int idx = tid + i * kThreads;
      *reinterpret_cast<u32x4*>(&xs[(idx / VPR) * LDX + (idx % VPR) * 8]) = v[i];
    }
  } else if (a.mode == kModeStrided) {
    // Full-row 16-byte vectors; vector v of a row holds tile columns [M v, M v + M).
    auto gather_strided = [&](auto m_tag) {
      constexpr int M = decltype(m_tag)::value;
      constexpr int VPR = D / M;  // vectors per row: C / 8 = n d / 8
      constexpr int NV = ROWS * VPR / kThreads;
      constexpr int NB = NV < kBatch ? NV : kBatch;
      static_assert(NV % NB == 0, "whole batches");
#pragma unroll 1
      for (int i0 = 0; i0 < NV; i0 += NB) {
        u32x4 v[NB];
#pragma unroll
        for (int j = 0; j < NB; ++j) {
          const int idx = tid + (i0 + j) * kThreads;
          const int64_t id = rowid[idx / VPR];
          v[j] = u32x4{0u, 0u, 0u, 0u};
          if (id >= 0) v[j] = *reinterpret_cast<const u32x4*>(a.x + id * a.channels + (idx % VPR) * 8);
        }
#pragma unroll
        for (int j = 0; j < NB; ++j) {
          const int idx = tid + (i0 + j) * kThreads;
          const StridedPack<M> e = strided_pack<M>(v[j], strided_res);
          uint16_t* dst = &xs[(idx / VPR) * LDX + (idx % VPR) * M];
          if constexpr (M == 1)
            *dst = static_cast<uint16_t>(e);
          else
            *reinterpret_cast<StridedPack<M>*>(dst) = e;
        }
      }
    };
    if (a.stride == 2) gather_strided(std::integral_constant<int, 4>{});
    else if (a.stride == 4) gather_strided(std::integral_constant<int, 2>{});
    else gather_strided(std::integral_constant<int, 1>{});
  } else {
    constexpr int NE = ROWS * D / kThreads;
    static_assert(NE % kBatch == 0, "whole batches");
#pragma unroll 1
    for (int i0 = 0; i0 < NE; i0 += kBatch) {
      uint16_t v[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int i = tid + (i0 + j) * kThreads;
        const int64_t id = rowid[i / D];
        const int c = chx[i % D];
        v[j] = (id >= 0 && c >= 0) ? a.x[id * a.channels + c] : static_cast<uint16_t>(0);
      }
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int i = tid + (i0 + j) * kThreads;
        xs[(i / D) * LDX + i % D] = v[j];
      }
    }
  }
  if (tid < ROWS && a.norm != kNormInline) rsc[tid] = my_rsc;

  // Token-operand rows of this lane: A_u, A_v rows for the K step of its token group, A_o row
  // for the output product.
  const u32x4 fAu = reinterpret_cast<const u32x4*>(a.packed)[lane];
  const u32x4 fAv = reinterpret_cast<const u32x4*>(a.packed + kFragElems)[lane];
  const u32x4 fAo = reinterpret_cast<const u32x4*>(a.packed + 2 * kFragElems)[lane];
  __syncthreads();

  // Token side per pair of groups (32 tokens), block-diagonal 32x32x16 products.
  const int hh = lane >> 5, l32 = lane & 31;
  int col[KS / 2];
#pragma unroll
  for (int cb = 0; cb < KS / 2; ++cb) col[cb] = 32 * cb + l32;
  // P^T operands: Ty K steps; with F8, P_v as fp8 K64 operands (KS / 4 of them).
  constexpr int KV = F8 ? KS / 4 : KS;
  using VOp = std::conditional_t<F8, u32x8, u32x4>;
  u32x4 Pu[NP][KS];
  VOp Pv[NP][KV];
  u32x4 xk[NP][KS / 2][2];  // the lane's x values, kept for the residual
  const float qv = F8 ? reinterpret_cast<const float*>(a.packed + kHeadElems)[kF8QuantPv] : 1.0f;  // fp8 scales
  const float deq8 = F8 ? f8_deq(a.packed) : 1.0f;
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int row0 = (wave * TPW + 2 * p) * kG;
    u32x4 bu = fAu, bv = fAv;
    if (a.norm != kNormNone) {  // lane's slots j are tokens 16 tg + kord(j, hh) of its group tg
      const float* r8 = &rsc[row0 + 16 * ((lane >> 4) & 1) + 4 * hh];
      bu = scale8<Ty>(fAu, r8);
      bv = F8 ? scale8m<Ty>(fAv, r8, qv) : scale8<Ty>(fAv, r8);  // fp8: P_v comes out quantised
    }
    if constexpr (F8)
      pair_token_side_f8<Ty, KS>(xs + row0 * LDX, LDX, col, bu, bv, lane, Pu[p], Pv[p], xk[p]);
    else
      pair_token_side<Ty, KS>(xs + row0 * LDX, LDX, col, bu, bv, lane, Pu[p], Pv[p], xk[p]);
  }

  // Channel side, streamed over 32-row chunks of the expanded dimension (double-buffered).
  f32x16 W[NP][MB];
#pragma unroll
  for (int p = 0; p < NP; ++p)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int i = 0; i < 16; ++i) W[p][mb][i] = 0.0f;

  if constexpr (PIPE && !F8) {
    // One step issues chunk ec + 1's U'/V' products and chunk ec's W += Z B_o, their weight
    // fragments read DEPTH ahead (lds_read_async), and computes one gate value of chunk ec per
    // U'/V' product, so the gate's VALU work runs while the products execute.
    constexpr int DEPTH = 4;
    const uint32_t lane16 = 16u * static_cast<uint32_t>(lane);
    auto stream = [&](auto nu_tag, auto no_tag, uint32_t bn, uint32_t bo, f32x16& Un, f32x16& Vn,
                      const f32x16& Uc, const f32x16& Vc) {
      constexpr int NU = decltype(nu_tag)::value;  // U'/V' fragments of chunk ec + 1 (0 or 2 KS)
      constexpr int NO = decltype(no_tag)::value;  // B_o fragments of chunk ec (0 or FR_O)
      constexpr int NF = NU + NO;
      static_assert(NO == 0 || NU == 0 || NU == 16, "one gate value per U'/V' product");
      auto read = [&](auto ic) -> u32x4 {
        constexpr int i = decltype(ic)::value;
        if constexpr (i < NU)
          return lds_read_async<((i & 1) ? FR_U + i / 2 : i / 2) * kFragElems * 2>(bn);
        else
          return lds_read_async<(i - NU) * kFragElems * 2>(bo);
      };
      u32x4 fr[DEPTH];
      static_for<0, DEPTH>([&](auto ic) {
        if constexpr (decltype(ic)::value < NF) fr[decltype(ic)::value] = read(ic);
      });
      // Gate values k = 8 s + 2 q + h of chunk ec -> Z[s] word q, half h.
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
            Un = Ty::mma32(fr[i % DEPTH], Pu[0][i / 2], Un);
          else
            Vn = Ty::mma32(fr[i % DEPTH], Pv[0][i / 2], Vn);
        } else {
          constexpr int j = i - NU;
          W[0][j / 2] = Ty::mma32(Z[j % 2], fr[i % DEPTH], W[0][j / 2]);
        }
        if constexpr (i + DEPTH < NF) fr[i % DEPTH] = read(std::integral_constant<int, i + DEPTH>{});
        if constexpr (NO > 0 && i < NU) gate(ic);
      });
      if constexpr (NU > 0 && NO > 0 && NCH >= 8) {  // (rd = 128 spills with the hint)
        // Interleave: each U'/V' product followed by about one gate value's VALU work.
        static_for<0, NU>([&](auto) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
          __builtin_amdgcn_sched_group_barrier(0x402, 6, 0);  // VALU, transcendental
        });
      }
    };
    using Nu = std::integral_constant<int, 2 * KS>;
    using No = std::integral_constant<int, FR_O>;
    using Zero = std::integral_constant<int, 0>;
    auto base = [&](int ec) { return lds_addr(chunk_buf(ec)) + lane16; };
    // Step ec: wait for chunk ec + 1 (at ec = 0 chunk 2 may still be in flight: nothing else is
    // outstanding during the loop, so the count is exact); the barrier also means every wave is
    // done with chunk ec - 1, whose buffer then takes chunk ec + 2.
    auto step = [&](int ec, f32x16& Uc, f32x16& Vc, f32x16& Un, f32x16& Vn) {
      const uint32_t bo = base(ec) + 2u * FR_U * kFragElems * 2u;
      if (ec + 1 < NCH) {
        if (ec == 0 && NCH > 2)
          wait_vmcnt<DPW>();
        else
          wait_lds_dma();
        __syncthreads();
        if (ec >= 1 && ec + 2 < NCH) issue_chunk(ec + 2);
        stream(Nu{}, No{}, base(ec + 1), bo, Un, Vn, Uc, Vc);
      } else {
        stream(Zero{}, No{}, 0u, bo, Un, Vn, Uc, Vc);
      }
    };
    wait_lds_dma();
    __syncthreads();
    if (NCH > 1) issue_chunk(1);
    if (NCH > 2) issue_chunk(2);
    f32x16 Ua, Va, Ub, Vb;
    stream(Nu{}, Zero{}, base(0), 0u, Ua, Va, Ub, Vb);
#pragma unroll
    for (int ec = 0; ec < NCH; ec += 2) {
      step(ec, Ua, Va, Ub, Vb);
      step(ec + 1, Ub, Vb, Ua, Va);
    }
  } else if constexpr (PIPE) {
    // U'/V' of chunk ec (fp8: e4m3 fragments and P operands, dequantised in the gate).
    auto uv = [&](int ec, f32x16& U, f32x16& V) {
      U = f32x16{};
      V = f32x16{};
      if constexpr (F8) {
        const u32x4* cf = reinterpret_cast<const u32x4*>(chunk_buf(ec));
        const u32x8* c8 = reinterpret_cast<const u32x8*>(chunk_buf(ec) + F8_BV * kFragElems);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) U = Ty::mma32(cf[ks * (kFragElems / 8) + lane], Pu[0][ks], U);
#pragma unroll
        for (int s = 0; s < KV; ++s) V = mma32x64_f8(c8[s * (kF8K64Bytes / 32) + lane], Pv[0][s], V);
      } else {
        const u32x4* cf = reinterpret_cast<const u32x4*>(chunk_buf(ec));
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          U = Ty::mma32(cf[ks * (kFragElems / 8) + lane], Pu[0][ks], U);
          V = Ty::mma32(cf[(FR_U + ks) * (kFragElems / 8) + lane], Pv[0][ks], V);
        }
      }
    };
    // Gate and W += Z B_o of chunk ec (fp8: the packed B_o carries V''s dequantisation).
    auto gate_w = [&](int ec, const f32x16& U, const f32x16& V) {
      const uint16_t* cw = chunk_buf(ec);
      const u32x4* co = reinterpret_cast<const u32x4*>(F8 ? cw + F8_BO * kFragElems : cw + 2 * FR_U * kFragElems);
      u32x4 Z[2];
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float u0 = U[8 * s + 2 * q], u1 = U[8 * s + 2 * q + 1];
          const float v0 = V[8 * s + 2 * q], v1 = V[8 * s + 2 * q + 1];
          Z[s][q] = Ty::pack2(f8_gate<Ty>(u0, v0, deq8), f8_gate<Ty>(u1, v1, deq8));
        }
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int s = 0; s < 2; ++s) W[0][mb] = Ty::mma32(Z[s], co[(2 * mb + s) * (kFragElems / 8) + lane], W[0][mb]);
    };
    // Step ec: wait for chunk ec + 1 (at ec = 0 chunk 2 may still be in flight: nothing else is
    // outstanding during the loop, so the count is exact); the barrier also means every wave is
    // done with chunk ec - 1, whose buffer then takes chunk ec + 2; chunk ec + 1's U'/V'
    // products are issued, then chunk ec's gate and Z B_o run while they execute.
    auto step = [&](int ec, f32x16& Uc, f32x16& Vc, f32x16& Un, f32x16& Vn) {
      if (ec + 1 < NCH) {
        if (ec == 0 && NCH > 2)
          wait_vmcnt<DPW>();
        else
          wait_lds_dma();
        __syncthreads();
        if (ec >= 1 && ec + 2 < NCH) issue_chunk(ec + 2);
        uv(ec + 1, Un, Vn);
      }
      gate_w(ec, Uc, Vc);
    };
    wait_lds_dma();
    __syncthreads();
    if (NCH > 1) issue_chunk(1);
    if (NCH > 2) issue_chunk(2);
    f32x16 Ua, Va, Ub, Vb;
    uv(0, Ua, Va);
#pragma unroll
    for (int ec = 0; ec < NCH; ec += 2) {
      step(ec, Ua, Va, Ub, Vb);
      step(ec + 1, Ub, Vb, Ua, Va);
    }
  } else
  for (int ec = 0; ec < NCH; ++ec) {
    wait_lds_dma();
    // Chunk ec has landed; every wave is done with chunk ec - 1 (and, at ec = 0, with the x
    // tile), so the buffer of chunk ec + 1 is free.
    __syncthreads();
    if (ec + 1 < NCH) issue_chunk(ec + 1);
    const uint16_t* cw = chunk_buf(ec);
    const u32x4* cf = reinterpret_cast<const u32x4*>(cw);
    if constexpr (F8) {
      const u32x8* c8 = reinterpret_cast<const u32x8*>(cw + F8_BV * kFragElems);
      const u32x4* co = reinterpret_cast<const u32x4*>(cw + F8_BO * kFragElems);
      auto fu = [&](int ks) { return cf[ks * (kFragElems / 8) + lane]; };
      auto fv = [&](int s) { return c8[s * (kF8K64Bytes / 32) + lane]; };
      auto fo = [&](int mb, int s) { return co[(2 * mb + s) * (kFragElems / 8) + lane]; };
#pragma unroll
      for (int p = 0; p < NP; ++p) pair_chunk_f8<Ty, KS, MB>(Pu[p], Pv[p], fu, fv, fo, W[p], deq8);
    } else {
      auto fu = [&](int ks) { return cf[ks * (kFragElems / 8) + lane]; };
      auto fv = [&](int ks) { return cf[(FR_U + ks) * (kFragElems / 8) + lane]; };
      auto fo = [&](int mb, int s) { return cf[(2 * FR_U + 2 * mb + s) * (kFragElems / 8) + lane]; };
#pragma unroll
      for (int p = 0; p < NP; ++p) pair_chunk<Ty, KS, MB>(Pu[p], Pv[p], fu, fv, fo, W[p]);
    }
  }

  // Output side: delta = A_o W per pair (lane = channel 32 mb + l32, registers = tokens;
  // LayerScale folded into B_o); the rounded delta, or round(x + delta) with x from the
  // token-side operands, is written over the pair's own 32 rows of xs.  The barrier first: the odd weight chunks live in
  // xs.  No branch separates an MFMA from the reads of its result.
  mfma_drain();
  __syncthreads();
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    f32x16 dl[MB];
    pair_output<Ty, MB>(W[p], fAo, lane, dl);
    mfma_drain();
    uint16_t* st = xs + (wave * TPW + 2 * p) * kG * LDX;
    const float s0 = dsc[wave * TPW + 2 * p], s1 = dsc[wave * TPW + 2 * p + 1];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      auto dst = [&](int i) { return &st[pair_token_row(i, hh) * LDX + 32 * mb + l32]; };
      // The residual is added in the store loop below, from x in memory: keeping the lane's
      // x values in registers through the chunk loop would cost 32 VGPRs there.
      if (a.drop_scale)
        pair_store_block<Ty, false, true>(dl[mb], xk[p][mb], dst, s0, s1);
      else
        pair_store_block<Ty, false>(dl[mb], xk[p][mb], dst);
    }
  }
  __syncthreads();

  // The finished tile to memory.  Each wave stores rows [32 wave, 32 wave + 32) of the tile;
  // the output-row ids and the tile data of a batch of rows are read from LDS first (and, with
  // the residual, the same elements of x from memory), then the stores are issued without
  // waiting in between (an LDS round trip per store would leave the loop latency-bound).  The
  // residual is round(x + tile value), the tile holding the rounded (drop-path scaled) delta.
  if (a.mode == kModeContig || a.mode == kModeStrided) {
    constexpr int WR = ROWS / kWaves;  // rows per wave
    static_assert(WR == 32, "32 rows per wave");
    // M tile columns per 16-byte row vector of out: 8 (contiguous) or 8 / stride.
    auto store_rows = [&](auto m_tag) {
      constexpr int M = decltype(m_tag)::value;
      constexpr int N = 8 / M;                   // element stride of the group in a vector
      constexpr int VPR = D / M;                 // row vectors holding the group's columns
      constexpr int LPR = VPR < 64 ? VPR : 64;   // lanes per row
      constexpr int RPI = 64 / LPR;              // rows per pass
      constexpr int NIT = WR / RPI;              // passes (rows per lane)
      constexpr int VPL = VPR / LPR;             // vectors per lane and row
      constexpr int KB = NIT < 8 ? NIT : 8;      // passes per batch
      static_assert(NIT % KB == 0, "whole batches");
      using Elt = std::conditional_t<M == 8, u32x4, std::conditional_t<M == 4, u32x2,
                                     std::conditional_t<M == 2, uint32_t, uint16_t>>>;
      const int sub = lane % LPR, rsub = lane / LPR;
      const int64_t col0 = M == 8 ? static_cast<int64_t>(qc) * D : strided_res;
#pragma unroll 1
      for (int k0 = 0; k0 < NIT; k0 += KB) {
        int32_t ids[KB];
        Elt val[KB][VPL];
        u32x4 xv[KB][VPL];
#pragma unroll
        for (int k = 0; k < KB; ++k) {
          const int r = wave * WR + rsub + RPI * (k0 + k);
          ids[k] = rowout[r];
          const int32_t in = rowid[r];  // >= 0 wherever the output row is
#pragma unroll
          for (int q = 0; q < VPL; ++q) {
            val[k][q] = *reinterpret_cast<const Elt*>(&xs[r * LDX + (sub + q * LPR) * M]);
            xv[k][q] = u32x4{0u, 0u, 0u, 0u};
            if (a.residual && in >= 0)
              xv[k][q] = *reinterpret_cast<const u32x4*>(a.x + static_cast<int64_t>(in) * a.channels +
                                                          (M == 8 ? col0 : 0) + (sub + q * LPR) * 8);
          }
        }
        if (a.residual) {
#pragma unroll
          for (int k = 0; k < KB; ++k)
#pragma unroll
            for (int q = 0; q < VPL; ++q) {
              if constexpr (M == 8) {
#pragma unroll
                for (int e = 0; e < 4; ++e) val[k][q][e] = add_residual2<Ty>(xv[k][q][e], val[k][q][e]);
              } else {
                const StridedPack<M> xe = strided_pack<M>(xv[k][q], strided_res);
                if constexpr (M == 4) {
                  val[k][q].x = add_residual2<Ty>(xe.x, val[k][q].x);
                  val[k][q].y = add_residual2<Ty>(xe.y, val[k][q].y);
                } else if constexpr (M == 2) {
                  val[k][q] = add_residual2<Ty>(xe, val[k][q]);
                } else {
                  val[k][q] = lo16(add_residual2<Ty>(xe, val[k][q]));
                }
              }
            }
        }
        if constexpr (M == 8) {
          // Sum of squares of the stored values of each row's group columns: the next block's
          // RMSNorm statistics (kNormPartials).  Contiguous groups only: 16 lanes per row.
          if (a.stats_out) {
#pragma unroll
            for (int k = 0; k < KB; ++k) {
              float acc = 0.0f;
#pragma unroll
              for (int e = 0; e < 4; ++e) acc = Ty::dot2sq(val[k][0][e], acc);
              acc = group_sum<LPR>(acc);
              if (sub == 0 && ids[k] >= 0) a.stats_out[static_cast<int64_t>(ids[k]) * a.q_c + qc] = acc;
            }
          }
        }
#pragma unroll
        for (int k = 0; k < KB; ++k) {
          if (ids[k] < 0) continue;
          uint16_t* row = a.out + static_cast<int64_t>(ids[k]) * a.channels + col0;
#pragma unroll
          for (int q = 0; q < VPL; ++q) {
            uint16_t* dst = row + (sub + q * LPR) * 8;
            const Elt e = val[k][q];
            if constexpr (M == 8) {
              *reinterpret_cast<u32x4*>(dst) = e;
            } else if constexpr (M == 4) {
              dst[0] = lo16(e.x);
              dst[N] = hi16(e.x);
              dst[2 * N] = lo16(e.y);
              dst[3 * N] = hi16(e.y);
            } else if constexpr (M == 2) {
              dst[0] = lo16(e);
              dst[N] = hi16(e);
            } else {
              dst[0] = e;
            }
          }
        }
      }
    };
    if (a.mode == kModeContig) store_rows(std::integral_constant<int, 8>{});
    else if (a.stride == 2) store_rows(std::integral_constant<int, 4>{});
    else if (a.stride == 4) store_rows(std::integral_constant<int, 2>{});
    else store_rows(std::integral_constant<int, 1>{});
  } else {
    constexpr int NE = ROWS * D / kThreads;
#pragma unroll 4
    for (int j = 0; j < NE; ++j) {
      const int i = tid + j * kThreads;
      const int r = i / D, k = i % D;
      const int64_t id = rowout[r];
      const int c = chx[k];
      if (id >= 0 && c >= 0) {
        uint16_t v = xs[r * LDX + k];
        if (a.residual) v = lo16(add_residual2<Ty>(a.x[static_cast<int64_t>(rowid[r]) * a.channels + c], v));
        a.out[id * a.channels + c] = v;
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
// Weight packing.

struct PackArgs {
  const void* a_u;
  const void* a_v;
  const void* a_o;
  const void* b_u;
  const void* b_v;
  const void* b_o;
  const float* norm_w;  // folded into B_u / B_v rows (NULL: weight 1)
  const float* gamma;   // folded into B_o columns (NULL: scale 1)
  const int32_t* chan;  // channel table [q_c * d] (routes norm_w / gamma; pads packed as 0)
  void* packed;
  int32_t wdtype, q_c, d, rd, channels;
  int64_t total;
};

__device__ __forceinline__ float load_f32(const void* p, int64_t i, int dtype) {
  if (dtype == OW_DTYPE_F32) return static_cast<const float*>(p)[i];
  const uint16_t u = static_cast<const uint16_t*>(p)[i];
  return dtype == OW_DTYPE_BF16 ? BF16::to_f32(u) : F16::to_f32(u);
}

// Packed order: three token-operand rows (64 lanes x 8), then per (q, chunk ec): KS B_u'^T
// fragments, KS B_v'^T fragments, 2*MB B_o fragments (32x32x16 operands, 64 lanes x 8).
//   A_u / A_v / A_o rows:       lane l slot j -> A[l32 % 16][8(j/4) + 4hh + j%4]
//   B_u'^T / B_v'^T, K step ks: lane l slot j -> row e = 32ec + l32, channel
//                               16ks + 8(j/4) + 4hh + j%4 (accumulator rows of P^T)
//   B_o (mb, s):                lane l slot j -> channel c = 32mb + l32, expanded index
//                               32ec + 16s + 8(j/4) + 4hh + j%4 (accumulator rows of U'^T)
template <class Ty>
__global__ void __launch_bounds__(256) pack_kernel(PackArgs p) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= p.total) return;
  float val;
  if (idx < kHeadElems) {
    const int frag = static_cast<int>(idx / kFragElems);
    const int e = static_cast<int>(idx % kFragElems);
    const int lane = e / 8, j = e % 8;
    const int t = lane & 15, hh = lane >> 5;
    const int k = 8 * (j / 4) + 4 * hh + (j % 4);
    val = load_f32(frag == 0 ? p.a_u : frag == 1 ? p.a_v : p.a_o, t * kG + k, p.wdtype);
  } else {
    const int ks_n = p.d / 16, mb_n = p.d / 32, nch = p.rd / 32;
    const int64_t ch_elems = static_cast<int64_t>(2 * ks_n + 2 * mb_n) * kFragElems;
    int64_t rem = idx - kHeadElems;
    const int q = static_cast<int>(rem / (nch * ch_elems));
    rem -= static_cast<int64_t>(q) * nch * ch_elems;
    const int ec = static_cast<int>(rem / ch_elems);
    rem -= static_cast<int64_t>(ec) * ch_elems;
    const int fr = static_cast<int>(rem / kFragElems);
    const int e = static_cast<int>(rem % kFragElems);
    const int lane = e / 8, j = e % 8;
    const int l32 = lane & 31, hh = lane >> 5;
    if (fr < 2 * ks_n) {
      const bool is_u = fr < ks_n;
      const int ks = fr % ks_n;
      const int col = 32 * ec + l32;
      const int c = 16 * ks + 8 * (j / 4) + 4 * hh + (j % 4);
      const int64_t src = (static_cast<int64_t>(q) * p.d + c) * p.rd + col;
      float w = 1.0f;
      if (p.chan) {
        const int gc = p.chan[q * p.d + c];
        w = (gc >= 0 && gc < p.channels) ? (p.norm_w ? p.norm_w[gc] : 1.0f) : 0.0f;
      }
      val = load_f32(is_u ? p.b_u : p.b_v, src, p.wdtype) * w * (is_u ? kNegLog2e : kNegLn2);
    } else {
      const int f = fr - 2 * ks_n;
      const int mb = f / 2, s = f % 2;
      const int c = 32 * mb + l32;
      const int ee = 32 * ec + 16 * s + 8 * (j / 4) + 4 * hh + (j % 4);
      const int64_t src = (static_cast<int64_t>(q) * p.rd + ee) * p.d + c;
      float w = 1.0f;
      if (p.chan) {
        const int gc = p.chan[q * p.d + c];
        w = (gc >= 0 && gc < p.channels) ? (p.gamma ? p.gamma[gc] : 1.0f) : 0.0f;
      }
      val = load_f32(p.b_o, src, p.wdtype) * w;
    }
  }
  static_cast<uint16_t*>(p.packed)[idx] = Ty::from_f32(val);
}

// Second section for d = 64, rd = 128 (the 16-token kernel, bigemm_fwd_wave16.hip), after
// the 32x32x16 fragments: per (q, chunk ec) 12 operands of v_mfma_f32_16x16x32 (64 lanes x 8),
// K order kord16(j, h) = 16 (j / 4) + 4 h + j % 4 for lane l = 16 h + l16, slot j:
//   BU'' (eb, s), BV'' (eb, s) for eb, s in {0, 1} (A operands): row e = 32 ec + 16 eb + l16,
//                               channel 32 s + kord16(j, h)
//   BO (cb), cb < 4 (B operand): channel 16 cb + l16, expanded index 32 ec + kord16(j, h)
// (the rows of the kernel's 16x16 accumulators, so each accumulator pair is the next operand).
template <class Ty>
__global__ void __launch_bounds__(256) pack16_kernel(PackArgs p, int64_t base, int64_t n) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= n) return;
  constexpr int kD16 = 64, kRD16 = 128, kFrames = 12;
  const int per_q = (kRD16 / 32) * kFrames * kFragElems;
  const int q = static_cast<int>(idx / per_q);
  int rem = static_cast<int>(idx - static_cast<int64_t>(q) * per_q);
  const int ec = rem / (kFrames * kFragElems);
  rem -= ec * kFrames * kFragElems;
  const int fr = rem / kFragElems, e = rem % kFragElems;
  const int lane = e / 8, j = e % 8;
  const int l16 = lane & 15, h = lane >> 4;
  const int k = 16 * (j / 4) + 4 * h + (j % 4);
  float val;
  if (fr < 8) {
    const bool is_u = fr < 4;
    const int eb = (fr & 3) >> 1, sk = fr & 1;
    const int col = 32 * ec + 16 * eb + l16;  // expanded row
    const int c = 32 * sk + k;                // channel of the group
    const int64_t src = (static_cast<int64_t>(q) * kD16 + c) * kRD16 + col;
    float w = 1.0f;
    if (p.chan) {
      const int gc = p.chan[q * kD16 + c];
      w = (gc >= 0 && gc < p.channels) ? (p.norm_w ? p.norm_w[gc] : 1.0f) : 0.0f;
    }
    val = load_f32(is_u ? p.b_u : p.b_v, src, p.wdtype) * w * (is_u ? kNegLog2e : kNegLn2);
  } else {
    const int cb = fr - 8;
    const int c = 16 * cb + l16;
    const int ee = 32 * ec + k;
    const int64_t src = (static_cast<int64_t>(q) * kRD16 + ee) * kD16 + c;
    float w = 1.0f;
    if (p.chan) {
      const int gc = p.chan[q * kD16 + c];
      w = (gc >= 0 && gc < p.channels) ? (p.gamma ? p.gamma[gc] : 1.0f) : 0.0f;
    }
    val = load_f32(p.b_o, src, p.wdtype) * w;
  }
  static_cast<uint16_t*>(p.packed)[base + idx] = Ty::from_f32(val);
}

// fp8 channel side: per-tensor scales, in three launches (f8_zero, f8_amax, f8_finalize).
// f8_amax: absmax of the folded B_v'' over all channel groups, 8 values per thread, wave
// maxima combined with atomic max on the (non-negative) float bits.
__global__ void __launch_bounds__(64) f8_zero_kernel(float* scales) {
  if (threadIdx.x < kF8ScaleFloats) scales[threadIdx.x] = 0.0f;
}

__global__ void __launch_bounds__(256) f8_amax_kernel(PackArgs p, float* scales) {
  const int n = p.q_c * p.d * p.rd;
  const int i0 = (blockIdx.x * 256 + threadIdx.x) * 8;
  float mv = 0.0f;
  for (int i = i0; i < i0 + 8 && i < n; ++i) {
    const int qc = i / p.rd;  // q * d + c
    float w = 1.0f;
    if (p.chan) {
      const int gc = p.chan[qc];
      w = (gc >= 0 && gc < p.channels) ? (p.norm_w ? p.norm_w[gc] : 1.0f) : 0.0f;
    }
    mv = fmaxf(mv, fabsf(load_f32(p.b_v, i, p.wdtype) * w * kNegLn2));
  }
  for (int m = 32; m > 0; m >>= 1) mv = fmaxf(mv, __shfl_xor(mv, m));
  if ((threadIdx.x & 63) == 0) atomicMax(reinterpret_cast<unsigned int*>(scales + kF8AmaxBv), __float_as_uint(mv));
}

// P_v is quantised with the static bound |P_v| <= ||A_v||_inf sqrt(C) (1.02): the RMSNorm'd
// rows satisfy |x_c r| <= sqrt(C), the 2% cover the Ty rounding of r and of the token operand.
// One wave: lane i < 16 sums |row i| of the Ty-rounded A_v.  V' = V'_q s_b / q_v.
template <class Ty>
__global__ void __launch_bounds__(64) f8_finalize_kernel(PackArgs p, float* scales) {
  const int lane = threadIdx.x;
  float sv = 0.0f;
  if (lane < kG)
    for (int j = 0; j < kG; ++j) sv += fabsf(Ty::to_f32(Ty::from_f32(load_f32(p.a_v, lane * kG + j, p.wdtype))));
  for (int m = 32; m > 0; m >>= 1) sv = fmaxf(sv, __shfl_xor(sv, m));
  if (lane == 0) {
    const float av = scales[kF8AmaxBv];
    const float root_c = sqrtf(static_cast<float>(p.channels)) * 1.02f;
    const float qv = sv > 0.0f ? kF8Max / (sv * root_c) : 1.0f;
    const float sbv = av > 0.0f ? av / kF8Max : 1.0f;
    scales[kF8DeqV] = sbv / qv;
    scales[kF8QuantPv] = qv;
  }
}

// fp8 packing, one thread per 16-bit unit of the packed buffer: the Ty head, then per (q, ec)
// the Ty B_u'^T fragments (pack_kernel's order), the e4m3fn B_v'^T K64 fragments (value / s_b,
// s_b = absmax / 448; lane (e, hh) byte j = B_v''[64 s + 32 (j / 16) + 8 ((j % 16) / 4) + 4 hh
// + j % 4][32 ec + e], two bytes per thread) and the Ty B_o fragments times V''s
// dequantisation factor, then the chunk's padding (zero).
template <class Ty>
__global__ void __launch_bounds__(256) pack_f8_kernel(PackArgs p, const float* scales) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= p.total) return;
  uint8_t* base = static_cast<uint8_t*>(p.packed);
  if (idx < kHeadElems) {
    const int frag = static_cast<int>(idx / kFragElems);
    const int e = static_cast<int>(idx % kFragElems);
    const int lane = e / 8, j = e % 8;
    const int t = lane & 15, hh = lane >> 5;
    const int k = 8 * (j / 4) + 4 * hh + (j % 4);
    const float val = load_f32(frag == 0 ? p.a_u : frag == 1 ? p.a_v : p.a_o, t * kG + k, p.wdtype);
    reinterpret_cast<uint16_t*>(base)[idx] = Ty::from_f32(val);
    return;
  }
  const int ks_n = p.d / 16, nk64 = p.d / 64, nch = p.rd / 32;
  const int64_t ch_units16 = static_cast<int64_t>(f8_chunk_units(p.d)) * kFragElems;  // 16-bit units per chunk
  int64_t rem = idx - kHeadElems;
  const int q = static_cast<int>(rem / (nch * ch_units16));
  rem -= static_cast<int64_t>(q) * nch * ch_units16;
  const int ec = static_cast<int>(rem / ch_units16);
  rem -= static_cast<int64_t>(ec) * ch_units16;
  uint16_t* chunk = reinterpret_cast<uint16_t*>(base + kF8HeadBytes) + (static_cast<int64_t>(q) * nch + ec) * ch_units16;
  const int fr = static_cast<int>(rem / kFragElems);  // 1 KB unit of the chunk
  const int e = static_cast<int>(rem % kFragElems);
  auto norm_w = [&](int c) {
    if (!p.chan) return 1.0f;
    const int gc = p.chan[q * p.d + c];
    return (gc >= 0 && gc < p.channels) ? (p.norm_w ? p.norm_w[gc] : 1.0f) : 0.0f;
  };
  float out = 0.0f;
  if (fr < ks_n) {  // Ty B_u'^T
    const int lane = e / 8, j = e % 8;
    const int l32 = lane & 31, hh = lane >> 5;
    const int c = 16 * fr + 8 * (j / 4) + 4 * hh + (j % 4);
    const int64_t src = (static_cast<int64_t>(q) * p.d + c) * p.rd + 32 * ec + l32;
    out = load_f32(p.b_u, src, p.wdtype) * norm_w(c) * kNegLog2e;
  } else if (fr < ks_n + 2 * nk64) {  // fp8 B_v'^T: bytes 2 e, 2 e + 1 of the K64 fragments
    const int64_t byte = static_cast<int64_t>(fr - ks_n) * 2 * kFragElems + 2 * e;
    const int s = static_cast<int>(byte / kF8K64Bytes);
    const int in = static_cast<int>(byte % kF8K64Bytes);
    const int lane = in / 32, j = in % 32;  // j even
    const int l32 = lane & 31, hh = lane >> 5;
    const float amax = scales[kF8AmaxBv];
    const float mul = amax > 0.0f ? kF8Max / amax : 1.0f;
    float v2[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int jj = j + t;
      const int c = 64 * s + 32 * (jj / 16) + 8 * ((jj % 16) / 4) + 4 * hh + (jj % 4);
      const int64_t src = (static_cast<int64_t>(q) * p.d + c) * p.rd + 32 * ec + l32;
      v2[t] = load_f32(p.b_v, src, p.wdtype) * norm_w(c) * kNegLn2 * mul;
    }
    chunk[static_cast<int64_t>(fr) * kFragElems + e] = static_cast<uint16_t>(cvt_fp8x2<false>(v2[0], v2[1], 0u));
    return;
  } else if (fr < ks_n + 2 * nk64 + 2 * (p.d / 32)) {  // Ty B_o x dequantisation of V'
    const int f = fr - ks_n - 2 * nk64;
    const int lane = e / 8, j = e % 8;
    const int l32 = lane & 31, hh = lane >> 5;
    const int mb = f / 2, s = f % 2;
    const int c = 32 * mb + l32;
    const int ee = 32 * ec + 16 * s + 8 * (j / 4) + 4 * hh + (j % 4);
    const int64_t src = (static_cast<int64_t>(q) * p.rd + ee) * p.d + c;
    float w = 1.0f;
    if (p.chan) {
      const int gc = p.chan[q * p.d + c];
      w = (gc >= 0 && gc < p.channels) ? (p.gamma ? p.gamma[gc] : 1.0f) : 0.0f;
    }
    // V''s dequantisation folded into B_o with bf16 activations; f16 applies it in the gate
    // (f8_gate: Z in the quantised scale would overflow f16).
    out = load_f32(p.b_o, src, p.wdtype) * w * (std::is_same_v<Ty, F16> ? 1.0f : scales[kF8DeqV]);
  }
  chunk[static_cast<int64_t>(fr) * kFragElems + e] = Ty::from_f32(out);
}

int64_t packed_elems(int32_t q_c, int32_t d, int32_t rd) {
  const int64_t per_chunk = static_cast<int64_t>(2 * (d / 16) + 2 * (d / 32)) * kFragElems;
  return kHeadElems + static_cast<int64_t>(q_c) * (rd / 32) * per_chunk;
}

int64_t packed16_elems(int32_t q_c, int32_t d, int32_t rd) {
  return d == 64 && rd == 128 ? static_cast<int64_t>(q_c) * 3 * d * rd : 0;
}

template <class Ty>
int launch_rms(const RmsArgs& a, hipStream_t s) {
  const int vprw = a.channels % 8 == 0 ? a.channels / 8 : 0;
  const unsigned blocks8 = static_cast<unsigned>((a.rows + kWaves * 8 - 1) / (kWaves * 8));
  auto rows16 = [&](auto j_tag) {
    constexpr int J = decltype(j_tag)::value;
    constexpr int RW = 4 * (J < 16 ? 16 / J : 1);  // rows per wave
    const unsigned blocks = static_cast<unsigned>((a.rows + kWaves * RW - 1) / (kWaves * RW));
    hipLaunchKernelGGL((rms_rows16_kernel<Ty, J>), dim3(blocks), dim3(kThreads), 0, s, a);
    return hip_status(hipGetLastError(), "rms_rows16_kernel launch");
  };
  switch (vprw) {
    case 16: return rows16(std::integral_constant<int, 1>{});
    case 32: return rows16(std::integral_constant<int, 2>{});
    case 64: return rows16(std::integral_constant<int, 4>{});
    case 128: return rows16(std::integral_constant<int, 8>{});
    default: break;
  }
  switch (vprw) {
    case 8: hipLaunchKernelGGL((rms_rows_kernel<Ty, 8>), dim3(blocks8), dim3(kThreads), 0, s, a); break;
    case 16: hipLaunchKernelGGL((rms_rows_kernel<Ty, 16>), dim3(blocks8), dim3(kThreads), 0, s, a); break;
    case 32: hipLaunchKernelGGL((rms_rows_kernel<Ty, 32>), dim3(blocks8), dim3(kThreads), 0, s, a); break;
    case 64: hipLaunchKernelGGL((rms_rows_kernel<Ty, 64>), dim3(blocks8), dim3(kThreads), 0, s, a); break;
    case 128: hipLaunchKernelGGL((rms_rows_kernel<Ty, 128>), dim3(blocks8), dim3(kThreads), 0, s, a); break;
    case 256: hipLaunchKernelGGL((rms_rows_kernel<Ty, 256>), dim3(blocks8), dim3(kThreads), 0, s, a); break;
    default: {
      const unsigned blocks = static_cast<unsigned>((a.rows + kWaves - 1) / kWaves);
      hipLaunchKernelGGL(rms_rows_generic_kernel<Ty>, dim3(blocks), dim3(kThreads), 0, s, a);
    }
  }
  return hip_status(hipGetLastError(), "rms_rows_kernel launch");
}

// Token groups per wave (TPW) and workgroups per CU (OCC) for the two channel tiles.
#ifndef OW_TPW_D128
#define OW_TPW_D128 2
#endif
#ifndef OW_OCC_D128
#define OW_OCC_D128 2
#endif
#ifndef OW_TPW_D64
#define OW_TPW_D64 2
#endif
#ifndef OW_OCC_D64
#define OW_OCC_D64 3
#endif

// d = 128: 4 token groups per wave (two 32-token MFMA blocks share each weight fragment read
// from LDS), one workgroup per CU.  d = 64: the same tiling fits two workgroups per CU.
template <class Ty, int D, int RD, bool F8>
int launch_fwd(const FwdArgs& a, hipStream_t stream) {
  constexpr int TPW = D == 64 ? OW_TPW_D64 : OW_TPW_D128;
  constexpr int OCC = D == 64 ? OW_OCC_D64 : OW_OCC_D128;
  constexpr int R = kWaves * TPW;
  FwdArgs args = a;
  const int64_t groups = static_cast<int64_t>(a.batch) * a.q_s;
  const int64_t chunks = (groups + R - 1) / R;
  const int64_t nwg = chunks * a.q_c;
  if (nwg == 0) return OW_OK;
  if (nwg > 0x7fffffff) return fail(OW_ERR_UNSUPPORTED, "grid too large (%lld workgroups)", (long long)nwg);
  args.n_chunks = static_cast<int32_t>(chunks);
  hipLaunchKernelGGL((bigemm_fwd_kernel<Ty, D, RD, TPW, OCC, F8>), dim3(static_cast<unsigned>(nwg)), dim3(kThreads),
                     0, stream, args);
  return hip_status(hipGetLastError(), "bigemm_fwd_kernel launch");
}

template <class Ty, bool F8>
int dispatch_fwd(const FwdArgs& a, int d, int rd, hipStream_t s) {
  if (d == 64 && rd == 128) return launch_fwd<Ty, 64, 128, F8>(a, s);
  if (d == 64 && rd == 256) return launch_fwd<Ty, 64, 256, F8>(a, s);
  if (d == 128 && rd == 128) return launch_fwd<Ty, 128, 128, F8>(a, s);
  if (d == 128 && rd == 256) return launch_fwd<Ty, 128, 256, F8>(a, s);
  return fail(OW_ERR_UNSUPPORTED, "unsupported channel tile d=%d / expanded dim rd=%d; expected d in {64,128}, rd in {128,256}", d, rd);
}

}  // namespace
}  // namespace ow

namespace ow {

// Kernel and channel-group access of a bf16 / f16 launch (routing.py:107-121: identity channel
// order at level 0 or with one group; at levels >= 1 group qc is the channels congruent to
// (qc + level) mod q_c).
FwdPath fwd_path(const void* x, const void* out, const OwPlan* plan, int32_t q_c, int32_t dtype, int32_t flags) {
  const int32_t c = plan->channels, d = plan->channel_tile;
  FwdPath p{};
  p.resident = dtype != OW_DTYPE_F32 && !(flags & OW_FUSE_FP8) && resident_supported(d, 2 * d, c, q_c) &&
               aligned16(x) && aligned16(out);
  const bool vec_ok = (c % 8 == 0) && aligned16(x) && aligned16(out);
  const bool identity = plan->radix_level == 0 || q_c <= 1;
  p.mode = kModeElement;
  if (vec_ok && identity && c % d == 0)
    p.mode = kModeContig;
  else if (vec_ok && !identity && c == q_c * d && (q_c == 2 || q_c == 4 || q_c == 8))
    p.mode = kModeStrided;
  return p;
}

// d = 128, rd = 256 launches with contiguous channel groups and 16-byte aligned rows (bf16 /
// f16, also with the fp8 channel side) take the persistent kernel.
bool fwd_uses_persist(const void* x, const void* out, const OwPlan* plan, int32_t rd, int32_t dtype, int32_t flags,
                      int32_t batch) {
  if (dtype != OW_DTYPE_BF16 && dtype != OW_DTYPE_F16) return false;
  int32_t q_s = 0, q_c = 0;
  if (ow_plan_dims(plan, &q_s, &q_c) != OW_OK) return false;
  const FwdPath p = fwd_path(x, out, plan, q_c, dtype, flags);
  if (p.resident || (p.mode != kModeContig && p.mode != kModeStrided)) return false;
  const int64_t elems = static_cast<int64_t>(batch) * plan->height * plan->width * plan->channels;
  return persist_supported(plan->channel_tile, rd, plan->channels, q_c, elems);
}

// The RMSNorm row scales of a launch come from one of four places (kNorm*); only kNormBuffer
// (and the fp32 kernel with OW_FUSE_NORM) uses the workspace, for batch * H * W floats.
bool fwd_needs_scale_buffer(const void* x, const void* out, const OwPlan* plan, int32_t rd, int32_t dtype,
                            int32_t flags, bool stats_in, int32_t batch) {
  if (!(flags & OW_FUSE_NORM)) return false;
  if (dtype == OW_DTYPE_F32) return true;
  int32_t q_s = 0, q_c = 0;
  if (ow_plan_dims(plan, &q_s, &q_c) != OW_OK) return false;
  const FwdPath p = fwd_path(x, out, plan, q_c, dtype, flags);
  if (p.resident && rd == 2 * plan->channel_tile) return false;
  if (p.mode == kModeElement) return true;
  if (stats_in) return false;
  // The persistent kernel reads whole rows only for strided groups (and forms their scales);
  // with contiguous groups its scales come from the statistics pass (measured: cheaper than
  // whole-row tile fetches through registers at 14x14x512 and 7x7x1024).
  if (fwd_uses_persist(x, out, plan, rd, dtype, flags, batch)) return p.mode != kModeStrided;
  const int32_t c = plan->channels, j = c / 128;
  return !(c % 128 == 0 && (j == 1 || j == 2 || j == 4 || j == 8));
}

}  // namespace ow

extern "C" {

size_t ow_packed_weight_bytes(int32_t q_c, int32_t d, int32_t rd, int32_t compute_dtype) {
  if (q_c < 1 || d < 32 || rd < 32 || d % 32 || rd % 32) return 0;
  if (compute_dtype == OW_DTYPE_F32) return static_cast<size_t>(ow::packed_elems(q_c, d, rd)) * 4;
  return static_cast<size_t>(ow::packed_elems(q_c, d, rd) + ow::packed16_elems(q_c, d, rd)) * 2;
}

size_t ow_fwd_workspace_bytes(const OwPlan* plan, int32_t batch, int32_t flags) {
  if (!plan || batch < 0 || !(flags & OW_FUSE_NORM)) return 0;
  return static_cast<size_t>(batch) * static_cast<size_t>(plan->height) * static_cast<size_t>(plan->width) *
         sizeof(float);
}

int ow_pack_weights(const void* a_u, const void* a_v, const void* a_o, const void* b_u, const void* b_v,
                    const void* b_o, int32_t weight_dtype, const float* norm_weight, const float* gamma,
                    const int32_t* channel_index, int32_t channels, int32_t g, int32_t q_c, int32_t d, int32_t rd,
                    int32_t compute_dtype, void* packed, void* stream) {
  OW_CHECK_ARG(a_u && a_v && a_o && b_u && b_v && b_o && packed, "weight or output pointer is NULL");
  OW_CHECK_ARG(!(norm_weight || gamma) || channel_index, "norm_weight / gamma need channel_index");
  OW_CHECK_ARG(channels >= 1, "channels must be >= 1 (got %d)", channels);
  OW_CHECK_ARG(weight_dtype >= OW_DTYPE_F32 && weight_dtype <= OW_DTYPE_F16, "unknown weight dtype %d", weight_dtype);
  OW_CHECK_SUPPORTED(g == ow::kG, "unsupported spatial tile g=%d; expected 16", g);
  OW_CHECK_ARG(q_c >= 1, "q_c must be >= 1 (got %d)", q_c);
  OW_CHECK_SUPPORTED((d == 64 || d == 128) && (rd == 128 || rd == 256),
                     "unsupported channel tile d=%d / expanded dim rd=%d", d, rd);
  OW_CHECK_SUPPORTED(compute_dtype == OW_DTYPE_BF16 || compute_dtype == OW_DTYPE_F16 || compute_dtype == OW_DTYPE_F32,
                     "unsupported compute dtype %d", compute_dtype);
  if (compute_dtype == OW_DTYPE_F32) {
    if (int rc = ow::pack_weights_f32(a_u, a_v, a_o, b_u, b_v, b_o, weight_dtype, norm_weight, gamma, channel_index,
                                      channels, q_c, d, rd, ow::packed_elems(q_c, d, rd), packed,
                                      static_cast<hipStream_t>(stream)))
      return rc;
    ow::clear_error();
    return OW_OK;
  }
  ow::PackArgs p{a_u, a_v, a_o, b_u, b_v, b_o, norm_weight, gamma, channel_index, packed,
                 weight_dtype, q_c, d, rd, channels, ow::packed_elems(q_c, d, rd)};
  const unsigned blocks = static_cast<unsigned>((p.total + 255) / 256);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (compute_dtype == OW_DTYPE_BF16)
    hipLaunchKernelGGL(ow::pack_kernel<ow::BF16>, dim3(blocks), dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(ow::pack_kernel<ow::F16>, dim3(blocks), dim3(256), 0, s, p);
  if (int rc = ow::hip_status(hipGetLastError(), "pack_kernel launch")) return rc;
  if (const int64_t n16 = ow::packed16_elems(q_c, d, rd)) {
    const unsigned blocks16 = static_cast<unsigned>((n16 + 255) / 256);
    if (compute_dtype == OW_DTYPE_BF16)
      hipLaunchKernelGGL(ow::pack16_kernel<ow::BF16>, dim3(blocks16), dim3(256), 0, s, p, p.total, n16);
    else
      hipLaunchKernelGGL(ow::pack16_kernel<ow::F16>, dim3(blocks16), dim3(256), 0, s, p, p.total, n16);
    if (int rc = ow::hip_status(hipGetLastError(), "pack16_kernel launch")) return rc;
  }
  ow::clear_error();
  return OW_OK;
}

size_t ow_packed_weight_bytes_fp8(int32_t q_c, int32_t d, int32_t rd) {
  if (q_c < 1 || d < 32 || rd < 32 || d % 32 || rd % 32) return 0;
  return static_cast<size_t>(ow::kF8HeadBytes) +
         static_cast<size_t>(q_c) * (rd / 32) * static_cast<size_t>(ow::f8_chunk_units(d)) * 1024;
}

int ow_pack_weights_fp8(const void* a_u, const void* a_v, const void* a_o, const void* b_u, const void* b_v,
                        const void* b_o, int32_t weight_dtype, const float* norm_weight, const float* gamma,
                        const int32_t* channel_index, int32_t channels, int32_t g, int32_t q_c, int32_t d, int32_t rd,
                        int32_t act_dtype, void* packed, void* stream) {
  OW_CHECK_ARG(a_u && a_v && a_o && b_u && b_v && b_o && packed, "tensor pointer is NULL");
  OW_CHECK_ARG(!(norm_weight || gamma) || channel_index, "norm_weight / gamma need channel_index");
  OW_CHECK_ARG(weight_dtype >= OW_DTYPE_F32 && weight_dtype <= OW_DTYPE_F16, "unknown weight dtype %d", weight_dtype);
  OW_CHECK_SUPPORTED(g == ow::kG, "unsupported spatial tile g=%d; expected 16", g);
  OW_CHECK_ARG(q_c >= 1 && channels >= 1, "bad shape q_c=%d channels=%d", q_c, channels);
  OW_CHECK_SUPPORTED((d == 64 || d == 128) && (rd == 128 || rd == 256),
                     "unsupported channel tile d=%d / expanded dim rd=%d", d, rd);
  OW_CHECK_SUPPORTED(act_dtype == OW_DTYPE_BF16 || act_dtype == OW_DTYPE_F16, "unsupported activation dtype %d",
                     act_dtype);
  OW_CHECK_ARG(ow::aligned16(packed), "packed weights must be 16-byte aligned");
  // One thread per 16-bit unit of the head and of the chunks (the scale floats between them are
  // written by f8_zero / f8_amax / f8_finalize).
  const int64_t units = ow::kHeadElems + static_cast<int64_t>(q_c) * (rd / 32) * ow::f8_chunk_units(d) * ow::kFragElems;
  ow::PackArgs p{a_u, a_v, a_o, b_u, b_v, b_o, norm_weight, gamma, channel_index, packed,
                 weight_dtype, q_c, d, rd, channels, units};
  float* scales = reinterpret_cast<float*>(static_cast<uint8_t*>(packed) + ow::kHeadElems * 2);
  const unsigned blocks = static_cast<unsigned>((p.total + 255) / 256);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int n_b = q_c * d * rd;
  hipLaunchKernelGGL(ow::f8_zero_kernel, dim3(1), dim3(64), 0, s, scales);
  hipLaunchKernelGGL(ow::f8_amax_kernel, dim3(static_cast<unsigned>((n_b + 2047) / 2048)), dim3(256), 0, s, p, scales);
  if (act_dtype == OW_DTYPE_BF16) {
    hipLaunchKernelGGL(ow::f8_finalize_kernel<ow::BF16>, dim3(1), dim3(64), 0, s, p, scales);
    hipLaunchKernelGGL(ow::pack_f8_kernel<ow::BF16>, dim3(blocks), dim3(256), 0, s, p, scales);
  } else {
    hipLaunchKernelGGL(ow::f8_finalize_kernel<ow::F16>, dim3(1), dim3(64), 0, s, p, scales);
    hipLaunchKernelGGL(ow::pack_f8_kernel<ow::F16>, dim3(blocks), dim3(256), 0, s, p, scales);
  }
  if (int rc = ow::hip_status(hipGetLastError(), "fp8 pack launch")) return rc;
  ow::clear_error();
  return OW_OK;
}

int ow_rms_scale(const void* x, float* scale, int64_t rows, int32_t channels, float eps, int32_t dtype,
                 void* stream) {
  OW_CHECK_ARG(rows >= 0 && channels >= 1, "bad shape rows=%lld channels=%d", (long long)rows, channels);
  if (rows == 0) {
    ow::clear_error();
    return OW_OK;
  }
  OW_CHECK_ARG(x && scale, "tensor pointer is NULL");
  OW_CHECK_SUPPORTED(dtype == OW_DTYPE_BF16 || dtype == OW_DTYPE_F16 || dtype == OW_DTYPE_F32, "unsupported dtype %d",
                     dtype);
  if (dtype == OW_DTYPE_F32) {
    if (int rc = ow::rms_scale_f32(static_cast<const float*>(x), scale, rows, channels, eps,
                                   static_cast<hipStream_t>(stream)))
      return rc;
    ow::clear_error();
    return OW_OK;
  }
  ow::RmsArgs r{static_cast<const uint16_t*>(x), scale, rows, channels, eps};
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (!ow::aligned16(x)) {  // element path
    const unsigned blocks = static_cast<unsigned>((rows + ow::kWaves - 1) / ow::kWaves);
    if (dtype == OW_DTYPE_BF16)
      hipLaunchKernelGGL(ow::rms_rows_generic_kernel<ow::BF16>, dim3(blocks), dim3(ow::kThreads), 0, s, r);
    else
      hipLaunchKernelGGL(ow::rms_rows_generic_kernel<ow::F16>, dim3(blocks), dim3(ow::kThreads), 0, s, r);
    if (int rc = ow::hip_status(hipGetLastError(), "rms_rows_generic_kernel launch")) return rc;
  } else {
    const int rc = dtype == OW_DTYPE_BF16 ? ow::launch_rms<ow::BF16>(r, s) : ow::launch_rms<ow::F16>(r, s);
    if (rc) return rc;
  }
  ow::clear_error();
  return OW_OK;
}

static int bigemm_fwd_entry(const void* x, void* out, float eps, const void* packed, size_t packed_bytes,
                            const int32_t* token_index, const int32_t* channel_index, const int32_t* out_rows,
                            const OwPlan* plan, int32_t batch, int32_t rd, int32_t dtype, int32_t flags,
                            const float* stats_in, int32_t stats_in_parts, float* stats_out,
                            int32_t* stats_written, const float* drop_scale, void* workspace,
                            size_t workspace_bytes, void* stream, float* scale_out = nullptr,
                            int32_t* scale_written = nullptr) {
  if (stats_written) *stats_written = 0;
  if (scale_written) *scale_written = 0;
  int32_t q_s = 0, q_c = 0;
  if (int rc = ow_plan_dims(plan, &q_s, &q_c)) return rc;
  OW_CHECK_ARG(batch >= 0, "batch must be >= 0 (got %d)", batch);
  OW_CHECK_ARG(packed && token_index && channel_index, "tensor pointer is NULL");
  OW_CHECK_ARG((flags & ~(OW_FUSE_NORM | OW_FUSE_RESIDUAL | OW_FUSE_FP8)) == 0, "unknown flags 0x%x", flags);
  const bool fp8 = (flags & OW_FUSE_FP8) != 0;
  const bool norm = (flags & OW_FUSE_NORM) != 0;
  OW_CHECK_SUPPORTED(!fp8 || (norm && dtype != OW_DTYPE_F32),
                     "OW_FUSE_FP8 needs OW_FUSE_NORM and bf16 / f16 activations");
  OW_CHECK_SUPPORTED(plan->spatial_tile == ow::kG, "unsupported spatial tile g=%d; expected 16", plan->spatial_tile);
  OW_CHECK_SUPPORTED(dtype == OW_DTYPE_BF16 || dtype == OW_DTYPE_F16 || dtype == OW_DTYPE_F32,
                     "unsupported dtype %d; expected bf16, f16 or f32", dtype);
  const int32_t n = plan->height * plan->width, c = plan->channels, d = plan->channel_tile;
  const size_t want = fp8 ? ow_packed_weight_bytes_fp8(q_c, d, rd) : ow_packed_weight_bytes(q_c, d, rd, dtype);
  OW_CHECK_ARG(want != 0 && packed_bytes == want,
               "packed weights hold %zu bytes; q_c=%d d=%d rd=%d needs %zu", packed_bytes, q_c, d, rd, want);
  OW_CHECK_ARG(ow::aligned16(packed), "packed weights must be 16-byte aligned");
  OW_CHECK_SUPPORTED(!out_rows || dtype != OW_DTYPE_F32, "an output-row table needs bf16 or f16 activations");
  OW_CHECK_SUPPORTED(!(out_rows && drop_scale), "a drop-path scale with an output-row table");
  if (batch == 0) {  // empty tensors may carry NULL data pointers; nothing to launch
    ow::clear_error();
    return OW_OK;
  }
  OW_CHECK_ARG(x && out, "tensor pointer is NULL");
  OW_CHECK_ARG(x != out, "out must not alias x");
  OW_CHECK_ARG(static_cast<int64_t>(batch) * n * c < (int64_t(1) << 40), "tensor too large");
  OW_CHECK_ARG(static_cast<int64_t>(batch) * n < (int64_t(1) << 31), "batch * H * W must be < 2^31");
  hipStream_t s = static_cast<hipStream_t>(stream);

  const bool fp32 = dtype == OW_DTYPE_F32;
  const ow::FwdPath path = ow::fwd_path(x, out, plan, q_c, dtype, flags);
  const bool resident = path.resident && rd == 2 * d;
  const int32_t mode = path.mode;
  float* scale = nullptr;
  // scale_out (ow_bigemm_fwd_scales): the row scales go to the caller's buffer where the launch
  // forms them in one place (the statistics pass, or the 16-token kernel below).
  const bool want_scales = scale_out && norm && !out_rows;
  if (ow::fwd_needs_scale_buffer(x, out, plan, rd, dtype, flags, stats_in != nullptr, batch)) {
    if (want_scales) {
      scale = scale_out;
    } else {
      const size_t need = ow_fwd_workspace_bytes(plan, batch, flags);
      OW_CHECK_ARG(workspace && workspace_bytes >= need, "workspace holds %zu bytes; %zu needed", workspace_bytes,
                   need);
      scale = static_cast<float*>(workspace);
    }
    if (int rc = ow_rms_scale(x, scale, static_cast<int64_t>(batch) * n, c, eps, dtype, stream)) return rc;
    if (want_scales) *scale_written = 1;
  }

  if (fp32) {
    if (int rc = ow::launch_fwd_f32(static_cast<const float*>(x), static_cast<float*>(out), scale,
                                    static_cast<const float*>(packed), token_index, channel_index, batch, n, c, q_s,
                                    q_c, d, rd, (flags & OW_FUSE_RESIDUAL) ? 1 : 0, drop_scale, s))
      return rc;
    ow::clear_error();
    return OW_OK;
  }
  if (resident) {
    ow::ResidentArgs r{};
    r.x = static_cast<const uint16_t*>(x);
    r.out = static_cast<uint16_t*>(out);
    r.packed = static_cast<const uint16_t*>(packed);
    r.tok = token_index;
    r.chan = channel_index;
    r.out_tok = out_rows;
    r.batch = batch;
    r.n_tok = n;
    r.channels = c;
    r.q_s = q_s;
    r.q_c = q_c;
    r.n_pairs = static_cast<int32_t>((static_cast<int64_t>(batch) * q_s + 1) / 2);
    r.norm = norm ? 1 : 0;
    r.residual = (flags & OW_FUSE_RESIDUAL) ? 1 : 0;
    r.eps = eps;
    r.drop_scale = drop_scale;
    const int64_t x_elems = static_cast<int64_t>(batch) * n * c;
    const bool wave16 = ow::wave16_supported(d, rd, c, q_c, x_elems);
    if (wave16 && want_scales) {
      r.rs_out = scale_out;
      *scale_written = 1;
    }
    const int rc =
        wave16 ? ow::launch_fwd_wave16(r, plan->radix_level, dtype, s) : ow::launch_fwd_resident(r, dtype, s);
    if (rc != OW_OK && scale_written) *scale_written = 0;
    if (rc == OW_OK) ow::clear_error();
    return rc;
  }
  if (ow::fwd_uses_persist(x, out, plan, rd, dtype, flags, batch)) {
    ow::PersistArgs p{};
    p.x = static_cast<const uint16_t*>(x);
    p.out = static_cast<uint16_t*>(out);
    p.packed = static_cast<const uint16_t*>(packed);
    p.tok = token_index;
    p.out_tok = out_rows;
    p.batch = batch;
    p.n_tok = n;
    p.channels = c;
    p.q_s = q_s;
    p.q_c = q_c;
    p.residual = (flags & OW_FUSE_RESIDUAL) ? 1 : 0;
    p.eps = eps;
    p.drop_scale = drop_scale;
    p.fp8 = fp8 ? 1 : 0;
    p.chan = channel_index;
    p.stride = mode == ow::kModeStrided ? q_c : 1;
    p.norm = ow::kNormNone;
    if (norm) {
      if (scale) {
        p.norm = ow::kNormBuffer;
        p.row_scale = scale;
      } else if (stats_in) {
        p.norm = ow::kNormPartials;
        p.row_scale = stats_in;
        p.parts = stats_in_parts;
      } else {
        p.norm = ow::kNormInline;  // strided groups: scales from the whole-row tile fetch
      }
    }
    if (stats_out && !out_rows) {
      p.stats_out = stats_out;
      if (stats_written) *stats_written = 1;
    }
    const int rc = ow::launch_fwd_persist(p, dtype, s);
    if (rc == OW_OK) ow::clear_error();
    return rc;
  }
  ow::FwdArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.out = static_cast<uint16_t*>(out);
  a.packed = static_cast<const uint16_t*>(packed);
  a.tok = token_index;
  a.chan = channel_index;
  a.out_tok = out_rows;
  a.batch = batch;
  a.n_tok = n;
  a.channels = c;
  a.q_s = q_s;
  a.q_c = q_c;
  a.residual = (flags & OW_FUSE_RESIDUAL) ? 1 : 0;
  a.eps = eps;
  a.drop_scale = drop_scale;
  a.mode = mode;
  a.stride = mode == ow::kModeStrided ? q_c : 1;
  // RMSNorm row scales: the statistics pass above (element access, or whole rows that are not
  // 16 lanes x 1, 2, 4 or 8 vectors), else the previous launch's partial sums when given, else
  // read with the tile.
  a.norm = ow::kNormNone;
  if (norm) {
    if (scale) {
      a.norm = ow::kNormBuffer;
      a.row_scale = scale;
    } else if (stats_in) {
      a.norm = ow::kNormPartials;
      a.row_scale = stats_in;
      a.parts = stats_in_parts;
    } else {
      a.norm = ow::kNormInline;
    }
  }
  if (stats_out && a.mode == ow::kModeContig && !out_rows) {
    a.stats_out = stats_out;
    if (stats_written) *stats_written = 1;
  }
  int rc;
  if (fp8)
    rc = dtype == OW_DTYPE_BF16 ? ow::dispatch_fwd<ow::BF16, true>(a, d, rd, s) : ow::dispatch_fwd<ow::F16, true>(a, d, rd, s);
  else
    rc = dtype == OW_DTYPE_BF16 ? ow::dispatch_fwd<ow::BF16, false>(a, d, rd, s)
                                : ow::dispatch_fwd<ow::F16, false>(a, d, rd, s);
  if (rc == OW_OK) ow::clear_error();
  return rc;
}

int ow_bigemm_fwd(const void* x, void* out, float eps, const void* packed, size_t packed_bytes,
                  const int32_t* token_index, const int32_t* channel_index, const OwPlan* plan, int32_t batch,
                  int32_t rd, int32_t dtype, int32_t flags, void* workspace, size_t workspace_bytes, void* stream) {
  return bigemm_fwd_entry(x, out, eps, packed, packed_bytes, token_index, channel_index, nullptr, plan, batch, rd,
                          dtype, flags, nullptr, 0, nullptr, nullptr, nullptr, workspace, workspace_bytes, stream);
}

int ow_bigemm_fwd_rows(const void* x, void* out, float eps, const void* packed, size_t packed_bytes,
                       const int32_t* token_index, const int32_t* channel_index, const int32_t* out_rows,
                       const OwPlan* plan, int32_t batch, int32_t rd, int32_t dtype, int32_t flags, void* workspace,
                       size_t workspace_bytes, void* stream) {
  OW_CHECK_ARG(out_rows, "out_rows is NULL");
  return bigemm_fwd_entry(x, out, eps, packed, packed_bytes, token_index, channel_index, out_rows, plan, batch, rd,
                          dtype, flags, nullptr, 0, nullptr, nullptr, nullptr, workspace, workspace_bytes, stream);
}

int ow_bigemm_fwd_chain(const void* x, void* out, float eps, const void* packed, size_t packed_bytes,
                        const int32_t* token_index, const int32_t* channel_index, const int32_t* out_rows,
                        const OwPlan* plan, int32_t batch, int32_t rd, int32_t dtype, int32_t flags,
                        const float* stats_in, int32_t stats_in_parts, float* stats_out, int32_t* stats_written,
                        void* workspace, size_t workspace_bytes, void* stream) {
  OW_CHECK_ARG(stats_written, "stats_written is NULL");
  *stats_written = 0;
  OW_CHECK_SUPPORTED(dtype != OW_DTYPE_F32, "row statistics between launches need bf16 or f16 activations");
  OW_CHECK_ARG(!stats_in || (stats_in_parts >= 1 && stats_in_parts <= 64),
               "stats_in_parts must be in [1, 64] (got %d)", stats_in_parts);
  OW_CHECK_ARG(!stats_in || (flags & OW_FUSE_NORM), "stats_in without OW_FUSE_NORM");
  if (stats_in && stats_out && batch > 0 && plan) {
    // The launch reads stats_in while it writes stats_out, from different workgroups: the two
    // must not share memory.
    int32_t q_s_chk = 0, q_c_chk = 0;
    if (int rc = ow_plan_dims(plan, &q_s_chk, &q_c_chk)) return rc;
    const int64_t rows = static_cast<int64_t>(batch) * plan->height * plan->width;
    const auto in0 = reinterpret_cast<uintptr_t>(stats_in), out0 = reinterpret_cast<uintptr_t>(stats_out);
    const uintptr_t in1 = in0 + static_cast<uintptr_t>(rows) * stats_in_parts * sizeof(float);
    const uintptr_t out1 = out0 + static_cast<uintptr_t>(rows) * q_c_chk * sizeof(float);
    OW_CHECK_ARG(in1 <= out0 || out1 <= in0, "stats_in and stats_out overlap");
  }
  return bigemm_fwd_entry(x, out, eps, packed, packed_bytes, token_index, channel_index, out_rows, plan, batch, rd,
                          dtype, flags, stats_in, stats_in_parts, stats_out, stats_written, nullptr, workspace,
                          workspace_bytes, stream);
}

int ow_bigemm_fwd_scales(const void* x, void* out, float eps, const void* packed, size_t packed_bytes,
                         const int32_t* token_index, const int32_t* channel_index, const OwPlan* plan,
                         int32_t batch, int32_t rd, int32_t dtype, int32_t flags, const float* drop_scale,
                         float* row_scale, int32_t* scales_written, void* workspace, size_t workspace_bytes,
                         void* stream) {
  OW_CHECK_ARG(scales_written, "scales_written is NULL");
  *scales_written = 0;
  OW_CHECK_ARG(row_scale || batch == 0, "row_scale is NULL");
  return bigemm_fwd_entry(x, out, eps, packed, packed_bytes, token_index, channel_index, nullptr, plan, batch, rd,
                          dtype, flags, nullptr, 0, nullptr, nullptr, drop_scale, workspace, workspace_bytes, stream,
                          row_scale, scales_written);
}

int ow_bigemm_fwd_drop(const void* x, void* out, float eps, const void* packed, size_t packed_bytes,
                       const int32_t* token_index, const int32_t* channel_index, const OwPlan* plan, int32_t batch,
                       int32_t rd, int32_t dtype, int32_t flags, const float* drop_scale, void* workspace,
                       size_t workspace_bytes, void* stream) {
  OW_CHECK_ARG(drop_scale || batch == 0, "drop_scale is NULL");
  return bigemm_fwd_entry(x, out, eps, packed, packed_bytes, token_index, channel_index, nullptr, plan, batch, rd,
                          dtype, flags, nullptr, 0, nullptr, nullptr, drop_scale, workspace, workspace_bytes,
                          stream);
}

}  // extern "C"
