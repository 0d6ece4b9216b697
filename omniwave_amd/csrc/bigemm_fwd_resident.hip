// Persistent BiGEMM forward for small channel counts: d = 64, rd = 128, C = q_c * 64 with
// q_c in {1, 2, 4} (the 56x56x128 and 28x28x256 stages of OmniWeave-T).
//
// Same math and operand packing as the streamed tile kernel (bigemm_fwd.hip; reference
// omniweave/ops/reference.py:147-171), organised so that nothing but activations moves:
//   * one workgroup = 2 q_c waves; waves 2g and 2g + 1 own channel group g and split its
//     expanded dimension: wave half h keeps the packed weights of chunks 2h and 2h + 1
//     (24 KB) resident in its registers, computes its share of W = Z B_o, and the two halves
//     exchange partial sums through LDS; each then finishes one 32-channel half of delta.
//     Two waves per SIMD let one wave's LDS / memory waits overlap the other's work;
//   * the workgroup walks 32-token pairs of token groups (pair p = groups 2p and 2p + 1 of the
//     flattened batch x q_s order), persistent over the grid;
//   * each pair's full rows (32 tokens x C channels) are prefetched into registers one pair
//     ahead, then written to a triple-buffered LDS tile; the RMSNorm statistics come from the
//     same registers, so no separate statistics pass reads x again;
//   * routes are address arithmetic: the token table picks rows, the channel table picks the
//     tile columns a wave reads and writes, so the radix channel rotation costs nothing;
//   * the residual is added in the LDS tile, which is then written back as whole rows with
//     16-byte stores.
// Pipeline per pair i: registers(i) -> RMS scales + LDS tile(i); barrier; issue the loads of
// pair i+1 (and token-table reads of pair i+2), store the rows of pair i-1 from LDS; token side
// and both chunks of this wave; partial-W exchange (barrier); delta into LDS tile(i).  Three
// tile buffers: the stores of pair i-1 may still be reading buffer (i-1) % 3 while a faster
// wave fills buffer (i+1) % 3.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "ow_device.h"

namespace ow {
namespace {

constexpr int kRD = 128;
constexpr int kD = 64;
constexpr int kKS = kD / 16;               // 16-deep K steps over a channel group
constexpr int kMB = kD / 32;               // 32-channel blocks of W (= halves of the group)
constexpr int kNCH = kRD / 32;             // 32-row chunks of the expanded dimension
constexpr int kHalfCh = kNCH / 2;          // chunks per wave
constexpr int kFrU = kKS;                  // B_u'^T fragments per chunk (B_v'^T the same)
constexpr int kFrCh = 2 * kFrU + 2 * kMB;  // fragments per chunk
constexpr int kChElems = kFrCh * kFragElems;
constexpr int kPairRows = 2 * kG;          // 32 tokens per pair
constexpr int kNBuf = 3;
static_assert(kMB == 2, "one 32-channel output half per wave of a group");

template <int QC>
struct ResidentLds {
  static constexpr int C = QC * kD;
  static constexpr int LDC = C + 8;  // tile row stride (elements)
  uint16_t tile[kNBuf][kPairRows * LDC];
  float rsc[kNBuf][kPairRows];
  float dsc[kNBuf][2];      // drop-path scale of the pair's two token groups (DROP)
  u32x4 xch[QC][2][4][64];  // partial W (f32x16 per lane as 4 quarters) by group and writer half
  u32x4 head[3][64];        // token-operand rows A_u, A_v, A_o
};

// Position of a pair's first token group 2 pair = b q_s + s (image b, group s of the image).
// The loop advances it by the grid stride with additions only: a division per pair would cost
// a long scalar sequence in every iteration.
struct PairPos {
  int32_t b, s;
};

__device__ __forceinline__ PairPos pair_pos(int64_t pair, int32_t q_s) {
  const int64_t tg0 = 2 * pair;
  const int32_t b = static_cast<int32_t>(tg0 / q_s);
  return PairPos{b, static_cast<int32_t>(tg0 - static_cast<int64_t>(b) * q_s)};
}

// pos += (step_b, step_s) with step_s < q_s: the position of the pair n_wg further on.
__device__ __forceinline__ void pair_advance(PairPos& pos, int32_t step_b, int32_t step_s, int32_t q_s) {
  pos.b += step_b;
  pos.s += step_s;
  if (pos.s >= q_s) {
    pos.s -= q_s;
    ++pos.b;
  }
}

// Token-table entries of the NI rows this lane loads and stores in a pair (with OM, also the
// output-row table entries), with the image index of each row (>= batch past the end).  Only
// loads: the values are examined one iteration later (row_id), so the loads are not waited on
// while the row prefetch is in flight.
template <int NI, int RPW, int RPI, int LPR, bool OM>
__device__ __forceinline__ void pair_row_tok(const ResidentArgs& a, PairPos pos, int wave, int lane,
                                             int32_t (&t)[NI], int32_t (&to)[NI], int32_t (&b)[NI]) {
  const int32_t b0 = pos.b, s0 = pos.s;  // uniform
#pragma unroll
  for (int j = 0; j < NI; ++j) {
    const int r = wave * RPW + j * RPI + lane / LPR;
    int32_t bb = b0, s = s0 + r / kG;
    if (s == a.q_s) {
      s = 0;
      ++bb;
    }
    b[j] = bb;
    t[j] = a.tok[s * kG + (r % kG)];  // s < q_s: in bounds even for rows past the end
    if (OM) to[j] = a.out_tok[s * kG + (r % kG)];
  }
}

__device__ __forceinline__ int32_t row_id(const ResidentArgs& a, int32_t t, int32_t b) {
  return (b < a.batch && t >= 0 && t < a.n_tok) ? b * a.n_tok + t : -1;
}

// Output row of a token slot whose input row is `in` (-1: pad slot, not stored).
template <bool OM>
__device__ __forceinline__ int32_t out_id(const ResidentArgs& a, int32_t in, int32_t to, int32_t b) {
  if (!OM) return in;
  return in >= 0 ? row_id(a, to, b) : -1;
}

template <int C>
__device__ __forceinline__ u32x4 load_row_vec(const uint16_t* x, int32_t id, int vcol) {
  u32x4 v = {0u, 0u, 0u, 0u};
  if (id >= 0) v = *reinterpret_cast<const u32x4*>(x + static_cast<int64_t>(id) * C + vcol);
  return v;
}

// The persistent loop of one wave: channel group g, expanded-dimension half HF.  OM: rows are
// stored at the output-row table's positions instead of their input positions.  DROP: the
// rounded delta of each image is multiplied by a.drop_scale[image] before the residual.
template <class Ty, int QC, int HF, bool OM, bool DROP>
__device__ __forceinline__ void resident_wave(const ResidentArgs& a, ResidentLds<QC>& sh, int g, int n_iter) {
  constexpr int C = QC * kD;
  constexpr int LDC = ResidentLds<QC>::LDC;
  constexpr int NW = 2 * QC;           // waves per workgroup
  constexpr int RPW = kPairRows / NW;  // rows each wave loads and stores
  constexpr int LPR = C / 8;           // lanes per row (16-byte vectors)
  constexpr int RPI = 64 / LPR;        // rows per wave-wide vector access
  constexpr int NI = RPW / RPI;        // row vectors per lane
  static_assert(NI == 2, "two row vectors per lane");

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int hh = lane >> 5, l32 = lane & 31;
  const int vcol = (lane % LPR) * 8;  // first column of this lane's row vectors
  const int64_t n_wg = gridDim.x;
  const int64_t first = blockIdx.x;

  // Resident weights of chunks 2 HF and 2 HF + 1 of channel group g (96 registers).  They stay
  // in ordinary VGPRs: with 2 waves per SIMD a wave has 256 registers, and pinning the weights
  // to AGPRs would split that budget 128 / 128 and spill the loop's VGPRs into AGPRs (a copy
  // each way per spilled value, ~50 VALU instructions per pair).
  const uint16_t* wsrc = a.packed + kHeadElems + (static_cast<size_t>(g) * kNCH + kHalfCh * HF) * kChElems;
  u32x4 wt[kHalfCh][kFrCh];
#pragma unroll
  for (int e = 0; e < kHalfCh; ++e)
#pragma unroll
    for (int f = 0; f < kFrCh; ++f) wt[e][f] = reinterpret_cast<const u32x4*>(wsrc + e * kChElems + f * kFragElems)[lane];
  int col[kMB];  // tile column of group channel 32 cb + l32
#pragma unroll
  for (int cb = 0; cb < kMB; ++cb) {
    const int c = a.chan[g * kD + 32 * cb + l32];
    col[cb] = (c >= 0 && c < C) ? c : 0;  // tables of a plan with C = q_c * d hold no pads
  }

  // ids_prev: output rows being stored (pair it - 1); ids_cur: output rows of pair it; tok_n /
  // tout_n / img_n: raw table entries of pair it + 1.
  int32_t ids_cur[NI], ids_prev[NI];
  int32_t tok_n[NI], tout_n[NI], img_n[NI];
  u32x4 xr[NI];
  // DROP: drop-path scale of the rows of pair it (loaded with the rows, one pair ahead).
  float ds_cur[NI];
  auto drop_of = [&](int32_t img) { return a.drop_scale[img < a.batch ? img : a.batch - 1]; };
  // pos: the pair whose table entries are read next; the grid stride in groups is 2 n_wg.
  const int32_t step_b = static_cast<int32_t>(2 * n_wg / a.q_s);
  const int32_t step_s = static_cast<int32_t>(2 * n_wg - static_cast<int64_t>(step_b) * a.q_s);
  PairPos pos = pair_pos(first, a.q_s);
  pair_row_tok<NI, RPW, RPI, LPR, OM>(a, pos, wave, lane, tok_n, tout_n, img_n);
#pragma unroll
  for (int j = 0; j < NI; ++j) {
    ids_prev[j] = -1;
    const int32_t in = row_id(a, tok_n[j], img_n[j]);
    ids_cur[j] = out_id<OM>(a, in, tout_n[j], img_n[j]);
    xr[j] = load_row_vec<C>(a.x, in, vcol);
    ds_cur[j] = DROP ? drop_of(img_n[j]) : 1.0f;
  }
  if (n_iter > 1) {
    pair_advance(pos, step_b, step_s, a.q_s);
    pair_row_tok<NI, RPW, RPI, LPR, OM>(a, pos, wave, lane, tok_n, tout_n, img_n);
  } else {
#pragma unroll
    for (int j = 0; j < NI; ++j) img_n[j] = a.batch;
  }

#pragma unroll 1
  for (int it = 0; it < n_iter; ++it) {
    const int buf = it % kNBuf;
    uint16_t* tl = sh.tile[buf];

    // (1) RMSNorm row scales and this wave's rows of the pair's tile.
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      const int r = wave * RPW + j * RPI + lane / LPR;
      if (a.norm) {
        float acc = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; ++e) acc = Ty::dot2sq(xr[j][e], acc);
        acc = group_sum<LPR>(acc);
        if (lane % LPR == LPR - 1) sh.rsc[buf][r] = rms_scale<Ty>(acc / static_cast<float>(C), a.eps);
      }
      *reinterpret_cast<u32x4*>(&tl[r * LDC + vcol]) = xr[j];
      if (DROP && lane % LPR == 0 && r % kG == 0) sh.dsc[buf][r / kG] = ds_cur[j];
    }
    __syncthreads();

    // (2) Loads first, then stores: rows of pair it + 1, token-table entries of pair it + 2,
    // then the rows of pair it - 1 (complete in their buffer since the barrier) to memory.
    int32_t ids_next[NI];
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      const int32_t in = row_id(a, tok_n[j], img_n[j]);
      ids_next[j] = out_id<OM>(a, in, tout_n[j], img_n[j]);
      xr[j] = load_row_vec<C>(a.x, in, vcol);
      if (DROP) ds_cur[j] = drop_of(img_n[j]);  // pair it + 1 (this pair's were written in (1))
    }
    if (it + 2 < n_iter) {
      pair_advance(pos, step_b, step_s, a.q_s);
      pair_row_tok<NI, RPW, RPI, LPR, OM>(a, pos, wave, lane, tok_n, tout_n, img_n);
    } else {
#pragma unroll
      for (int j = 0; j < NI; ++j) img_n[j] = a.batch;
    }
    if (it > 0) {
      const uint16_t* pt = sh.tile[(it + kNBuf - 1) % kNBuf];
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        const int r = wave * RPW + j * RPI + lane / LPR;
        if (ids_prev[j] >= 0)
          *reinterpret_cast<u32x4*>(a.out + static_cast<int64_t>(ids_prev[j]) * C + vcol) =
              *reinterpret_cast<const u32x4*>(&pt[r * LDC + vcol]);
      }
    }
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      ids_prev[j] = ids_cur[j];
      ids_cur[j] = ids_next[j];
    }
    // Keep the loads and stores ahead of the compute: the next iteration waits on the prefetch,
    // and the counter it waits on also covers these stores, so they must be issued early.
    __builtin_amdgcn_sched_barrier(0);

    // (3) Token side (the whole group's P, both halves compute it), (4) this wave's chunks.
    u32x4 bu = sh.head[0][lane], bv = sh.head[1][lane];
    if (a.norm) {  // lane's slots j are tokens 16 tg + kord(j, hh) of its group tg
      const float* r8 = &sh.rsc[buf][16 * ((lane >> 4) & 1) + 4 * hh];
      bu = scale8<Ty>(bu, r8);
      bv = scale8<Ty>(bv, r8);
    }
    u32x4 Pu[kKS], Pv[kKS], xk[kMB][2];
    pair_token_side<Ty, kKS>(tl, LDC, col, bu, bv, lane, Pu, Pv, xk);
    f32x16 W[kMB] = {};
#pragma unroll
    for (int e = 0; e < kHalfCh; ++e) {
      auto fu = [&](int ks) { return wt[e][ks]; };
      auto fv = [&](int ks) { return wt[e][kFrU + ks]; };
      auto fo = [&](int mb, int s) { return wt[e][2 * kFrU + 2 * mb + s]; };
      pair_chunk<Ty, kKS, kMB>(Pu, Pv, fu, fv, fo, W);
    }

    // (5) Partial-W exchange: hand the partner its half (channels 32 (1-HF) ..), take ours.
    mfma_drain();
#pragma unroll
    for (int q = 0; q < 4; ++q)
      sh.xch[g][HF][q][lane] = u32x4{__float_as_uint(W[1 - HF][4 * q]), __float_as_uint(W[1 - HF][4 * q + 1]),
                                     __float_as_uint(W[1 - HF][4 * q + 2]), __float_as_uint(W[1 - HF][4 * q + 3])};
    __syncthreads();
    f32x16 Wh[1];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const u32x4 o = sh.xch[g][1 - HF][q][lane];
#pragma unroll
      for (int k = 0; k < 4; ++k) Wh[0][4 * q + k] = W[HF][4 * q + k] + __uint_as_float(o[k]);
    }

    // (6) delta = A_o W for channels 32 HF + l32, (7) rounded (plus x with the residual) into
    // the own columns of the tile.
    f32x16 dl[1];
    pair_output<Ty, 1>(Wh, sh.head[2][lane], lane, dl);
    mfma_drain();
    auto dst = [&](int i) { return &tl[pair_token_row(i, hh) * LDC + col[HF]]; };
    const float s0 = DROP ? sh.dsc[buf][0] : 1.0f, s1 = DROP ? sh.dsc[buf][1] : 1.0f;
    if (a.residual)
      pair_store_block<Ty, true, DROP>(dl[0], xk[HF], dst, s0, s1);
    else
      pair_store_block<Ty, false, DROP>(dl[0], xk[HF], dst, s0, s1);
  }

  // Rows of the last pair (ids_prev was rotated to it by the last iteration).
  __syncthreads();
  const uint16_t* pt = sh.tile[(n_iter - 1) % kNBuf];
#pragma unroll
  for (int j = 0; j < NI; ++j) {
    const int r = wave * RPW + j * RPI + lane / LPR;
    if (ids_prev[j] >= 0)
      *reinterpret_cast<u32x4*>(a.out + static_cast<int64_t>(ids_prev[j]) * C + vcol) =
          *reinterpret_cast<const u32x4*>(&pt[r * LDC + vcol]);
  }
}

template <class Ty, int QC, bool OM, bool DROP>
__global__ void __attribute__((amdgpu_flat_work_group_size(128 * QC, 128 * QC), amdgpu_waves_per_eu(2, 2)))
bigemm_fwd_resident_kernel(ResidentArgs a) {
  __shared__ __attribute__((aligned(16))) ResidentLds<QC> sh;
  const int64_t n_wg = gridDim.x;
  const int64_t first = blockIdx.x;
  const int n_iter = first < a.n_pairs ? static_cast<int>((a.n_pairs - 1 - first) / n_wg + 1) : 0;
  if (n_iter == 0) return;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int f = wave; f < 3; f += 2 * QC)  // 2 waves when q_c = 1
    sh.head[f][lane] = reinterpret_cast<const u32x4*>(a.packed + f * kFragElems)[lane];
  __syncthreads();
  if (wave & 1)
    resident_wave<Ty, QC, 1, OM, DROP>(a, sh, wave >> 1, n_iter);
  else
    resident_wave<Ty, QC, 0, OM, DROP>(a, sh, wave >> 1, n_iter);
}

template <class Ty, int QC>
int launch_qc(const ResidentArgs& a, hipStream_t stream) {
  // Two waves per SIMD, 2 QC waves per workgroup: 4 / QC workgroups per CU.
  const int64_t slots = static_cast<int64_t>(device_cus()) * (4 / QC);
  const int64_t grid = a.n_pairs < slots ? a.n_pairs : slots;
  if (grid <= 0) return OW_OK;
  if (a.out_tok && a.drop_scale) return fail(OW_ERR_UNSUPPORTED, "an output-row table with a drop-path scale");
  if (a.out_tok)
    hipLaunchKernelGGL((bigemm_fwd_resident_kernel<Ty, QC, true, false>), dim3(static_cast<unsigned>(grid)),
                       dim3(128 * QC), 0, stream, a);
  else if (a.drop_scale)
    hipLaunchKernelGGL((bigemm_fwd_resident_kernel<Ty, QC, false, true>), dim3(static_cast<unsigned>(grid)),
                       dim3(128 * QC), 0, stream, a);
  else
    hipLaunchKernelGGL((bigemm_fwd_resident_kernel<Ty, QC, false, false>), dim3(static_cast<unsigned>(grid)),
                       dim3(128 * QC), 0, stream, a);
  return hip_status(hipGetLastError(), "bigemm_fwd_resident_kernel launch");
}

template <class Ty>
int launch_ty(const ResidentArgs& a, hipStream_t stream) {
  switch (a.q_c) {
    case 1: return launch_qc<Ty, 1>(a, stream);
    case 2: return launch_qc<Ty, 2>(a, stream);
    case 4: return launch_qc<Ty, 4>(a, stream);
    default: return fail(OW_ERR_UNSUPPORTED, "resident forward needs q_c in {1, 2, 4} (got %d)", a.q_c);
  }
}

}  // namespace

bool resident_supported(int32_t d, int32_t rd, int32_t channels, int32_t q_c) {
  return d == kD && rd == kRD && (q_c == 1 || q_c == 2 || q_c == 4) && channels == q_c * kD;
}

int launch_fwd_resident(const ResidentArgs& a, int32_t dtype, hipStream_t stream) {
  if (dtype == OW_DTYPE_BF16) return launch_ty<BF16>(a, stream);
  if (dtype == OW_DTYPE_F16) return launch_ty<F16>(a, stream);
  return fail(OW_ERR_UNSUPPORTED, "unsupported dtype %d", dtype);
}

}  // namespace ow
