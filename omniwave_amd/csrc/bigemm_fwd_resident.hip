// Persistent BiGEMM forward for small channel counts: d = 64, rd = 128, C = q_c * 64 with
// q_c in {1, 2, 4} (the 56x56x128 and 28x28x256 stages of OmniWeave-T).
//
// Same math and operand packing as the streamed tile kernel (bigemm_fwd.hip; reference
// omniweave/ops/reference.py:147-171), organised so that nothing but activations moves:
//   * one workgroup = q_c waves, wave w owns channel group w; its 48 KB of packed weights
//     (B_u'^T, B_v'^T, B_o fragments) are loaded into registers once and stay there;
//   * the workgroup walks 32-token pairs of token groups (pair p = groups 2p and 2p + 1 of the
//     flattened batch x q_s order), persistent over the grid;
//   * each pair's full rows (32 tokens x C channels) are prefetched into registers one pair
//     ahead, then written to a triple-buffered LDS tile; the RMSNorm statistics come from the
//     same registers, so no separate statistics pass reads x again;
//   * routes are address arithmetic: the token table picks rows, the channel table picks the
//     tile columns a wave reads and writes, so the radix channel rotation costs nothing;
//   * the residual is added in the LDS tile, which is then written back as whole rows with
//     16-byte stores.
// Pipeline per pair i: registers(i) -> RMS scales + LDS tile(i); barrier; store rows of pair
// i-1 from LDS; issue the loads of pair i+1 (and token-table reads of pair i+2); compute pair
// i into LDS tile(i).  Three tile buffers: the stores of pair i-1 may still be reading
// buffer (i-1) % 3 while a faster wave fills buffer (i+1) % 3.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "ow_device.h"

namespace ow {
namespace {

constexpr int kRD = 128;
constexpr int kD = 64;
constexpr int kKS = kD / 16;               // 16-deep K steps over a channel group
constexpr int kMB = kD / 32;               // 32-channel blocks of W
constexpr int kNCH = kRD / 32;             // 32-row chunks of the expanded dimension
constexpr int kFrU = kKS;                  // B_u'^T fragments per chunk (B_v'^T the same)
constexpr int kFrCh = 2 * kFrU + 2 * kMB;  // fragments per chunk
constexpr int kChElems = kFrCh * kFragElems;
constexpr int kPairRows = 2 * kG;          // 32 tokens per pair
constexpr int kNBuf = 3;

// Token-table entries of the 4 rows this lane loads and stores in a pair, with the image
// index of each row (>= batch past the end).  Only loads: the values are examined one
// iteration later (row_id), so the loads are not waited on while the row prefetch is in flight.
template <int RPW, int RPI, int LPR>
__device__ __forceinline__ void pair_row_tok(const ResidentArgs& a, int64_t pair, int wave, int lane,
                                             int32_t (&t)[4], int32_t (&b)[4]) {
  const int64_t tg0 = 2 * pair;  // first group of the pair (uniform)
  const int32_t b0 = static_cast<int32_t>(tg0 / a.q_s);
  const int32_t s0 = static_cast<int32_t>(tg0 - static_cast<int64_t>(b0) * a.q_s);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = wave * RPW + j * RPI + lane / LPR;
    int32_t bb = b0, s = s0 + r / kG;
    if (s == a.q_s) {
      s = 0;
      ++bb;
    }
    b[j] = bb;
    t[j] = a.tok[s * kG + (r % kG)];  // s < q_s: in bounds even for rows past the end
  }
}

__device__ __forceinline__ int32_t row_id(const ResidentArgs& a, int32_t t, int32_t b) {
  return (b < a.batch && t >= 0 && t < a.n_tok) ? b * a.n_tok + t : -1;
}

template <int C>
__device__ __forceinline__ u32x4 load_row_vec(const uint16_t* x, int32_t id, int vcol) {
  u32x4 v = {0u, 0u, 0u, 0u};
  if (id >= 0) v = *reinterpret_cast<const u32x4*>(x + static_cast<int64_t>(id) * C + vcol);
  return v;
}

template <class Ty, int QC>
__global__ void __attribute__((amdgpu_flat_work_group_size(64 * QC, 64 * QC), amdgpu_waves_per_eu(1, 1)))
bigemm_fwd_resident_kernel(ResidentArgs a) {
  constexpr int C = QC * kD;
  constexpr int LDC = C + 8;           // tile row stride (elements)
  constexpr int RPW = kPairRows / QC;  // rows each wave loads and stores
  constexpr int LPR = C / 8;           // lanes per row (16-byte vectors)
  constexpr int RPI = 64 / LPR;        // rows per wave-wide vector access
  static_assert(RPW / RPI == 4, "four row vectors per lane");

  __shared__ __attribute__((aligned(16))) uint16_t tile[kNBuf][kPairRows * LDC];
  __shared__ __attribute__((aligned(16))) float rsc[kNBuf][kPairRows];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int hh = lane >> 5, l32 = lane & 31;
  const int vcol = (lane % LPR) * 8;  // first column of this lane's row vectors

  const int64_t n_wg = gridDim.x;
  const int64_t first = blockIdx.x;
  const int n_iter = first < a.n_pairs ? static_cast<int>((a.n_pairs - 1 - first) / n_wg + 1) : 0;
  if (n_iter == 0) return;

  // Resident operands of channel group `wave`.
  const uint16_t* wsrc = a.packed + kHeadElems + static_cast<size_t>(wave) * kNCH * kChElems;
  u32x4 wt[kNCH][kFrCh];
#pragma unroll
  for (int ec = 0; ec < kNCH; ++ec)
#pragma unroll
    for (int f = 0; f < kFrCh; ++f)
      wt[ec][f] = reinterpret_cast<const u32x4*>(wsrc + ec * kChElems + f * kFragElems)[lane];
  const u32x4 fAu = reinterpret_cast<const u32x4*>(a.packed)[lane];
  const u32x4 fAv = reinterpret_cast<const u32x4*>(a.packed + kFragElems)[lane];
  const u32x4 fAo = reinterpret_cast<const u32x4*>(a.packed + 2 * kFragElems)[lane];
  int col[kMB];     // tile column of group channel 32 cb + l32
  float gmv[kMB];   // LayerScale of that column
#pragma unroll
  for (int cb = 0; cb < kMB; ++cb) {
    int c = a.chan[wave * kD + 32 * cb + l32];
    c = (c >= 0 && c < C) ? c : 0;  // tables of a plan with C = q_c * d hold no pads
    col[cb] = c;
    gmv[cb] = a.gamma[c];
  }

  // ids_prev: rows being stored (pair it - 1); ids_cur: rows of pair it; tok_n / img_n: raw
  // table entries of pair it + 1.
  int32_t ids_cur[4], ids_prev[4] = {-1, -1, -1, -1};
  int32_t tok_n[4], img_n[4];
  u32x4 xr[4];
  pair_row_tok<RPW, RPI, LPR>(a, first, wave, lane, tok_n, img_n);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    ids_cur[j] = row_id(a, tok_n[j], img_n[j]);
    xr[j] = load_row_vec<C>(a.x, ids_cur[j], vcol);
  }
  if (n_iter > 1) {
    pair_row_tok<RPW, RPI, LPR>(a, first + n_wg, wave, lane, tok_n, img_n);
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) img_n[j] = a.batch;
  }

#pragma unroll 1
  for (int it = 0; it < n_iter; ++it) {
    const int buf = it % kNBuf;
    uint16_t* tl = tile[buf];

    // (1) RMSNorm row scales and the tile of this pair.
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = wave * RPW + j * RPI + lane / LPR;
      if (a.norm) {
        float acc = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; ++e) acc = Ty::dot2sq(xr[j][e], acc);
        acc = group_sum<LPR>(acc);
        if (lane % LPR == LPR - 1) rsc[buf][r] = rms_scale<Ty>(acc / static_cast<float>(C), a.eps);
      }
      *reinterpret_cast<u32x4*>(&tl[r * LDC + vcol]) = xr[j];
    }
    __syncthreads();

    // (2) Loads first, then stores: rows of pair it + 1, token-table entries of pair it + 2,
    // then the rows of pair it - 1 (complete in their buffer since the barrier) to memory.
    int32_t ids_next[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      ids_next[j] = row_id(a, tok_n[j], img_n[j]);
      xr[j] = load_row_vec<C>(a.x, ids_next[j], vcol);
    }
    if (it + 2 < n_iter) {
      pair_row_tok<RPW, RPI, LPR>(a, first + (it + 2) * n_wg, wave, lane, tok_n, img_n);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) img_n[j] = a.batch;
    }
    if (it > 0) {
      const uint16_t* pt = tile[(it + kNBuf - 1) % kNBuf];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = wave * RPW + j * RPI + lane / LPR;
        if (ids_prev[j] >= 0)
          *reinterpret_cast<u32x4*>(a.out + static_cast<int64_t>(ids_prev[j]) * C + vcol) =
              *reinterpret_cast<const u32x4*>(&pt[r * LDC + vcol]);
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      ids_prev[j] = ids_cur[j];
      ids_cur[j] = ids_next[j];
    }
    // Keep the loads and stores ahead of the compute: the next iteration waits on the prefetch,
    // and the counter it waits on also covers these stores, so they must be issued early.
    __builtin_amdgcn_sched_barrier(0);

    // (4) Token side, (5) channel side with the resident weights, (6) delta = A_o W.
    u32x4 bu = fAu, bv = fAv;
    if (a.norm) {  // lane's slots j are tokens 16 tg + kord(j, hh) of its group tg
      const float* r8 = &rsc[buf][16 * ((lane >> 4) & 1) + 4 * hh];
      bu = scale8<Ty>(fAu, r8);
      bv = scale8<Ty>(fAv, r8);
    }
    u32x4 Pu[kKS], Pv[kKS], xk[kMB][2];
    pair_token_side<Ty, kKS>(tl, LDC, col, bu, bv, lane, Pu, Pv, xk);
    f32x16 W[kMB] = {};
#pragma unroll
    for (int ec = 0; ec < kNCH; ++ec) {
      auto fu = [&](int ks) { return wt[ec][ks]; };
      auto fv = [&](int ks) { return wt[ec][kFrU + ks]; };
      auto fo = [&](int mb, int s) { return wt[ec][2 * kFrU + 2 * mb + s]; };
      pair_chunk<Ty, kKS, kMB>(Pu, Pv, fu, fv, fo, W);
    }
    f32x16 dl[kMB];
    pair_output<Ty, kMB>(W, fAo, lane, dl);
    mfma_drain();

    // (7) delta (rounded, LayerScale applied), plus x from the token-side operands with the
    // residual, written over the own columns.
    if (a.residual) {
#pragma unroll
      for (int mb = 0; mb < kMB; ++mb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float xv = Ty::to_f32(packed_elem(xk[mb][i >> 3], i & 7));
          tl[pair_token_row(i, hh) * LDC + col[mb]] = Ty::from_f32(xv + round_to<Ty>(dl[mb][i] * gmv[mb]));
        }
    } else {
#pragma unroll
      for (int mb = 0; mb < kMB; ++mb)
#pragma unroll
        for (int i = 0; i < 16; ++i) tl[pair_token_row(i, hh) * LDC + col[mb]] = Ty::from_f32(dl[mb][i] * gmv[mb]);
    }
  }

  // Rows of the last pair (ids_prev was rotated to it by the last iteration).
  __syncthreads();
  const uint16_t* pt = tile[(n_iter - 1) % kNBuf];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = wave * RPW + j * RPI + lane / LPR;
    if (ids_prev[j] >= 0)
      *reinterpret_cast<u32x4*>(a.out + static_cast<int64_t>(ids_prev[j]) * C + vcol) =
          *reinterpret_cast<const u32x4*>(&pt[r * LDC + vcol]);
  }
}

// Compute units of the current device (cached per device id).
int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

template <class Ty, int QC>
int launch_qc(const ResidentArgs& a, hipStream_t stream) {
  // One wave per SIMD (the weights take most of the register file): 4 / QC workgroups per CU.
  const int64_t slots = static_cast<int64_t>(device_cus()) * (4 / QC);
  const int64_t grid = a.n_pairs < slots ? a.n_pairs : slots;
  if (grid <= 0) return OW_OK;
  hipLaunchKernelGGL((bigemm_fwd_resident_kernel<Ty, QC>), dim3(static_cast<unsigned>(grid)), dim3(64 * QC), 0,
                     stream, a);
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
