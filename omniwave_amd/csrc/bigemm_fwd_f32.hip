// fp32 BiGEMM forward: the operator evaluated in fp32 end to end for fp32 activations (the
// reference backend's fp32 semantics, omniweave/ops/reference.py:120-173, with the block's
// RMSNorm prologue and residual epilogue of omniweave/models/block.py:83-108).
//
// One workgroup per tile (image b, token group s, channel group q), 256 threads, fp32 FMAs
// staged through LDS:
//   T = routed [16, d] tile of x (x * r with the RMSNorm, pads 0)
//   P_u = A_u T, P_v = A_v T                     [16, d]
//   Z   = SiLU(P_u B_u') * (P_v B_v')            [16, rd]   (B_u' = w B_u, B_v' = w B_v)
//   W   = Z B_o'                                 [16, d]    (B_o' = B_o diag(gamma))
//   out = (x +) A_o W at the valid routed positions.
// Packed operand layout (fp32, same byte count as the 16-bit layouts' element count x 4):
//   [0, 768): A_u, A_v, A_o row-major [16][16];   [768, 1536): unused;
//   then per channel group q: B_u' [d][rd], B_v' [d][rd], B_o' [rd][d].
#include <hip/hip_runtime.h>

#include <cstdint>

#include "ow_common.h"
#include "ow_device.h"

namespace ow {
namespace {

constexpr int kF32Threads = 256;

__device__ __forceinline__ float load_weight(const void* p, int64_t i, int dtype) {
  if (dtype == OW_DTYPE_F32) return static_cast<const float*>(p)[i];
  const uint16_t u = static_cast<const uint16_t*>(p)[i];
  return dtype == OW_DTYPE_BF16 ? BF16::to_f32(u) : F16::to_f32(u);
}

struct PackF32Args {
  const void* a_u;
  const void* a_v;
  const void* a_o;
  const void* b_u;
  const void* b_v;
  const void* b_o;
  const float* norm_w;
  const float* gamma;
  const int32_t* chan;
  float* packed;
  int32_t wdtype, q_c, d, rd, channels;
  int64_t total;
};

__global__ void __launch_bounds__(256) pack_f32_kernel(PackF32Args p) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= p.total) return;
  float val = 0.0f;
  if (idx < kHeadElems) {
    if (idx < 3 * kG * kG) {
      const int frag = static_cast<int>(idx / (kG * kG));
      const int e = static_cast<int>(idx % (kG * kG));
      val = load_weight(frag == 0 ? p.a_u : frag == 1 ? p.a_v : p.a_o, e, p.wdtype);
    }
  } else {
    const int64_t mat = static_cast<int64_t>(p.d) * p.rd;
    int64_t rem = idx - kHeadElems;
    const int q = static_cast<int>(rem / (3 * mat));
    rem -= static_cast<int64_t>(q) * 3 * mat;
    const int part = static_cast<int>(rem / mat);
    rem -= static_cast<int64_t>(part) * mat;
    int c;
    if (part < 2) {  // [d][rd]
      c = static_cast<int>(rem / p.rd);
    } else {         // [rd][d]
      c = static_cast<int>(rem % p.d);
    }
    float scale = 1.0f;
    if (p.chan) {
      const int gc = p.chan[q * p.d + c];
      const bool ok = gc >= 0 && gc < p.channels;
      const float* vec = part < 2 ? p.norm_w : p.gamma;
      scale = ok ? (vec ? vec[gc] : 1.0f) : 0.0f;
    }
    const void* src = part == 0 ? p.b_u : part == 1 ? p.b_v : p.b_o;
    val = load_weight(src, static_cast<int64_t>(q) * mat + rem, p.wdtype) * scale;
  }
  p.packed[idx] = val;
}

// One wave per row: scale = 1 / sqrt(mean(x^2) + eps) in fp32.
__global__ void __launch_bounds__(256) rms_rows_f32_kernel(const float* x, float* scale, int64_t rows,
                                                           int32_t channels, float eps) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float* xr = x + row * channels;
  float acc = 0.0f;
  for (int c = lane; c < channels; c += 64) acc = fmaf(xr[c], xr[c], acc);
  for (int m = 32; m > 0; m >>= 1) acc += __shfl_xor(acc, m);
  if (lane == 0) scale[row] = 1.0f / sqrtf(acc / static_cast<float>(channels) + eps);
}

struct F32Args {
  const float* x;
  float* out;
  const float* row_scale;  // NULL: no RMSNorm
  const float* packed;
  const int32_t* tok;
  const int32_t* chan;
  int32_t n_tok, channels, q_s, q_c, d, rd, residual;
  const float* drop_scale;  // [batch] per-image multiplier of delta (drop-path); NULL: none
};

template <int D, int RD>
__global__ void __launch_bounds__(kF32Threads) bigemm_fwd_f32_kernel(F32Args a) {
  __shared__ float s_a[3][kG * kG];
  __shared__ float s_t[kG][D];
  __shared__ float s_pu[kG][D];  // later W
  __shared__ float s_pv[kG][D];
  __shared__ float s_z[kG][RD];
  __shared__ int64_t s_row[kG];
  __shared__ int32_t s_ch[D];
  const int tid = threadIdx.x;
  const int64_t tile = blockIdx.x;
  const int q = static_cast<int>(tile % a.q_c);
  const int64_t bs = tile / a.q_c;
  const int s = static_cast<int>(bs % a.q_s);
  const int64_t b = bs / a.q_s;

  for (int i = tid; i < 3 * kG * kG; i += kF32Threads) s_a[i / (kG * kG)][i % (kG * kG)] = a.packed[i];
  if (tid < kG) {
    const int32_t tk = a.tok[s * kG + tid];
    s_row[tid] = (tk >= 0 && tk < a.n_tok) ? b * a.n_tok + tk : -1;
  }
  for (int c = tid; c < D; c += kF32Threads) {
    const int32_t ch = a.chan[q * D + c];
    s_ch[c] = (ch >= 0 && ch < a.channels) ? ch : -1;
  }
  __syncthreads();
  for (int i = tid; i < kG * D; i += kF32Threads) {
    const int r = i / D, c = i % D;
    const int64_t row = s_row[r];
    const int32_t ch = s_ch[c];
    float v = 0.0f;
    if (row >= 0 && ch >= 0) {
      v = a.x[row * a.channels + ch];
      if (a.row_scale) v *= a.row_scale[row];
    }
    s_t[r][c] = v;
  }
  __syncthreads();
  // Token side: P_u, P_v.
  for (int i = tid; i < 2 * kG * D; i += kF32Threads) {
    const int which = i / (kG * D);
    const int r = (i / D) % kG, c = i % D;
    const float* am = s_a[which] + r * kG;
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < kG; ++j) acc = fmaf(am[j], s_t[j][c], acc);
    (which ? s_pv : s_pu)[r][c] = acc;
  }
  __syncthreads();
  // Channel side + gate: thread -> column e, rows [r0, r0 + RPT).
  {
    constexpr int kGroups = kF32Threads / RD;  // 1 (rd 256) or 2 (rd 128)
    constexpr int kRpt = kG / kGroups;
    const int e = tid % RD, r0 = (tid / RD) * kRpt;
    const float* bu = a.packed + kHeadElems + static_cast<int64_t>(q) * 3 * D * RD;
    const float* bv = bu + D * RD;
    float u[kRpt], v[kRpt];
#pragma unroll
    for (int r = 0; r < kRpt; ++r) u[r] = v[r] = 0.0f;
    for (int k = 0; k < D; ++k) {
      const float wu = bu[k * RD + e], wv = bv[k * RD + e];
#pragma unroll
      for (int r = 0; r < kRpt; ++r) {
        u[r] = fmaf(s_pu[r0 + r][k], wu, u[r]);
        v[r] = fmaf(s_pv[r0 + r][k], wv, v[r]);
      }
    }
#pragma unroll
    for (int r = 0; r < kRpt; ++r) s_z[r0 + r][e] = u[r] / (1.0f + expf(-u[r])) * v[r];
  }
  __syncthreads();
  // W = Z B_o': thread -> column c, rows [r0, r0 + RPT).
  constexpr int kGroupsD = kF32Threads / D;  // 2 (d 128) or 4 (d 64)
  constexpr int kRptD = kG / kGroupsD;
  const int c = tid % D, r0 = (tid / D) * kRptD;
  {
    const float* bo = a.packed + kHeadElems + static_cast<int64_t>(q) * 3 * D * RD + 2 * D * RD;
    float w[kRptD];
#pragma unroll
    for (int r = 0; r < kRptD; ++r) w[r] = 0.0f;
    for (int e = 0; e < RD; ++e) {
      const float wo = bo[e * D + c];
#pragma unroll
      for (int r = 0; r < kRptD; ++r) w[r] = fmaf(s_z[r0 + r][e], wo, w[r]);
    }
#pragma unroll
    for (int r = 0; r < kRptD; ++r) s_pu[r0 + r][c] = w[r];
  }
  __syncthreads();
  // delta = A_o W, then the residual and the routed store.
  const int32_t ch = s_ch[c];
  if (ch < 0) return;
#pragma unroll
  for (int r = 0; r < kRptD; ++r) {
    const int64_t row = s_row[r0 + r];
    if (row < 0) continue;
    const float* am = s_a[2] + (r0 + r) * kG;
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < kG; ++j) acc = fmaf(am[j], s_pu[j][c], acc);
    const int64_t off = row * a.channels + ch;
    if (a.drop_scale) acc *= a.drop_scale[b];  // block.py:99-107: delta * keep_mask / keep_probability
    a.out[off] = a.residual ? a.x[off] + acc : acc;
  }
}

}  // namespace

int pack_weights_f32(const void* a_u, const void* a_v, const void* a_o, const void* b_u, const void* b_v,
                     const void* b_o, int32_t weight_dtype, const float* norm_weight, const float* gamma,
                     const int32_t* channel_index, int32_t channels, int32_t q_c, int32_t d, int32_t rd,
                     int64_t total, void* packed, hipStream_t stream) {
  PackF32Args p{a_u, a_v, a_o, b_u, b_v, b_o, norm_weight, gamma, channel_index, static_cast<float*>(packed),
                weight_dtype, q_c, d, rd, channels, total};
  hipLaunchKernelGGL(pack_f32_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, stream, p);
  return hip_status(hipGetLastError(), "pack_f32_kernel launch");
}

int rms_scale_f32(const float* x, float* scale, int64_t rows, int32_t channels, float eps, hipStream_t stream) {
  hipLaunchKernelGGL(rms_rows_f32_kernel, dim3(static_cast<unsigned>((rows + 3) / 4)), dim3(256), 0, stream, x, scale,
                     rows, channels, eps);
  return hip_status(hipGetLastError(), "rms_rows_f32_kernel launch");
}

int launch_fwd_f32(const float* x, float* out, const float* row_scale, const float* packed, const int32_t* tok,
                   const int32_t* chan, int32_t batch, int32_t n_tok, int32_t channels, int32_t q_s, int32_t q_c,
                   int32_t d, int32_t rd, int32_t residual, const float* drop_scale, hipStream_t stream) {
  F32Args a{x, out, row_scale, packed, tok, chan, n_tok, channels, q_s, q_c, d, rd, residual, drop_scale};
  const dim3 grid(static_cast<unsigned>(static_cast<int64_t>(batch) * q_s * q_c));
  if (d == 64 && rd == 128)
    hipLaunchKernelGGL((bigemm_fwd_f32_kernel<64, 128>), grid, dim3(kF32Threads), 0, stream, a);
  else if (d == 64 && rd == 256)
    hipLaunchKernelGGL((bigemm_fwd_f32_kernel<64, 256>), grid, dim3(kF32Threads), 0, stream, a);
  else if (d == 128 && rd == 128)
    hipLaunchKernelGGL((bigemm_fwd_f32_kernel<128, 128>), grid, dim3(kF32Threads), 0, stream, a);
  else if (d == 128 && rd == 256)
    hipLaunchKernelGGL((bigemm_fwd_f32_kernel<128, 256>), grid, dim3(kF32Threads), 0, stream, a);
  else
    return fail(OW_ERR_UNSUPPORTED, "unsupported fp32 tile d=%d rd=%d", d, rd);
  return hip_status(hipGetLastError(), "bigemm_fwd_f32_kernel launch");
}

}  // namespace ow
