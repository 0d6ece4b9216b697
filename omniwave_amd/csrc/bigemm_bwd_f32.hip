// fp32 backward building blocks: the same steps as bigemm_bwd.hip for fp32 activations, as
// plain one-element-per-thread kernels (fp32 FMAs; no MFMA or vector packing).  The C-ABI
// launchers of bigemm_bwd.hip call these when dtype is OW_DTYPE_F32.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "ow_common.h"
#include "ow_device.h"

namespace ow {
namespace {

constexpr float kLn2f = 0.6931471805599453f;

unsigned grid_for(int64_t n) { return static_cast<unsigned>((n + 255) / 256); }

__device__ __forceinline__ float weight_at(const void* p, int64_t i, int dtype) {
  if (dtype == OW_DTYPE_F32) return static_cast<const float*>(p)[i];
  const uint16_t u = static_cast<const uint16_t*>(p)[i];
  return dtype == OW_DTYPE_BF16 ? BF16::to_f32(u) : F16::to_f32(u);
}

__device__ __forceinline__ int64_t slot_row_f32(const int32_t* tok, int64_t k, int32_t q_s, int32_t n_tok) {
  const int64_t tile = k >> 4;
  const int64_t b = tile / q_s;
  const int32_t s = static_cast<int32_t>(tile - b * q_s);
  const int32_t tk = tok[s * kG + static_cast<int32_t>(k & 15)];
  return (tk >= 0 && tk < n_tok) ? b * n_tok + tk : -1;
}

__global__ void __launch_bounds__(256) gather_f32_kernel(const float* x, const float* dy, const float* rscale,
                                                         const int32_t* tok, const int32_t* chan, float* xt,
                                                         float* dyt, int64_t slots, int32_t n_tok, int32_t channels,
                                                         int32_t q_s, int32_t d, int64_t total) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= total) return;
  const int32_t c = static_cast<int32_t>(i % d);
  const int64_t qk = i / d;
  const int64_t k = qk % slots;
  const int32_t q = static_cast<int32_t>(qk / slots);
  const int64_t row = slot_row_f32(tok, k, q_s, n_tok);
  const int32_t ch = chan[q * d + c];
  float xv = 0.0f, dv = 0.0f;
  if (row >= 0 && ch >= 0 && ch < channels) {
    xv = x[row * channels + ch] * (rscale ? rscale[row] : 1.0f);
    dv = dy[row * channels + ch];
  }
  xt[i] = xv;
  dyt[i] = dv;
}

__global__ void __launch_bounds__(256) gate_f32_kernel(const float* u, const float* v, const float* dz, float* z,
                                                       float* du, float* dv, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  const float up = u[i], vp = v[i], g = dz[i];
  const float s = 1.0f / (1.0f + exp2f(up));
  z[i] = up * vp * s;
  du[i] = g * vp * s * (1.0f - kLn2f * up * (1.0f - s));
  dv[i] = g * up * s;
}

__global__ void __launch_bounds__(256) scatter_f32_kernel(const float* dxt, const int32_t* tok, const int32_t* chan,
                                                          float* g, int64_t slots, int32_t n_tok, int32_t channels,
                                                          int32_t q_s, int32_t d, int64_t total) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= total) return;
  const int32_t c = static_cast<int32_t>(i % d);
  const int64_t qk = i / d;
  const int64_t k = qk % slots;
  const int32_t q = static_cast<int32_t>(qk / slots);
  const int64_t row = slot_row_f32(tok, k, q_s, n_tok);
  const int32_t ch = chan[q * d + c];
  if (row >= 0 && ch >= 0 && ch < channels) g[row * channels + ch] = dxt[i];
}

__global__ void __launch_bounds__(256) rmsnorm_bwd_f32_kernel(const float* x, const float* g, const float* rscale,
                                                              const float* dout, float* dx, int64_t rows,
                                                              int32_t channels, int32_t residual) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float* xr = x + row * channels;
  const float* gr = g + row * channels;
  float r = 1.0f, coef = 0.0f;
  if (rscale) {
    r = rscale[row];
    float dot = 0.0f;
    for (int c = lane; c < channels; c += 64) dot = fmaf(gr[c], xr[c], dot);
    for (int m = 32; m > 0; m >>= 1) dot += __shfl_xor(dot, m);
    coef = dot * r * r * r / static_cast<float>(channels);
  }
  for (int c = lane; c < channels; c += 64) {
    float v = r * gr[c] - coef * xr[c];
    if (residual) v += dout[row * channels + c];
    dx[row * channels + c] = v;
  }
}

struct FoldF32Args {
  const void* b_u;
  const void* b_v;
  const void* b_o;
  const float* norm_w;
  const float* gamma;
  const int32_t* chan;
  float* bu;
  float* buT;
  float* bv;
  float* bvT;
  float* bo;
  float* boT;
  int32_t wdtype, q_c, d, rd, channels;
};

__global__ void __launch_bounds__(256) fold_f32_kernel(FoldF32Args a, int64_t total) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= total) return;
  const int32_t e = static_cast<int32_t>(i % a.rd);
  const int64_t qc = i / a.rd;
  const int32_t c = static_cast<int32_t>(qc % a.d);
  const int32_t q = static_cast<int32_t>(qc / a.d);
  const int32_t ch = a.chan[q * a.d + c];
  const bool ok = ch >= 0 && ch < a.channels;
  const float w = ok ? (a.norm_w ? a.norm_w[ch] : 1.0f) : 0.0f;
  const float gm = ok ? (a.gamma ? a.gamma[ch] : 1.0f) : 0.0f;
  const int64_t cd = (static_cast<int64_t>(q) * a.d + c) * a.rd + e;
  const int64_t ec = (static_cast<int64_t>(q) * a.rd + e) * a.d + c;
  const float u = weight_at(a.b_u, cd, a.wdtype) * w * kNegLog2e;
  const float v = weight_at(a.b_v, cd, a.wdtype) * w * kNegLn2;
  const float o = weight_at(a.b_o, ec, a.wdtype) * gm;
  a.bu[cd] = u;
  a.buT[ec] = u;
  a.bv[cd] = v;
  a.bvT[ec] = v;
  a.bo[ec] = o;
  a.boT[cd] = o;
}

// out[t][i][c] = sum_j M1[i][j] in1[t][j][c] (+ M2[i][j] in2[t][j][c]).
__global__ void __launch_bounds__(256) tile_mix_f32_kernel(const float* in1, const float* m1, const float* in2,
                                                           const float* m2, float* out, int64_t total, int32_t d) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= total) return;
  const int32_t c = static_cast<int32_t>(idx % d);
  const int32_t i = static_cast<int32_t>((idx / d) % kG);
  const int64_t base = (idx / (static_cast<int64_t>(kG) * d)) * kG * d + c;
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < kG; ++j) acc = fmaf(m1[i * kG + j], in1[base + static_cast<int64_t>(j) * d], acc);
  if (in2) {
#pragma unroll
    for (int j = 0; j < kG; ++j) acc = fmaf(m2[i * kG + j], in2[base + static_cast<int64_t>(j) * d], acc);
  }
  out[idx] = acc;
}

// partial[i][j][w] = sum over tiles t = w, w + n_waves, ... of sum_c in1[t][i][c] in2[t][j][c];
// lane l of wave w owns outputs 4l .. 4l + 3.
__global__ void __launch_bounds__(256) tile_outer_f32_kernel(const float* in1, const float* in2, float* partial,
                                                             int64_t n_tiles, int32_t d) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int64_t n_waves = static_cast<int64_t>(gridDim.x) * 4;
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int64_t t = wave; t < n_tiles; t += n_waves) {
    const int64_t base = t * kG * d;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int o = 4 * lane + k, i = o / kG, j = o % kG;
      const float* a = in1 + base + static_cast<int64_t>(i) * d;
      const float* b = in2 + base + static_cast<int64_t>(j) * d;
      float s = 0.0f;
      for (int c = 0; c < d; ++c) s = fmaf(a[c], b[c], s);
      acc[k] += s;
    }
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) partial[(4 * lane + k) * n_waves + wave] = acc[k];
}

}  // namespace

int bwd_gather_f32(const float* x, const float* dy, const float* rscale, const int32_t* tok, const int32_t* chan,
                   float* xt, float* dyt, int64_t slots, int32_t n_tok, int32_t channels, int32_t q_s, int32_t q_c,
                   int32_t d, hipStream_t s) {
  const int64_t total = static_cast<int64_t>(q_c) * slots * d;
  hipLaunchKernelGGL(gather_f32_kernel, dim3(grid_for(total)), dim3(256), 0, s, x, dy, rscale, tok, chan, xt, dyt,
                     slots, n_tok, channels, q_s, d, total);
  return hip_status(hipGetLastError(), "gather_f32_kernel launch");
}

int bwd_gate_f32(const float* u, const float* v, const float* dz, float* z, float* du, float* dv, int64_t n,
                 hipStream_t s) {
  hipLaunchKernelGGL(gate_f32_kernel, dim3(grid_for(n)), dim3(256), 0, s, u, v, dz, z, du, dv, n);
  return hip_status(hipGetLastError(), "gate_f32_kernel launch");
}

int bwd_scatter_f32(const float* dxt, const int32_t* tok, const int32_t* chan, float* g, int64_t slots,
                    int32_t n_tok, int32_t channels, int32_t q_s, int32_t q_c, int32_t d, hipStream_t s) {
  const int64_t total = static_cast<int64_t>(q_c) * slots * d;
  hipLaunchKernelGGL(scatter_f32_kernel, dim3(grid_for(total)), dim3(256), 0, s, dxt, tok, chan, g, slots, n_tok,
                     channels, q_s, d, total);
  return hip_status(hipGetLastError(), "scatter_f32_kernel launch");
}

int bwd_rmsnorm_f32(const float* x, const float* g, const float* rscale, const float* dout, float* dx, int64_t rows,
                    int32_t channels, int32_t residual, hipStream_t s) {
  hipLaunchKernelGGL(rmsnorm_bwd_f32_kernel, dim3(static_cast<unsigned>((rows + 3) / 4)), dim3(256), 0, s, x, g,
                     rscale, dout, dx, rows, channels, residual);
  return hip_status(hipGetLastError(), "rmsnorm_bwd_f32_kernel launch");
}

int fold_weights_f32(const void* b_u, const void* b_v, const void* b_o, int32_t wdtype, const float* norm_w,
                     const float* gamma, const int32_t* chan, int32_t channels, int32_t q_c, int32_t d, int32_t rd,
                     float* bu, float* buT, float* bv, float* bvT, float* bo, float* boT, hipStream_t s) {
  FoldF32Args a{b_u, b_v, b_o, norm_w, gamma, chan, bu, buT, bv, bvT, bo, boT, wdtype, q_c, d, rd, channels};
  const int64_t total = static_cast<int64_t>(q_c) * d * rd;
  hipLaunchKernelGGL(fold_f32_kernel, dim3(grid_for(total)), dim3(256), 0, s, a, total);
  return hip_status(hipGetLastError(), "fold_f32_kernel launch");
}

int tile_mix_f32(const float* in1, const float* m1, const float* in2, const float* m2, float* out, int64_t n_tiles,
                 int32_t d, hipStream_t s) {
  const int64_t total = n_tiles * kG * d;
  hipLaunchKernelGGL(tile_mix_f32_kernel, dim3(grid_for(total)), dim3(256), 0, s, in1, m1, in2, m2, out, total, d);
  return hip_status(hipGetLastError(), "tile_mix_f32_kernel launch");
}

int tile_outer_f32(const float* in1, const float* in2, float* partial, int32_t n_waves, int64_t n_tiles, int32_t d,
                   hipStream_t s) {
  hipLaunchKernelGGL(tile_outer_f32_kernel, dim3(static_cast<unsigned>(n_waves / 4)), dim3(256), 0, s, in1, in2,
                     partial, n_tiles, d);
  return hip_status(hipGetLastError(), "tile_outer_f32_kernel launch");
}

}  // namespace ow
