// BiGEMM backward.  bf16 / fp16 with d = 64: one fused kernel (token side, channel side and
// gate, dX', token-matrix gradients) and the parameter-gradient reduction over its
// fragment-ordered intermediates; with d = 128: two persistent channel kernels, the
// parameter-gradient reductions left to batched GEMMs; fp32 and other shapes: the routing,
// gating and token-mixing kernels here around batched GEMMs the caller runs (hipBLASLt).  The
// RMSNorm backward and the parameter fold-back are shared.
//
// Gradients are taken with respect to the folded weights the forward evaluates (per channel
// group q, token slot k of the flattened (image, token group, row) order, channel c < d,
// expanded row e < rd):
//     X'   = x r                          (r = RMSNorm row scale, 1 without the norm)
//     P_u  = A_u X'_tile,  P_v = A_v X'_tile                      (token mixing per 16-row tile)
//     U'   = P_u B_u'',  V' = P_v B_v''   B_u'' = -log2(e) w B_u, B_v'' = -ln(2) w B_v
//     Z    = U'V' s,  s = 1 / (1 + 2^U')  (= SiLU(U) V, omniweave/ops/reference.py:155-159)
//     W'   = Z B_o'',  B_o'' = B_o diag(gamma)
//     delta = A_o W'_tile                                          (reference.py:162-171)
// Backward for dY = d delta:
//     dW' = A_o^T dY_tile,  dZ = dW' B_o''^T
//     dU' = dZ V' s (1 - ln2 U' (1 - s)),  dV' = dZ U' s
//     dB_u'' = P_u^T dU', dB_v'' = P_v^T dV', dB_o'' = Z^T dW'   (sums over all slots)
//     dP_u = dU' B_u''^T, dP_v = dV' B_v''^T,  dX' = A_u^T dP_u + A_v^T dP_v
//     dx = r g - x r^3 / C sum_c(g x),  g = dX' scattered to NHWC    (bwd_rmsnorm_kernel)
// and the parameter gradients follow from the folded ones (bwd_params_kernel).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "ow_device.h"

namespace ow {
namespace {

constexpr float kLn2 = 0.6931471805599453f;

// s = 1 / (1 + 2^U') with the hardware exp2 and reciprocal (each within about 1 ulp), as in the
// forward's gate (silu_gate); the fp32 kernels divide exactly.
__device__ __forceinline__ float gate_sigmoid(float up) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(up));
}

__device__ __forceinline__ float load_any(const void* p, int64_t i, int dtype) {
  if (dtype == OW_DTYPE_F32) return static_cast<const float*>(p)[i];
  const uint16_t u = static_cast<const uint16_t*>(p)[i];
  return dtype == OW_DTYPE_BF16 ? BF16::to_f32(u) : F16::to_f32(u);
}

// Slot k = (tile, row t) of a channel group -> NHWC row (b * N + token), -1 for pads.
__device__ __forceinline__ int64_t slot_row(const int32_t* tok, int64_t k, int32_t q_s, int32_t n_tok) {
  const int64_t tile = k >> 4;
  const int32_t t = static_cast<int32_t>(k & 15);
  const int64_t b = tile / q_s;
  const int32_t s = static_cast<int32_t>(tile - b * q_s);
  const int32_t tk = tok[s * kG + t];
  return (tk >= 0 && tk < n_tok) ? b * n_tok + tk : -1;
}

struct GatherArgs {
  const uint16_t* x;
  const uint16_t* dy;
  const float* rscale;  // NULL: 1
  const int32_t* tok;
  const int32_t* chan;
  uint16_t* xt;   // [q_c][slots][d]: x * r (pads 0)
  uint16_t* dyt;  // [q_c][slots][d]: dy (pads 0)
  int64_t slots;  // batch * q_s * 16
  int32_t n_tok, channels, q_s, d;
  int32_t vec;    // x, dy 16-byte aligned and C % 8 == 0: runs of 8 channels load as one vector
};

// Channels chan[0..7] are the aligned run c0..c0+7 of one row (one 16-byte access).
__device__ __forceinline__ bool channel_run8(const int32_t* chan, int32_t channels) {
  const int32_t c0 = chan[0];
  bool run = (c0 & 7) == 0 && c0 + 7 < channels;
#pragma unroll
  for (int j = 1; j < 8; ++j) run = run && chan[j] == c0 + j;
  return run;
}

// One thread per (q, slot, 8 channels): 16-byte stores of both tiles.
template <class Ty>
__global__ void __launch_bounds__(256) bwd_gather_kernel(GatherArgs a, int64_t total8) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= total8) return;
  const int32_t d8 = a.d >> 3;
  const int32_t c0 = static_cast<int32_t>(i % d8) * 8;
  const int64_t qk = i / d8;
  const int64_t k = qk % a.slots;
  const int32_t q = static_cast<int32_t>(qk / a.slots);
  const int64_t row = slot_row(a.tok, k, a.q_s, a.n_tok);
  const int32_t* chp = a.chan + q * a.d + c0;
  uint16_t xv[8], dv[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) xv[j] = dv[j] = 0;
  if (row >= 0) {
    const float r = a.rscale ? a.rscale[row] : 1.0f;
    const int64_t base = row * a.channels;
    if (a.vec && channel_run8(chp, a.channels)) {
      const uint4 xr = *reinterpret_cast<const uint4*>(a.x + base + chp[0]);
      const uint4 dr = *reinterpret_cast<const uint4*>(a.dy + base + chp[0]);
      const uint32_t xw[4] = {xr.x, xr.y, xr.z, xr.w}, dw[4] = {dr.x, dr.y, dr.z, dr.w};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        xv[j] = static_cast<uint16_t>(xw[j >> 1] >> (16 * (j & 1)));
        dv[j] = static_cast<uint16_t>(dw[j >> 1] >> (16 * (j & 1)));
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int32_t ch = chp[j];
        if (ch >= 0 && ch < a.channels) {
          xv[j] = a.x[base + ch];
          dv[j] = a.dy[base + ch];
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) xv[j] = Ty::from_f32(Ty::to_f32(xv[j]) * r);
  }
  auto pack = [](const uint16_t* v) {
    return uint4{v[0] | (static_cast<uint32_t>(v[1]) << 16), v[2] | (static_cast<uint32_t>(v[3]) << 16),
                 v[4] | (static_cast<uint32_t>(v[5]) << 16), v[6] | (static_cast<uint32_t>(v[7]) << 16)};
  };
  *reinterpret_cast<uint4*>(a.xt + i * 8) = pack(xv);
  *reinterpret_cast<uint4*>(a.dyt + i * 8) = pack(dv);
}

// Elementwise gate backward over n values (folded operands, see the file comment), 8 values
// per thread with 16-byte accesses (n % 8 == 0, all buffers 16-byte aligned).
template <class Ty>
__global__ void __launch_bounds__(256) bwd_gate_kernel(const uint16_t* u, const uint16_t* v, const uint16_t* dz,
                                                       uint16_t* z, uint16_t* du, uint16_t* dv, int64_t n8) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n8) return;
  const uint4 uu = reinterpret_cast<const uint4*>(u)[i];
  const uint4 vv = reinterpret_cast<const uint4*>(v)[i];
  const uint4 gg = reinterpret_cast<const uint4*>(dz)[i];
  const uint32_t uw[4] = {uu.x, uu.y, uu.z, uu.w}, vw[4] = {vv.x, vv.y, vv.z, vv.w}, gw[4] = {gg.x, gg.y, gg.z, gg.w};
  uint32_t zo[4], uo[4], vo[4];
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    float zf[2], uf[2], vf[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float up = Ty::to_f32(static_cast<uint16_t>(uw[w] >> (16 * h)));
      const float vp = Ty::to_f32(static_cast<uint16_t>(vw[w] >> (16 * h)));
      const float g = Ty::to_f32(static_cast<uint16_t>(gw[w] >> (16 * h)));
      const float s = gate_sigmoid(up);
      zf[h] = up * vp * s;
      uf[h] = g * vp * s * (1.0f - kLn2 * up * (1.0f - s));
      vf[h] = g * up * s;
    }
    zo[w] = Ty::pack2(zf[0], zf[1]);
    uo[w] = Ty::pack2(uf[0], uf[1]);
    vo[w] = Ty::pack2(vf[0], vf[1]);
  }
  reinterpret_cast<uint4*>(z)[i] = uint4{zo[0], zo[1], zo[2], zo[3]};
  reinterpret_cast<uint4*>(du)[i] = uint4{uo[0], uo[1], uo[2], uo[3]};
  reinterpret_cast<uint4*>(dv)[i] = uint4{vo[0], vo[1], vo[2], vo[3]};
}

// dX' slots -> g [rows, C] (activation dtype), 8 channels per thread (every valid (row,
// channel) is written exactly once: the routes are permutations of tokens and channels, so g
// needs no clearing).
__global__ void __launch_bounds__(256) bwd_scatter_kernel(const uint16_t* dxt, const int32_t* tok, const int32_t* chan,
                                                          uint16_t* g, int64_t slots, int32_t n_tok, int32_t channels,
                                                          int32_t q_s, int32_t d, int32_t vec, int64_t total8) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= total8) return;
  const int32_t d8 = d >> 3;
  const int32_t c0 = static_cast<int32_t>(i % d8) * 8;
  const int64_t qk = i / d8;
  const int64_t k = qk % slots;
  const int32_t q = static_cast<int32_t>(qk / slots);
  const int64_t row = slot_row(tok, k, q_s, n_tok);
  if (row < 0) return;
  const uint4 src = *reinterpret_cast<const uint4*>(dxt + i * 8);
  const int32_t* chp = chan + q * d + c0;
  uint16_t* dst = g + row * channels;
  if (vec && channel_run8(chp, channels)) {
    *reinterpret_cast<uint4*>(dst + chp[0]) = src;
  } else {
    const uint32_t sw[4] = {src.x, src.y, src.z, src.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int32_t ch = chp[j];
      if (ch >= 0 && ch < channels) dst[ch] = static_cast<uint16_t>(sw[j >> 1] >> (16 * (j & 1)));
    }
  }
}

// Rows of `lpr` lanes (a power of two <= 64, 64 / lpr rows per wave), 8 channels per lane
// step: dx = (dout) + r g - x r^3 / C sum(g x)   (norm)   or   (dout) + g.  C % 8 == 0 and
// 16-byte aligned x / dout / dx (the caller checks).
template <class Ty>
__global__ void __launch_bounds__(256) bwd_rmsnorm_kernel(const uint16_t* x, const uint16_t* g, const float* rscale,
                                                          const uint16_t* dout, uint16_t* dx, int64_t rows,
                                                          int32_t channels, int32_t residual, int32_t lpr) {
  const int lane = threadIdx.x & 63;
  const int rows_per_wave = 64 / lpr;
  const int64_t row = (static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6)) * rows_per_wave + lane / lpr;
  const int sub = lane % lpr;
  const bool live = row < rows;
  const int64_t base = live ? row * channels : 0;
  const int c8n = channels >> 3;
  auto unpack8 = [](uint4 q, float* f) {
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) f[j] = Ty::to_f32(static_cast<uint16_t>(w[j >> 1] >> (16 * (j & 1))));
  };
  float r = 1.0f, coef = 0.0f;
  if (rscale) {
    r = live ? rscale[row] : 0.0f;
    float dot = 0.0f;
    if (live) {
      for (int c8 = sub; c8 < c8n; c8 += lpr) {
        float xf[8], gf[8];
        unpack8(*reinterpret_cast<const uint4*>(x + base + 8 * c8), xf);
        unpack8(*reinterpret_cast<const uint4*>(g + base + 8 * c8), gf);
#pragma unroll
        for (int j = 0; j < 8; ++j) dot = fmaf(gf[j], xf[j], dot);
      }
    }
    for (int m = lpr >> 1; m > 0; m >>= 1) dot += __shfl_xor(dot, m);
    coef = dot * r * r * r / static_cast<float>(channels);
  }
  if (!live) return;
  for (int c8 = sub; c8 < c8n; c8 += lpr) {
    float xf[8], df[8];
    unpack8(*reinterpret_cast<const uint4*>(x + base + 8 * c8), xf);
    if (residual) {
      unpack8(*reinterpret_cast<const uint4*>(dout + base + 8 * c8), df);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) df[j] = 0.0f;
    }
    float gf[8];
    unpack8(*reinterpret_cast<const uint4*>(g + base + 8 * c8), gf);
    uint32_t o[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float lo = df[2 * w] + r * gf[2 * w] - coef * xf[2 * w];
      const float hi = df[2 * w + 1] + r * gf[2 * w + 1] - coef * xf[2 * w + 1];
      o[w] = Ty::pack2(lo, hi);
    }
    *reinterpret_cast<uint4*>(dx + base + 8 * c8) = uint4{o[0], o[1], o[2], o[3]};
  }
}

// Any C and alignment: one wave per row, one channel per lane step.
template <class Ty>
__global__ void __launch_bounds__(256) bwd_rmsnorm_scalar_kernel(const uint16_t* x, const uint16_t* g, const float* rscale,
                                                                 const uint16_t* dout, uint16_t* dx, int64_t rows,
                                                                 int32_t channels, int32_t residual) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const uint16_t* xr = x + row * channels;
  const uint16_t* gr = g + row * channels;
  float r = 1.0f, coef = 0.0f;
  if (rscale) {
    r = rscale[row];
    float dot = 0.0f;
    for (int c = lane; c < channels; c += 64) dot = fmaf(Ty::to_f32(gr[c]), Ty::to_f32(xr[c]), dot);
    for (int m = 32; m > 0; m >>= 1) dot += __shfl_xor(dot, m);
    coef = dot * r * r * r / static_cast<float>(channels);
  }
  for (int c = lane; c < channels; c += 64) {
    float v = r * Ty::to_f32(gr[c]) - coef * Ty::to_f32(xr[c]);
    if (residual) v += Ty::to_f32(dout[row * channels + c]);
    dx[row * channels + c] = Ty::from_f32(v);
  }
}

struct FoldArgs {
  const void* b_u;
  const void* b_v;
  const void* b_o;
  const float* norm_w;  // NULL: 1
  const float* gamma;   // NULL: 1
  const int32_t* chan;
  uint16_t* bu;   // [q][d][rd]  B_u''
  uint16_t* buT;  // [q][rd][d]  B_u''^T
  uint16_t* bv;
  uint16_t* bvT;
  uint16_t* bo;   // [q][rd][d]  B_o''
  uint16_t* boT;  // [q][d][rd]  B_o''^T
  int32_t wdtype, q_c, d, rd, channels;
};

// One thread per (q, c, e).
template <class Ty>
__global__ void __launch_bounds__(256) fold_weights_kernel(FoldArgs a, int64_t total) {
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
  const int64_t cd = (static_cast<int64_t>(q) * a.d + c) * a.rd + e;  // [q][c][e]
  const int64_t ec = (static_cast<int64_t>(q) * a.rd + e) * a.d + c;  // [q][e][c]
  const uint16_t u = Ty::from_f32(load_any(a.b_u, cd, a.wdtype) * w * kNegLog2e);
  const uint16_t v = Ty::from_f32(load_any(a.b_v, cd, a.wdtype) * w * kNegLn2);
  const uint16_t o = Ty::from_f32(load_any(a.b_o, ec, a.wdtype) * gm);
  a.bu[cd] = u;
  a.buT[ec] = u;
  a.bv[cd] = v;
  a.bvT[ec] = v;
  a.bo[ec] = o;
  a.boT[cd] = o;
}

struct ParamArgs {
  const void* b_u;
  const void* b_v;
  const void* b_o;
  const float* norm_w;  // NULL: no RMSNorm weight (its gradient is not produced)
  const float* gamma;   // NULL: 1
  const int32_t* chan;
  const float* dbu;  // [q][d][rd] dB_u''
  const float* dbv;
  const float* dbo;  // [q][rd][d] dB_o''
  float* g_bu;       // [q][d][rd]
  float* g_bv;
  float* g_bo;       // [q][rd][d]
  float* g_gamma;    // [C]
  float* g_norm_w;   // [C] or NULL
  int32_t wdtype, q_c, d, rd, channels;
};

// The folded gradients mapped back to the parameters.  Blocks [0, n_a): one wave per (q, c):
// dB_u, dB_v and the norm-weight gradient (a sum over the expanded dimension of the [d][rd] rows,
// reduced across the wave).  Blocks [n_a, ..): 16 channels of one group per block, thread t
// taking channel 16 b + t % 16 and every 16th expanded row from t / 16, so that the [rd][d]
// rows of dB_o'' and B_o are read 16 channels at a time: dB_o and the gamma gradient, the 16
// partial sums of a channel added in a fixed order.
constexpr int kParamC = 16;  // channels per dB_o block
__global__ void __launch_bounds__(256) bwd_params_kernel(ParamArgs a, int32_t n_a) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  if (static_cast<int32_t>(blockIdx.x) < n_a) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 4 + wv;
    if (i >= static_cast<int64_t>(a.q_c) * a.d) return;
    const int32_t c = static_cast<int32_t>(i % a.d);
    const int32_t q = static_cast<int32_t>(i / a.d);
    const int32_t ch = a.chan[q * a.d + c];
    const bool ok = ch >= 0 && ch < a.channels;
    const float w = ok ? (a.norm_w ? a.norm_w[ch] : 1.0f) : 0.0f;
    // Every load of the row is issued before the stores (rd <= 4 * 64 here: the loop runs once
    // for rd in {128, 256}).
    const float* __restrict__ dbu = a.dbu;
    const float* __restrict__ dbv = a.dbv;
    float* __restrict__ gbu = a.g_bu;
    float* __restrict__ gbv = a.g_bv;
    float sum_w = 0.0f;
    for (int32_t e0 = 0; e0 < a.rd; e0 += 4 * 64) {
      float du[4], dv[4], bu[4], bv[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int32_t e = e0 + 64 * k + lane;
        const int64_t cd = (static_cast<int64_t>(q) * a.d + c) * a.rd + e;
        const bool in = e < a.rd;
        du[k] = in ? dbu[cd] : 0.0f;
        dv[k] = in ? dbv[cd] : 0.0f;
        bu[k] = in ? load_any(a.b_u, cd, a.wdtype) : 0.0f;
        bv[k] = in ? load_any(a.b_v, cd, a.wdtype) : 0.0f;
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int32_t e = e0 + 64 * k + lane;
        const int64_t cd = (static_cast<int64_t>(q) * a.d + c) * a.rd + e;
        if (e < a.rd) {
          gbu[cd] = du[k] * kNegLog2e * w;
          gbv[cd] = dv[k] * kNegLn2 * w;
        }
        sum_w += du[k] * kNegLog2e * bu[k] + dv[k] * kNegLn2 * bv[k];
      }
    }
    for (int m = 32; m > 0; m >>= 1) sum_w += __shfl_xor(sum_w, m);
    if (ok && lane == 0 && a.g_norm_w) a.g_norm_w[ch] = sum_w;
    return;
  }
  __shared__ float part[256 / kParamC][kParamC];
  const int32_t cblocks = (a.d + kParamC - 1) / kParamC;
  const int32_t b = static_cast<int32_t>(blockIdx.x) - n_a;
  const int32_t q = b / cblocks;
  const int32_t c = (b % cblocks) * kParamC + (threadIdx.x % kParamC);
  const int32_t eg = threadIdx.x / kParamC;  // 0 .. 15
  const bool in = c < a.d;
  const int32_t ch = in ? a.chan[q * a.d + c] : -1;
  const bool ok = ch >= 0 && ch < a.channels;
  const float gm = ok ? (a.gamma ? a.gamma[ch] : 1.0f) : 0.0f;
  const float* __restrict__ dbo = a.dbo;
  float* __restrict__ gbo = a.g_bo;
  float sum_g = 0.0f;
  if (in) {
    constexpr int kBatch = 8;
    for (int32_t e0 = eg; e0 < a.rd; e0 += kBatch * (256 / kParamC)) {
      float dob[kBatch], bo[kBatch];
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        const int32_t e = e0 + k * (256 / kParamC);
        const int64_t ec = (static_cast<int64_t>(q) * a.rd + e) * a.d + c;
        dob[k] = e < a.rd ? dbo[ec] : 0.0f;
        bo[k] = e < a.rd ? load_any(a.b_o, ec, a.wdtype) : 0.0f;
      }
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        const int32_t e = e0 + k * (256 / kParamC);
        if (e < a.rd) gbo[(static_cast<int64_t>(q) * a.rd + e) * a.d + c] = dob[k] * gm;
        sum_g += dob[k] * bo[k];
      }
    }
  }
  part[eg][threadIdx.x % kParamC] = sum_g;
  __syncthreads();
  if (threadIdx.x < kParamC && ok) {
    float v = part[0][threadIdx.x];
#pragma unroll
    for (int k = 1; k < 256 / kParamC; ++k) v += part[k][threadIdx.x];
    a.g_gamma[ch] = v;
  }
}

// The small parameters of the backward (norm weight, gamma, the token matrices) as one fp32
// buffer: source k (dtype[k], off[k + 1] - off[k] values) into dst[off[k] ..].
struct SmallF32Args {
  const void* src[8];
  int32_t dtype[8];
  int64_t off[9];
  int32_t n;
  float* dst;
};
__global__ void __launch_bounds__(256) small_to_f32_kernel(SmallF32Args a) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= a.off[a.n]) return;
  const void* src = a.src[0];
  int32_t dt = a.dtype[0];
  int64_t o = 0;
#pragma unroll
  for (int k = 1; k < 8; ++k)
    if (k < a.n && i >= a.off[k]) {
      src = a.src[k];
      dt = a.dtype[k];
      o = a.off[k];
    }
  a.dst[i] = load_any(src, i - o, dt);
}

// Token mixing per 16-row tile: out = M1 in1 (+ M2 in2), M* [16][16] fp32, in/out tiles
// [16][NB*16] of the compute dtype.  One wave per tile, 16x16x16 MFMAs: A operand lane (l16, h)
// slot j = M[l16][4h + j], B operand = in[4h + j][16 cb + l16].  All loads are issued before
// the MFMAs and all stores after one drain.
template <class Ty, bool TWO, int NB>
__global__ void __launch_bounds__(256) tile_mix_kernel(const uint16_t* in1, const float* m1, const uint16_t* in2,
                                                       const float* m2, uint16_t* out, int64_t n_tiles) {
  constexpr int D = NB * 16;
  const int lane = threadIdx.x & 63;
  const int64_t tile = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (tile >= n_tiles) return;
  const int l16 = lane & 15, h = lane >> 4;
  auto a_op = [&](const float* m) {
    return u32x2{Ty::pack2(m[l16 * 16 + 4 * h + 0], m[l16 * 16 + 4 * h + 1]),
                 Ty::pack2(m[l16 * 16 + 4 * h + 2], m[l16 * 16 + 4 * h + 3])};
  };
  const int64_t base = tile * 16 * D + (4 * h) * D + l16;
  uint16_t e1[NB][4], e2[NB][4];
#pragma unroll
  for (int cb = 0; cb < NB; ++cb) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      e1[cb][j] = in1[base + j * D + 16 * cb];
      if constexpr (TWO) e2[cb][j] = in2[base + j * D + 16 * cb];
    }
  }
  const u32x2 a1 = a_op(m1);
  u32x2 a2 = {0u, 0u};
  if constexpr (TWO) a2 = a_op(m2);
  const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  auto b_op = [](const uint16_t* e) {
    return u32x2{e[0] | (static_cast<uint32_t>(e[1]) << 16), e[2] | (static_cast<uint32_t>(e[3]) << 16)};
  };
  f32x4 acc[NB];
#pragma unroll
  for (int cb = 0; cb < NB; ++cb) {
    acc[cb] = Ty::mma16(a1, b_op(e1[cb]), zero);
    if constexpr (TWO) acc[cb] = Ty::mma16(a2, b_op(e2[cb]), acc[cb]);
  }
  mfma_drain();
#pragma unroll
  for (int cb = 0; cb < NB; ++cb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) out[base + i * D + 16 * cb] = Ty::from_f32(acc[cb][i]);
  }
}

// Sum over tiles of in1_tile in2_tile^T ([16][d] x [d][16] -> [16][16]), grid-strided; each wave
// writes its partial sum (lane (l16, h) register i = out[4h + i][l16]) to partial[256][n_waves]
// (element-major, so the sum over waves is a contiguous reduction).  With d % 32 == 0 the K
// order inside each pair of 16-deep steps is lane-major: lane (l16, h) holds channels
// 32 s + 8 h .. + 8 of row l16 (one 16-byte load per operand), the first MFMA of the pair takes
// elements 0..3 and the second 4..7 — both operands use the same order, so the sum is the full
// contraction — and two tiles are loaded before their MFMAs, so each wave keeps 4 d / 32 loads
// in flight.
template <class Ty>
__global__ void __launch_bounds__(256) tile_outer_kernel(const uint16_t* in1, const uint16_t* in2, float* partial,
                                                         int64_t n_tiles, int32_t d, int32_t vec) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int64_t n_waves = static_cast<int64_t>(gridDim.x) * 4;
  const int l16 = lane & 15, h = lane >> 4;
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  auto tile_pair = [&](auto nk_tag) {
    constexpr int NK = decltype(nk_tag)::value;  // 16-byte loads per row and operand (d / 32)
    constexpr int D = 32 * NK;
    auto mma_pair = [&](const u32x4& a, const u32x4& b) {
      acc = Ty::mma16(u32x2{a.x, a.y}, u32x2{b.x, b.y}, acc);
      acc = Ty::mma16(u32x2{a.z, a.w}, u32x2{b.z, b.w}, acc);
    };
    int64_t tile = wave;
    for (; tile + n_waves < n_tiles; tile += 2 * n_waves) {
      const uint16_t* p0 = in1 + tile * 16 * D + l16 * D + 8 * h;
      const uint16_t* q0 = in2 + tile * 16 * D + l16 * D + 8 * h;
      const int64_t step = n_waves * 16 * D;
      u32x4 a0[NK], b0[NK], a1[NK], b1[NK];
#pragma unroll
      for (int s = 0; s < NK; ++s) {
        a0[s] = *reinterpret_cast<const u32x4*>(p0 + 32 * s);
        b0[s] = *reinterpret_cast<const u32x4*>(q0 + 32 * s);
        a1[s] = *reinterpret_cast<const u32x4*>(p0 + step + 32 * s);
        b1[s] = *reinterpret_cast<const u32x4*>(q0 + step + 32 * s);
      }
#pragma unroll
      for (int s = 0; s < NK; ++s) mma_pair(a0[s], b0[s]);
#pragma unroll
      for (int s = 0; s < NK; ++s) mma_pair(a1[s], b1[s]);
    }
    if (tile < n_tiles) {
      const uint16_t* p0 = in1 + tile * 16 * D + l16 * D + 8 * h;
      const uint16_t* q0 = in2 + tile * 16 * D + l16 * D + 8 * h;
      u32x4 a0[NK], b0[NK];
#pragma unroll
      for (int s = 0; s < NK; ++s) {
        a0[s] = *reinterpret_cast<const u32x4*>(p0 + 32 * s);
        b0[s] = *reinterpret_cast<const u32x4*>(q0 + 32 * s);
      }
#pragma unroll
      for (int s = 0; s < NK; ++s) mma_pair(a0[s], b0[s]);
    }
  };
  if (vec && d == 64) {
    tile_pair(std::integral_constant<int, 2>{});
  } else if (vec && d == 128) {
    tile_pair(std::integral_constant<int, 4>{});
  } else {
    for (int64_t tile = wave; tile < n_tiles; tile += n_waves) {
      const int64_t base = tile * 16 * d;
      for (int ks = 0; ks < d / 16; ++ks) {
        // A: row l16 of in1, K slots 16 ks + 4h + j; B: column l16 = row l16 of in2, same K.
        const uint2 av = *reinterpret_cast<const uint2*>(in1 + base + l16 * d + 16 * ks + 4 * h);
        const uint2 bv = *reinterpret_cast<const uint2*>(in2 + base + l16 * d + 16 * ks + 4 * h);
        acc = Ty::mma16(u32x2{av.x, av.y}, u32x2{bv.x, bv.y}, acc);
      }
    }
  }
  mfma_drain();
#pragma unroll
  for (int i = 0; i < 4; ++i) partial[((4 * h + i) * 16 + l16) * n_waves + wave] = acc[i];
}

// ---- Fused channel side of the backward -----------------------------------------------
// Packed backward weights, per (group q, 32-row chunk ec of the expanded dimension), 3 KS + 6 MB
// fragments of 64 lanes x 8 (KS = d / 16, MB = d / 32; the 32x32x16 operand layouts of the
// forward; kord(j, hh) = 8(j/4) + 4hh + j%4):
//   [0, KS)          B_u''^T  A operand: lane -> row e = 32 ec + l32, slot j -> channel 16 ks + kord
//   [KS, 2 KS)       B_v''^T  A operand (same)
//   [2 KS, 3 KS)     B_o''    A operand: lane -> row e, slot j -> channel 16 ks + kord
//   then 2 MB each:  B_o''    B operand (mb, s): lane -> channel 32 mb + l32, slot j -> e = 32 ec + 16 s + kord
//                    B_u''^T  B operand (mb, s): lane -> channel, slot j -> e (same order)
//                    B_v''^T  B operand (mb, s)
// (d = 64: 24 fragments per chunk; d = 128: 48, the first 24 of which the d = 128 channel kernel reads.)
constexpr int kBwdD = 64;
constexpr int kBwdKS = kBwdD / 16;
constexpr int kBwdMB = kBwdD / 32;
constexpr int kBwdFr = 3 * kBwdKS + 6 * kBwdMB;  // 24 fragments per chunk
__host__ __device__ constexpr int bwd_frags(int d) { return 3 * (d / 16) + 6 * (d / 32); }

struct BwdPackArgs {
  const void* b_u;
  const void* b_v;
  const void* b_o;
  const float* norm_w;  // NULL: 1
  const float* gamma;   // NULL: 1
  const int32_t* chan;
  uint16_t* packed;
  int32_t wdtype, q_c, rd, channels;
  int64_t total;
  int32_t d;
};

template <class Ty>
__global__ void __launch_bounds__(256) pack_bwd_kernel(BwdPackArgs p) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= p.total) return;
  const int nch = p.rd / 32;
  const int ks_n = p.d / 16, mb_n = p.d / 32;
  const int64_t per_chunk = static_cast<int64_t>(bwd_frags(p.d)) * kFragElems;
  const int q = static_cast<int>(idx / (nch * per_chunk));
  int64_t rem = idx - static_cast<int64_t>(q) * nch * per_chunk;
  const int ec = static_cast<int>(rem / per_chunk);
  rem -= static_cast<int64_t>(ec) * per_chunk;
  const int fr = static_cast<int>(rem / kFragElems);
  const int e8 = static_cast<int>(rem % kFragElems);
  const int lane = e8 / 8, j = e8 % 8;
  const int l32 = lane & 31, hh = lane >> 5;
  const int kord = 8 * (j / 4) + 4 * hh + (j % 4);
  int c, e, mat;  // mat: 0 = B_u, 1 = B_v, 2 = B_o
  if (fr < 3 * ks_n) {
    mat = fr / ks_n;
    e = 32 * ec + l32;
    c = 16 * (fr % ks_n) + kord;
  } else {
    const int f = fr - 3 * ks_n;
    const int m = f / (2 * mb_n);  // 0: B_o, 1: B_u, 2: B_v
    mat = m == 0 ? 2 : m - 1;
    const int mb = (f % (2 * mb_n)) / 2, sh = f % 2;
    c = 32 * mb + l32;
    e = 32 * ec + 16 * sh + kord;
  }
  const int32_t ch = p.chan[q * p.d + c];
  const bool ok = ch >= 0 && ch < p.channels;
  float val;
  if (mat == 2) {
    const float gm = ok ? (p.gamma ? p.gamma[ch] : 1.0f) : 0.0f;
    val = load_any(p.b_o, (static_cast<int64_t>(q) * p.rd + e) * p.d + c, p.wdtype) * gm;
  } else {
    const float w = ok ? (p.norm_w ? p.norm_w[ch] : 1.0f) : 0.0f;
    val = load_any(mat == 0 ? p.b_u : p.b_v, (static_cast<int64_t>(q) * p.d + c) * p.rd + e, p.wdtype) * w *
          (mat == 0 ? kNegLog2e : kNegLn2);
  }
  p.packed[idx] = Ty::from_f32(val);
}

__device__ __forceinline__ void bwd_copy_frag(const uint16_t* src, uint16_t* dst, int lane) {
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(src + lane * 8),
                                   (__attribute__((address_space(3))) void*)(dst), 16, 0, 0);
}

// ---- Fused backward, d = 64: token side + channel side + token-side gradients ------------
// One workgroup = 4 waves; per round, 4 consecutive 32-slot pairs of one channel group (one
// per wave), rounds grid-strided.  Per pair and wave:
//   * P_u^T = X'^T (A_u)^T, P_v^T, dW'^T = dY^T A_o (block-diagonal 32x32x16 products over the
//     pair, as in the forward) from the X' and dY tiles staged in the second weight buffer,
//     which no copy targets before the first barrier of the chunk loop; P_u, P_v, dW' are also
//     stored (straight from the operand registers, rows in the pair-operand channel order) for
//     the parameter-gradient reduction, which recomputes the gate from them;
//   * the channel loop (U'^T, V'^T, dZ^T per 32-row chunk, gate, W' += Z B_o'',
//     dP_u += dU' B_u''^T, dP_v += dV' B_v''^T);
//   * dX' = A_u^T dP_u + A_v^T dP_v (block-diagonal, the forward's output product), stored;
//   * dA_u += dP_u X'^T, dA_v += dP_v X'^T, dA_o += dY W'^T per 16-slot tile with 16x16x16
//     products over the channels (dP_u, dP_v, W' as rows through a per-wave LDS tile, X' and
//     dY rows from memory), accumulated over all rounds of the wave.
// At the end the four waves' dA sums are added in a fixed order and the workgroup writes
// partial[blockIdx][3][256] (dA_u, dA_v, dA_o, element 16 t + k).
constexpr int64_t kBwdFusedGrid = 1024;  // at most 2 workgroups per CU x 2 rounds in flight

struct BwdFusedArgs {
  const uint16_t* xt;   // [q_c][slots][64] X' tiles
  const uint16_t* dyt;  // [q_c][slots][64] dY tiles
  const float* a_u;     // [16][16] token matrices, fp32
  const float* a_v;
  const float* a_o;
  const uint16_t* packed;  // ow_pack_bwd_weights
  uint16_t* pu;            // [q_c][slots][64] outputs for the parameter-gradient reduction, rows
  uint16_t* pv;            // in the pair-operand channel order (bwd_param_reduce64_kernel)
  uint16_t* dw;
  uint16_t* dxt;   // [q_c][slots][64]
  float* partial;  // [gridDim][3][256]
  int64_t slots;
  int64_t pairs_per_q;  // slots / 32
  int64_t rounds;       // q_c * ceil(pairs_per_q / 4)
  int32_t q_c;
  // Routed mode (identity channel order, C = q_c * 64): X' and dY rows are read from x, dy
  // ([rows][C]) through the token table and dX' is written to g ([rows][C]) the same way;
  // xt, dyt, dxt are unused.
  const uint16_t* x;
  const uint16_t* dy;
  const float* rscale;  // NULL: 1
  const int32_t* tok;   // [q_s * 16]
  uint16_t* g;
  int32_t batch, n_tok, q_s, channels;
};

// 8 / 4 values of the compute dtype times r, rounded (x r of the gather).
template <class Ty>
__device__ __forceinline__ uint32_t scale2(uint32_t v, float r) {
  return Ty::pack2(Ty::to_f32(static_cast<uint16_t>(v & 0xffffu)) * r, Ty::to_f32(static_cast<uint16_t>(v >> 16)) * r);
}

// Token-operand fragment of a 16x16 token matrix (lane (t, hh) slot j = M[t % 16][kord(j, hh)],
// or the transpose with T), rounded to Ty.
template <class Ty, bool T>
__device__ __forceinline__ u32x4 token_frag(const float* m, int lane) {
  const int t = lane & 15, hh = lane >> 5;
  u32x4 v;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int k0 = 8 * (q >> 1) + 4 * hh + 2 * (q & 1);
    const float lo = T ? m[k0 * 16 + t] : m[t * 16 + k0];
    const float hi = T ? m[(k0 + 1) * 16 + t] : m[t * 16 + k0 + 1];
    v[q] = Ty::pack2(lo, hi);
  }
  return v;
}

// RES (rd = 128): the resident-weights organisation.  One workgroup of 8 waves per CU holds its
// channel group's packed weights (4 chunks, 96 KB) in LDS for the whole launch: workgroup b
// takes group b % q_c, and its waves take the group's pairs w, w + 8 R, .. (R = gridDim.x /
// q_c workgroups per group) independently, with no barrier and no weight copy after the start
// (the forward wave kernel's scheme); the dA sums stay in registers until the end.  Otherwise
// (rd = 256, whose 192 KB of weights do not fit): 4 waves per workgroup, rounds of 4 pairs, the
// chunks streamed through two LDS buffers with a barrier per chunk, as described above.
constexpr int kBwdResWaves = 8;

template <class Ty, int RD, bool RT, bool RES>
__global__ void __attribute__((amdgpu_flat_work_group_size(RES ? 512 : 256, RES ? 512 : 256), amdgpu_waves_per_eu(2, 2)))
bwd_fused_d64_kernel(BwdFusedArgs a) {
  constexpr int NCH = RD / 32;
  constexpr int CH_ELEMS = kBwdFr * kFragElems;
  constexpr int kLd = kBwdD + 8;  // staged tile row stride (elements): conflict-free columns
  constexpr int NW = RES ? kBwdResWaves : 4;
  static_assert(!RES || RD == 128, "resident weights: rd = 128");
  static_assert(RES || 4 * 32 * kLd <= CH_ELEMS, "a tile per wave fits in one weight buffer");
  static_assert(!RES || NW * 3 * 256 * 4 <= NW * 32 * kLd * 2, "the final dA sums fit in the tiles");
  // RES: the group's NCH chunks; else two chunk buffers.
  __shared__ __attribute__((aligned(16))) uint16_t wb[RES ? NCH : 2][CH_ELEMS];
  __shared__ __attribute__((aligned(16))) uint16_t tiles[RES ? NW : 1][32 * kLd];  // RES: per wave
  __shared__ __attribute__((aligned(16))) u32x4 tok[5][64];  // A_u, A_v, A_o^T, A_u^T, A_v^T operand rows
  __shared__ float red[RES ? 1 : 4][3][256];
  // wave is uniform: readfirstlane keeps it and the pair, slot and tile positions derived from it in
  // scalar registers.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int hh = lane >> 5, l32 = lane & 31, l16 = lane & 15, h4 = lane >> 4;
  const bool g0 = (lane & 16) == 0;
  const int64_t wg_per_q = (a.pairs_per_q + 3) / 4;  // rounds per group (not RES)

  if (wave == 0) {
    tok[0][lane] = token_frag<Ty, false>(a.a_u, lane);
    tok[1][lane] = token_frag<Ty, false>(a.a_v, lane);
    tok[2][lane] = token_frag<Ty, true>(a.a_o, lane);
  } else if (wave == 1) {
    tok[3][lane] = token_frag<Ty, true>(a.a_u, lane);
    tok[4][lane] = token_frag<Ty, true>(a.a_v, lane);
  }
  // Not RES: red[wave] holds the wave's running dA sums (lane (l16, h4) element (4 h4 + i) * 16 +
  // l16), in LDS rather than registers across the channel loop.  RES: registers.
  f32x4 dA_run[3] = {};
  if constexpr (!RES) {
#pragma unroll
    for (int m = 0; m < 3; ++m)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[wave][m][(4 * h4 + i) * 16 + l16] = 0.0f;
  }

  // Routed: the token-table entry of slot l32 of a pair (its first tile 2 pair = b q_s + s; the
  // load only, so that the next pair's is in flight during this one) and the NHWC row it gives
  // (-1 for pads and waves past the end).
  struct PairTok {
    int32_t b, tk;
    bool live;
  };
  auto pair_tok = [&](int64_t pair, bool live) {
    PairTok t{0, -1, live};
    if constexpr (RT) {
      const uint32_t tile0 = static_cast<uint32_t>(2 * (live ? pair : 0));
      int32_t b = static_cast<int32_t>(tile0 / static_cast<uint32_t>(a.q_s));
      int32_t st = static_cast<int32_t>(tile0 - static_cast<uint32_t>(b) * static_cast<uint32_t>(a.q_s)) + (l32 >> 4);
      if (st == a.q_s) {
        st = 0;
        ++b;
      }
      t.b = b;
      t.tk = a.tok[st * kG + (l32 & 15)];
    }
    return t;
  };
  auto tok_row = [&](const PairTok& t) -> int32_t {  // < 2^31: host check
    return (t.live && t.b < a.batch && t.tk >= 0 && t.tk < a.n_tok) ? t.b * a.n_tok + t.tk : -1;
  };
  const uint32_t nbytes_rows = static_cast<uint32_t>(static_cast<int64_t>(a.batch) * a.n_tok * a.channels * 2);
  const uint32_t tile_bytes = static_cast<uint32_t>(a.q_c * a.slots * kBwdD * 2);
  const __amdgpu_buffer_rsrc_t rrs =
      buffer_rsrc(a.rscale, a.rscale ? static_cast<uint32_t>(static_cast<int64_t>(a.batch) * a.n_tok * 4) : 0u);

  // One pair of group q (32 slots from slot0): token side, channel loop, dX', dA.  tx: the wave's
  // tile [32][kLd] for X, dY and the dA rows; next: the token-table entry of the wave's next pair;
  // chunk_begin(ec) / chunk_frag(ec): the chunk loop's synchronisation and chunk ec's fragments.
  auto do_pair = [&](int q, int64_t pair, bool live, PairTok& cur_tok, const PairTok& next_tok, uint16_t* tx,
                     uint16_t* stage, auto chunk_begin, auto chunk_frags) {
    const int64_t slot0 = static_cast<int64_t>(q) * a.slots + (live ? pair : 0) * 32;
    const int64_t cbase = static_cast<int64_t>(q) * kBwdD;  // routed: first channel of group q
    auto row_off = [&](int64_t nr, int64_t c) {
      return nr >= 0 ? static_cast<uint32_t>((nr * a.channels + cbase + c) * 2) : kOffOut;
    };
    // Routed: the NHWC row of this lane's slot l32 (lanes l32 and l32 + 32 alike) and its RMSNorm
    // scale, looked up once per pair; every other use takes slot r's from lane r (__shfl).
    int32_t my_row = -1;
    float my_rs = 1.0f;
    if constexpr (RT) {
      my_row = tok_row(cur_tok);
      if (a.rscale)
        my_rs = __uint_as_float(
            __builtin_amdgcn_raw_buffer_load_b32(rrs, my_row >= 0 ? static_cast<uint32_t>(my_row) * 4u : kOffOut, 0, 0));
    }
    auto row_of = [&](int r) { return __shfl(my_row, r); };
    // A tile's rows (lane: row (lane + 64 k) / 8, channels 8 ((lane + 64 k) % 8) ..), every load
    // issued before any is waited on; pads and rows past the end read as zero.
    auto load_rows = [&](const uint16_t* src, u32x4 (&val)[4]) {
      if constexpr (RT) {
        const __amdgpu_buffer_rsrc_t rsrc = buffer_rsrc(src, nbytes_rows);
#pragma unroll
        for (int k = 0; k < 4; ++k)
          val[k] = __builtin_amdgcn_raw_buffer_load_b128(
              rsrc, row_off(row_of((lane + 64 * k) >> 3), ((lane + 64 * k) & 7) * 8), 0, 0);
      } else {
        // The gathered tiles (below 2 GiB: host check), through 32-bit buffer offsets.
        const __amdgpu_buffer_rsrc_t rsrc = buffer_rsrc(src, tile_bytes);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int v = lane + 64 * k, r = v >> 3, c8 = (v & 7) * 8;
          val[k] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, static_cast<uint32_t>(((slot0 + r) * kBwdD + c8) * 2), 0, 0);
        }
      }
    };
    // The rows into the wave's tile [32][kLd]; routed X rows times their RMSNorm scales (X').
    auto write_tile = [&](u32x4 (&val)[4], bool scale) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int v = lane + 64 * k, r = v >> 3, c8 = (v & 7) * 8;
        if (RT && scale && a.rscale) {
          const float rs = __shfl(my_rs, r);
#pragma unroll
          for (int w = 0; w < 4; ++w) val[k][w] = scale2<Ty>(val[k][w], rs);
        }
        *reinterpret_cast<u32x4*>(tx + r * kLd + c8) = val[k];
      }
      wave_lds_sync();
    };
    auto token_side = [&](u32x4 f, u32x4 (&out)[kBwdKS]) {
      const u32x4 f0 = keep_if(g0, f), f1 = keep_if(!g0, f);
      const f32x16 zero = {};
#pragma unroll
      for (int cb = 0; cb < kBwdMB; ++cb) {
        const u32x4 x0 = column8(tx + (4 * hh) * kLd + 32 * cb + l32, kLd);
        const u32x4 x1 = column8(tx + (16 + 4 * hh) * kLd + 32 * cb + l32, kLd);
        f32x16 acc = Ty::mma32(x0, f0, zero);
        acc = Ty::mma32(x1, f1, acc);
#pragma unroll
        for (int s = 0; s < 2; ++s) out[2 * cb + s] = pack_kstep<Ty>(acc, s);
      }
    };
    u32x4 Pu[kBwdKS], Pv[kBwdKS], Dw[kBwdKS];
    {
      // X and dY rows requested together; dY's land while X's token side runs.
      u32x4 vx[4], vy[4];
      load_rows(RT ? a.x : a.xt, vx);
      load_rows(RT ? a.dy : a.dyt, vy);
      cur_tok = next_tok;  // the next pair's entry (requested by the caller), used at its start
      write_tile(vx, true);
      token_side(tok[0][lane], Pu);
      token_side(tok[1][lane], Pv);
      wave_lds_sync();
      write_tile(vy, false);
      token_side(tok[2][lane], Dw);
    }
    const f32x16 zero = {};
    const int64_t row = slot0 + l32;  // this lane's slot
    if (live) {
      // P_u, P_v, dW' rows: lane (slot l32, hh) holds K-step ks = channels 16 ks + kord(j, hh),
      // stored as the 16-byte piece at element 16 ks + 8 hh of the slot's row (the pair-operand
      // channel order).  Non-temporal: at a 56x56x128 batch of 128 they are 0.3 GB, read once by
      // the reduction after this pass.
#pragma unroll
      for (int t = 0; t < 3; ++t) {
        const u32x4(&pk)[kBwdKS] = t == 0 ? Pu : t == 1 ? Pv : Dw;
        uint16_t* dst = (t == 0 ? a.pu : t == 1 ? a.pv : a.dw) + row * kBwdD + 8 * hh;
#pragma unroll
        for (int ks = 0; ks < kBwdKS; ++ks) __builtin_nontemporal_store(pk[ks], reinterpret_cast<u32x4*>(dst + 16 * ks));
      }
    }

    // Channel side.
    f32x16 W[kBwdMB] = {}, DPu[kBwdMB] = {}, DPv[kBwdMB] = {};
    for (int ec = 0; ec < NCH; ++ec) {
      chunk_begin(ec);
      const u32x4* cf = chunk_frags(ec);
      auto frag = [&](int f) { return cf[f * (kFragElems / 8) + lane]; };
      f32x16 U = {}, V = {}, G = {};
#pragma unroll
      for (int ks = 0; ks < kBwdKS; ++ks) {
        U = Ty::mma32(frag(ks), Pu[ks], U);
        V = Ty::mma32(frag(kBwdKS + ks), Pv[ks], V);
        G = Ty::mma32(frag(2 * kBwdKS + ks), Dw[ks], G);
      }
      mfma_drain();
      f32x16 Z, DU, DV;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float up = U[i], vp = V[i], g = G[i];
        const float s = gate_sigmoid(up);
        Z[i] = up * vp * s;
        DU[i] = g * vp * s * (1.0f - kLn2 * up * (1.0f - s));
        DV[i] = g * up * s;
      }
      u32x4 zs[2], dus[2], dvs[2];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        zs[s] = pack_kstep<Ty>(Z, s);
        dus[s] = pack_kstep<Ty>(DU, s);
        dvs[s] = pack_kstep<Ty>(DV, s);
      }
#pragma unroll
      for (int mb = 0; mb < kBwdMB; ++mb)
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          W[mb] = Ty::mma32(zs[s], frag(3 * kBwdKS + 2 * mb + s), W[mb]);
          DPu[mb] = Ty::mma32(dus[s], frag(3 * kBwdKS + 2 * kBwdMB + 2 * mb + s), DPu[mb]);
          DPv[mb] = Ty::mma32(dvs[s], frag(3 * kBwdKS + 4 * kBwdMB + 2 * mb + s), DPv[mb]);
        }
    }
    mfma_drain();

    // The rows of the dA products, requested before the dX' products so that they land
    // meanwhile: rows 16 g + l16 of X (routed: x, scaled at use) and of dY, channels
    // 16 ks + 4 h4 .. + 3 (waves past the end read pads or their group's first rows, unused).
    int64_t orow[2];
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      if constexpr (RT)
        orow[g] = row_of(16 * g + l16);
      else
        orow[g] = slot0 + 16 * g + l16;
    }
    auto other_rows = [&](const uint16_t* tiles_src, const uint16_t* rows, int g, int ks) -> u32x2 {
      if constexpr (RT) {
        return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(
                                             buffer_rsrc(rows, nbytes_rows), row_off(orow[g], 16 * ks + 4 * h4), 0, 0));
      } else {
        return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(
                                             buffer_rsrc(tiles_src, tile_bytes),
                                             static_cast<uint32_t>((orow[g] * kBwdD + 16 * ks + 4 * h4) * 2), 0, 0));
      }
    };
    u32x2 xo[2][kBwdKS], yo[2][kBwdKS];
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int ks = 0; ks < kBwdKS; ++ks) xo[g][ks] = other_rows(a.xt, a.x, g, ks);
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int ks = 0; ks < kBwdKS; ++ks) yo[g][ks] = other_rows(a.dyt, a.dy, g, ks);

    // dX' = A_u^T dP_u + A_v^T dP_v (lane = channel 32 mb + l32, register i = slot
    // pair_token_row(i, hh)).
    f32x16 DX[kBwdMB];
    {
      const u32x4 tu = tok[3][lane], tv = tok[4][lane];
      const u32x4 tu0 = keep_if(g0, tu), tu1 = keep_if(!g0, tu);
      const u32x4 tv0 = keep_if(g0, tv), tv1 = keep_if(!g0, tv);
#pragma unroll
      for (int mb = 0; mb < kBwdMB; ++mb) {
        DX[mb] = Ty::mma32(tu0, pack_kstep<Ty>(DPu[mb], 0), zero);
        DX[mb] = Ty::mma32(tu1, pack_kstep<Ty>(DPu[mb], 1), DX[mb]);
        DX[mb] = Ty::mma32(tv0, pack_kstep<Ty>(DPv[mb], 0), DX[mb]);
        DX[mb] = Ty::mma32(tv1, pack_kstep<Ty>(DPv[mb], 1), DX[mb]);
      }
    }
    mfma_drain();

    // Through the wave's staging tile [32 slots][kLd]: dP_u, dP_v, W' as rows for the dA
    // products, dX' as 16-byte row vectors to memory.
    auto put = [&](const f32x16 (&m)[kBwdMB]) {
#pragma unroll
      for (int mb = 0; mb < kBwdMB; ++mb)
#pragma unroll
        for (int i = 0; i < 16; ++i) stage[pair_token_row(i, hh) * kLd + 32 * mb + l32] = Ty::from_f32(m[mb][i]);
      wave_lds_sync();
    };
    // dA_m += sum over the pair's two tiles of rows(stage) rows(other)^T: A operand lane (t, h4)
    // = stage row 16 g + t, channels 16 ks + 4 h4 .. + 3; B operand = row 16 g + l16 of other.
    auto staged_row = [&](int g, int ks) {
      return *reinterpret_cast<const u32x2*>(stage + (16 * g + l16) * kLd + 16 * ks + 4 * h4);
    };
    f32x4 dA[3] = {};
    if (live) {
      if (RT && a.rscale) {
        // X' = x r for the routed rows.
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          const float rs = __shfl(my_rs, 16 * g + l16);
#pragma unroll
          for (int ks = 0; ks < kBwdKS; ++ks) xo[g][ks] = u32x2{scale2<Ty>(xo[g][ks][0], rs), scale2<Ty>(xo[g][ks][1], rs)};
        }
      }
      put(DPu);
#pragma unroll
      for (int g = 0; g < 2; ++g)
#pragma unroll
        for (int ks = 0; ks < kBwdKS; ++ks) dA[0] = Ty::mma16(staged_row(g, ks), xo[g][ks], dA[0]);
      wave_lds_sync();
      put(DPv);
#pragma unroll
      for (int g = 0; g < 2; ++g)
#pragma unroll
        for (int ks = 0; ks < kBwdKS; ++ks) dA[1] = Ty::mma16(staged_row(g, ks), xo[g][ks], dA[1]);
      wave_lds_sync();
      // dA_o = dY W'^T: A operand from dY rows, B from the staged W' rows.
      put(W);
#pragma unroll
      for (int g = 0; g < 2; ++g)
#pragma unroll
        for (int ks = 0; ks < kBwdKS; ++ks) dA[2] = Ty::mma16(yo[g][ks], staged_row(g, ks), dA[2]);
      wave_lds_sync();
      put(DX);
      // dX' leaves non-temporally too (buffer cache policy 2 = nt): it is not read again by
      // this pass (0.785 -> 0.774 ms at the batch above).
      if constexpr (RT) {
        uint32_t goff[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) goff[k] = row_off(row_of((lane + 64 * k) >> 3), ((lane + 64 * k) & 7) * 8);
        const __amdgpu_buffer_rsrc_t rg = buffer_rsrc(a.g, nbytes_rows);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int v = lane + 64 * k, r = v >> 3, c8 = (v & 7) * 8;
          __builtin_amdgcn_raw_buffer_store_b128(*reinterpret_cast<const u32x4*>(stage + r * kLd + c8), rg, goff[k], 0, 2);
        }
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int v = lane + 64 * k, r = v >> 3, c8 = (v & 7) * 8;
          __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(stage + r * kLd + c8),
                                      reinterpret_cast<u32x4*>(a.dxt + (slot0 + r) * kBwdD + c8));
        }
      }
      wave_lds_sync();  // the staging tile is read before the next pair's rows replace it
    }
    mfma_drain();
    if constexpr (RES) {
#pragma unroll
      for (int m = 0; m < 3; ++m) dA_run[m] += dA[m];
    } else {
#pragma unroll
      for (int m = 0; m < 3; ++m)
#pragma unroll
        for (int i = 0; i < 4; ++i) red[wave][m][(4 * h4 + i) * 16 + l16] += dA[m][i];
    }
  };

  float(*sums)[3][256];  // the waves' dA sums for the final fixed-order addition
  if constexpr (RES) {
    // The group's weights into LDS once (12 KB per wave); then every wave on its own.
    const int q = static_cast<int>(blockIdx.x % a.q_c);
    const int64_t wg_in_q = blockIdx.x / a.q_c, wpg = gridDim.x / a.q_c;
    const uint16_t* wsrc = a.packed + static_cast<int64_t>(q) * NCH * CH_ELEMS;
    for (int f = wave; f < NCH * kBwdFr; f += NW) bwd_copy_frag(wsrc + f * kFragElems, &wb[0][0] + f * kFragElems, lane);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();  // weights and tok are written
    uint16_t* tx = tiles[wave];
    const int64_t pstride = wpg * NW;
    int64_t pair = wg_in_q * NW + wave;
    PairTok cur_tok = pair_tok(pair, pair < a.pairs_per_q);
    for (; pair < a.pairs_per_q; pair += pstride) {
      const int64_t nxt = pair + pstride;
      const PairTok next_tok = pair_tok(nxt, nxt < a.pairs_per_q);
      do_pair(q, pair, true, cur_tok, next_tok, tx, tx, [](int) {},
              [&](int ec) { return reinterpret_cast<const u32x4*>(wb[ec]); });
    }
    __syncthreads();  // every wave is done with its tile
    sums = reinterpret_cast<float(*)[3][256]>(&tiles[0][0]);
#pragma unroll
    for (int m = 0; m < 3; ++m)
#pragma unroll
      for (int i = 0; i < 4; ++i) sums[wave][m][(4 * h4 + i) * 16 + l16] = dA_run[m][i];
  } else {
    PairTok cur_tok = pair_tok((blockIdx.x % wg_per_q) * 4 + wave,
                               blockIdx.x < a.rounds && (blockIdx.x % wg_per_q) * 4 + wave < a.pairs_per_q);
    for (int64_t round = blockIdx.x; round < a.rounds; round += gridDim.x) {
      const int q = static_cast<int>(round / wg_per_q);
      const int64_t pair = (round % wg_per_q) * 4 + wave;
      const bool live = pair < a.pairs_per_q;  // waves past the end still take part in the barriers
      const uint16_t* wsrc = a.packed + static_cast<int64_t>(q) * NCH * CH_ELEMS;
      auto issue = [&](int ec) {
        for (int f = wave; f < kBwdFr; f += 4)
          bwd_copy_frag(wsrc + static_cast<int64_t>(ec) * CH_ELEMS + f * kFragElems, wb[ec & 1] + f * kFragElems, lane);
      };
      __syncthreads();  // the previous round is done with both weight buffers; tok is written
      issue(0);
      const int64_t nr = round + gridDim.x;
      const int64_t npair = (nr % wg_per_q) * 4 + wave;
      const PairTok next_tok = pair_tok(npair, nr < a.rounds && npair < a.pairs_per_q);
      // The token side's tile is in the second weight buffer (no copy targets it before the
      // first barrier of the chunk loop); the dA staging in the buffer of chunk NCH, which no copy
      // targets after the loop's last barrier.
      do_pair(q, pair, live, cur_tok, next_tok, wb[1] + wave * 32 * kLd, wb[NCH & 1] + wave * 32 * kLd,
              [&](int ec) {
                // Chunk ec's copies: chunk 0 landed before the tile loads the compiler waited on;
                // chunk ec >= 1 was issued at step ec - 1, and nothing follows it.
                if (ec > 0) wait_vmcnt<0>();
                __syncthreads();  // chunk ec landed; every wave is done with chunk ec - 1 (ec = 0: its tiles)
                if (ec + 1 < NCH) issue(ec + 1);
              },
              [&](int ec) { return reinterpret_cast<const u32x4*>(wb[ec & 1]); });
    }
    __syncthreads();
    sums = red;
  }
  // The workgroup's dA sums, the waves added in order.
  if constexpr (RES) __syncthreads();
  for (int e = threadIdx.x; e < 3 * 256; e += 64 * NW) {
    const int m = e >> 8, k = e & 255;
    float v = sums[0][m][k];
#pragma unroll
    for (int w = 1; w < NW; ++w) v += sums[w][m][k];
    a.partial[static_cast<int64_t>(blockIdx.x) * 768 + e] = v;
  }
}

// Workgroups of the resident-weights kernel: about one per CU, a multiple of q_c (at least one
// per group), no more per group than it has 8-pair rows.
int64_t bwd_fused_res_grid(int64_t pairs, int32_t q_c) {
  int64_t per = static_cast<int64_t>(device_cus()) / q_c;
  const int64_t need = (pairs + kBwdResWaves - 1) / kBwdResWaves;
  if (per > need) per = need;
  if (per < 1) per = 1;
  return per * q_c;
}

template <bool RT>
int launch_bwd_fused(const BwdFusedArgs& a, int64_t grid, int32_t rd, int32_t dtype, hipStream_t s) {
  const dim3 g(static_cast<unsigned>(grid));
  if (dtype == OW_DTYPE_BF16) {
    if (rd == 128)
      hipLaunchKernelGGL((bwd_fused_d64_kernel<BF16, 128, RT, true>), g, dim3(64 * kBwdResWaves), 0, s, a);
    else
      hipLaunchKernelGGL((bwd_fused_d64_kernel<BF16, 256, RT, false>), g, dim3(256), 0, s, a);
  } else {
    if (rd == 128)
      hipLaunchKernelGGL((bwd_fused_d64_kernel<F16, 128, RT, true>), g, dim3(64 * kBwdResWaves), 0, s, a);
    else
      hipLaunchKernelGGL((bwd_fused_d64_kernel<F16, 256, RT, false>), g, dim3(256), 0, s, a);
  }
  if (int rc = hip_status(hipGetLastError(), "bwd_fused_d64_kernel launch")) return rc;
  clear_error();
  return OW_OK;
}

// ---- Parameter-gradient reduction, d = 64, recomputing the gate --------------------------
// dB_u'' = P_u^T dU', dB_v'' = P_v^T dV' ([64][rd]) and dB_o'' = Z^T dW' ([rd][64]), summed over
// the slots of one channel group, from P_u, P_v, dW' alone (as ow_bwd_fused stores them): the
// chunk products U' = P_u B_u'', V' = P_v B_v'', dZ = dW' B_o''^T and the gate backward (Z, dU',
// dV') are recomputed here from the same 16-bit operands and packed weights instead of being
// stored by the fused kernel and read back (at rd = 128 that is 768 bytes per slot more of each).
// P rows are kept in the pair-operand channel order: element 16 k + 8 h + j of a row is channel
// 16 k + kord(j, h), so lane (slot, h) of a K-step operand is one 16-byte piece.
// Workgroup b takes group q = b % q_c and 2-pair steps s, s + R, .. (s = b / q_c, R = gridDim.x /
// q_c).  Each step's 2 x 3 [32 slots][64] tiles are copied by the 8 waves (buffer_load ... lds, 3
// per wave, untracked) into one of kR64Stages LDS stages, kR64Ahead steps ahead; one barrier
// per step.  Wave w owns the 32-row chunk ec = w % (rd / 32) of the expanded dimension
// (its 12 weight fragments stay in registers) for pair w / (rd / 32) of each step (rd = 256:
// both pairs): U', V', dZ of its chunk with lane = expanded row, registers = slots (K-step
// operands read as 16-byte pieces), the gate, then dB_u''[:, ec] += P_u^T dU', dB_v''[:, ec] +=
// P_v^T dV' and dB_o''[ec, :] += Z^T dW' with the P^T / dW' operands by transposed LDS reads
// (ds_read_b64_tr_b16) and the gate outputs as the other operand.  Rows hold their 16-byte
// pieces swizzled (piece p of row r at p ^ kR64Swz(r)), which keeps both read forms free of
// bank conflicts.  At rd = 128 the two waves of a chunk add their sums through LDS (in a fixed
// order) before the workgroup writes range s's partial row, laid out [3][q_c][64 rd]; their
// sum over s (ow_sum_rows) is the [3][q_c][64 rd] gradient buffer.
struct ParamReduceArgs {
  const uint16_t* pu;      // [q_c][pairs * 32][64], pair-operand channel order
  const uint16_t* pv;
  const uint16_t* dw;
  const uint16_t* packed;  // ow_pack_bwd_weights, d = 64
  float* partial;          // [ranges][3][q_c][64 * rd]
  int64_t pairs;           // per group
  int32_t q_c;
};
constexpr int kR64Waves = 8;
constexpr int kR64Ahead = 2;   // steps copied ahead
constexpr int kR64Stages = 4;  // kR64Ahead + 2: the lagging waves still read step i - 1
constexpr int kR64Pairs = 2;                            // pairs per step
constexpr int kR64Tile = 32 * kBwdD;                    // elements of one [32][64] tile
constexpr int kR64Stage = kR64Pairs * 3 * kR64Tile * 2;  // bytes per stage (24 KB)

__device__ __forceinline__ int kR64Swz(int r) { return 4 * ((r >> 1) & 1) + ((r >> 2) & 3); }
// Position of channel c within a stored row (bits 2 and 3 swapped: the pair-operand order).
__device__ __forceinline__ int r64_pos(int c) { return (c & ~12) | ((c & 4) << 1) | ((c & 8) >> 1); }
// LDS byte address of element position p of row r in a swizzled [32][64] tile at base.
__device__ __forceinline__ uint32_t r64_at(uint32_t base, int r, int p) {
  return base + static_cast<uint32_t>(r * 128 + (((p >> 3) ^ kR64Swz(r)) << 4) + 2 * (p & 7));
}

template <class Ty, int RD>
__global__ void __launch_bounds__(64 * kR64Waves) bwd_param_reduce64_kernel(ParamReduceArgs a) {
  constexpr int NCH = RD / 32;
  constexpr int WPP = kR64Waves / NCH;  // waves per chunk (2 at rd = 128, 1 at rd = 256)
  constexpr int CH_ELEMS = kBwdFr * kFragElems;
  constexpr int COMBINE = (WPP - 1) * (kR64Waves / WPP) * 96 * 64 * 4;  // bytes of the rd = 128 combine
  constexpr int LDS = kR64Stages * kR64Stage > COMBINE ? kR64Stages * kR64Stage : COMBINE;
  static_assert(WPP == 1 || WPP == 2, "rd in {128, 256}");
  __shared__ __attribute__((aligned(16))) uint8_t lds[LDS];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hh = lane >> 5, l32 = lane & 31, l16 = lane & 15, half = (lane >> 4) & 1;
  const int ec = w % NCH, pp0 = w / NCH;
  const int q = blockIdx.x % a.q_c;
  const int64_t s0 = blockIdx.x / a.q_c, sstep = gridDim.x / a.q_c;
  const int64_t steps = (a.pairs + kR64Pairs - 1) / kR64Pairs;
  const int64_t n_iter = s0 < steps ? (steps - s0 + sstep - 1) / sstep : 0;  // same for every wave
  const uint32_t lds0 = lds_addr(lds);

  // The chunk's weight operands (lane = expanded row 32 ec + l32, K = channels): fragments
  // ks, 4 + ks, 8 + ks of the chunk are B_u'', B_v'', B_o'' for K-step ks.
  u32x4 wu[kBwdKS], wv[kBwdKS], wo[kBwdKS];
  {
    const u32x4* src = reinterpret_cast<const u32x4*>(a.packed + (static_cast<size_t>(q) * NCH + ec) * CH_ELEMS);
#pragma unroll
    for (int ks = 0; ks < kBwdKS; ++ks) {
      wu[ks] = src[ks * (kFragElems / 8) + lane];
      wv[ks] = src[(kBwdKS + ks) * (kFragElems / 8) + lane];
      wo[ks] = src[(2 * kBwdKS + ks) * (kFragElems / 8) + lane];
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  const uint32_t tbytes = static_cast<uint32_t>(a.q_c * a.pairs * kR64Tile * 2);
  const __amdgpu_buffer_rsrc_t rt[3] = {buffer_rsrc(a.pu, tbytes), buffer_rsrc(a.pv, tbytes), buffer_rsrc(a.dw, tbytes)};
  // This wave's copies per step: 1 KB pieces k = w + 8 c (pair k / 12, tensor (k % 12) / 4, rows
  // 8 (k % 4) .. + 7); lane -> row rr, LDS slot lane % 8 holding piece (lane % 8) ^ kR64Swz(rr).
  uint32_t loff[3];
  int kpair[3], ktensor[3];
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    const int k = w + kR64Waves * c;
    kpair[c] = k / 12;
    ktensor[c] = (k % 12) / 4;
    const int rr = 8 * (k % 4) + (lane >> 3), sl = lane & 7;
    loff[c] = static_cast<uint32_t>(rr * 128 + 16 * (sl ^ kR64Swz(rr)));
  }
  auto issue = [&](int64_t i) {
    const int64_t st = s0 + i * sstep;
    const uint32_t stage = lds0 + static_cast<uint32_t>((i % kR64Stages) * kR64Stage);
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      const int k = w + kR64Waves * c;
      const int64_t pair = st * kR64Pairs + kpair[c];
      const bool ok = st < steps && pair < a.pairs;
      const uint32_t voff = ok ? static_cast<uint32_t>((q * a.pairs + pair) * kR64Tile * 2) + loff[c] : kOffOut;
      tile_copy_nt(ktensor[c] == 0 ? rt[0] : ktensor[c] == 1 ? rt[1] : rt[2], voff, stage + 1024u * k);
    }
  };

  f32x16 acc_u[kBwdMB] = {}, acc_v[kBwdMB] = {}, acc_o[kBwdMB] = {};
  auto stage_of = [&](int64_t i) { return lds0 + static_cast<uint32_t>((i % kR64Stages) * kR64Stage); };
  // U', V', dZ of the chunk for pair pp of a stage: A = the P rows (lane = slot l32, K-step ks =
  // piece 2 ks + hh), B = the chunk's weights.
  auto products = [&](uint32_t stage, int pp, f32x16& U, f32x16& V, f32x16& G) {
    const uint32_t tu = stage + static_cast<uint32_t>(pp * 3 * kR64Tile * 2);
    const uint32_t tv = tu + kR64Tile * 2, tw = tv + kR64Tile * 2;
    U = f32x16{};
    V = f32x16{};
    G = f32x16{};
#pragma unroll
    for (int ks = 0; ks < kBwdKS; ++ks) {
      const int pos = 16 * ks + 8 * hh;
      const u32x4 xu = *reinterpret_cast<const u32x4*>(lds + (r64_at(tu, l32, pos) - lds0));
      const u32x4 xv = *reinterpret_cast<const u32x4*>(lds + (r64_at(tv, l32, pos) - lds0));
      const u32x4 xw = *reinterpret_cast<const u32x4*>(lds + (r64_at(tw, l32, pos) - lds0));
      U = Ty::mma32(xu, wu[ks], U);
      V = Ty::mma32(xv, wv[ks], V);
      G = Ty::mma32(xw, wo[ks], G);
    }
  };
  // The gate on U', V', dZ (register i of lane (l32, hh): expanded row 32 ec + l32, slot
  // kord(i, hh)) and the sums dB_u'' += P_u^T dU', dB_v'' += P_v^T dV', dB_o'' += Z^T dW'.
  auto gate_sums = [&](uint32_t stage, int pp, const f32x16& U, const f32x16& V, const f32x16& G) {
    const uint32_t tu = stage + static_cast<uint32_t>(pp * 3 * kR64Tile * 2);
    const uint32_t tv = tu + kR64Tile * 2, tw = tv + kR64Tile * 2;
    // Slot-K operands: lane (l32, hh) = channel 32 cb + l32 of P^T / dW', slots 16 s + kord(j, hh):
    // two transposed reads (rows 16 s + 4 hh + 0..3 and + 8).
    auto tr = [&](uint32_t t, int cb, int sk) {
      const int r = 16 * sk + 4 * hh + (l16 >> 2);
      const int p = r64_pos(32 * cb + 16 * half + 4 * (l16 & 3));
      const u32x2 x = lds_read_tr16(r64_at(t, r, p)), y = lds_read_tr16(r64_at(t, r + 8, p));
      return u32x4{x[0], x[1], y[0], y[1]};
    };
#pragma unroll
    for (int sk = 0; sk < 2; ++sk) {
      // The gate on registers 8 sk .. 8 sk + 7 (slots 16 sk + kord(j, hh)), packed straight into
      // the K-step sk operands.
      uint32_t zp[4], dup[4], dvp[4];
#pragma unroll
      for (int j = 0; j < 8; j += 2) {
        float z2[2], du2[2], dv2[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const float up = U[8 * sk + j + e], vp = V[8 * sk + j + e], g = G[8 * sk + j + e];
          const float sg = gate_sigmoid(up);
          z2[e] = up * vp * sg;
          du2[e] = g * vp * sg * (1.0f - kLn2 * up * (1.0f - sg));
          dv2[e] = g * up * sg;
        }
        zp[j / 2] = Ty::pack2(z2[0], z2[1]);
        dup[j / 2] = Ty::pack2(du2[0], du2[1]);
        dvp[j / 2] = Ty::pack2(dv2[0], dv2[1]);
      }
      const u32x4 zs = u32x4{zp[0], zp[1], zp[2], zp[3]}, dus = u32x4{dup[0], dup[1], dup[2], dup[3]},
                  dvs = u32x4{dvp[0], dvp[1], dvp[2], dvp[3]};
#pragma unroll
      for (int cb = 0; cb < kBwdMB; ++cb) {
        acc_u[cb] = Ty::mma32(tr(tu, cb, sk), dus, acc_u[cb]);
        acc_v[cb] = Ty::mma32(tr(tv, cb, sk), dvs, acc_v[cb]);
        acc_o[cb] = Ty::mma32(zs, tr(tw, cb, sk), acc_o[cb]);
      }
    }
  };
  // Step i is issued at iteration i - kR64Ahead into stage i % kR64Stages; at iteration i the
  // stages of steps i - 1 .. i + kR64Ahead are in use (see the rd = 128 schedule below).
  static_assert(kR64Stages == kR64Ahead + 2, "a stage for the lagging waves' previous step");
#pragma unroll
  for (int i = 0; i < kR64Ahead; ++i) issue(i);
  // One iteration's start: this wave's copies of step i landed (those of steps i + 1 ..
  // i + kR64Ahead - 1 may be in flight); the barrier makes every wave's visible and means every
  // wave is done with step i - 2, whose stage step i + kR64Ahead takes.  Every wave passes the
  // same number of barriers (n_iter is the workgroup's).
  auto next_step = [&](int64_t i) {
    wait_vmcnt<3 * (kR64Ahead - 1)>();
    __syncthreads();
    issue(i + kR64Ahead);
  };
  f32x16 U, V, G;
  if (WPP == 2 && pp0 == 1) {
    // rd = 128: waves w and w + 4 share a SIMD (and a chunk).  Wave w does step i's pair 0
    // (products, gate, sums) in iteration i; wave w + 4 runs half a step behind: the gate and
    // sums of step i - 1's pair 1 (its products held from the last iteration), then step i's
    // pair 1 products.  So one wave's MFMAs meet the other's gate VALU work instead of both
    // entering each phase together after the barrier.
    for (int64_t i = 0; i < n_iter; ++i) {
      next_step(i);
      if (i > 0) {
        mfma_drain();
        gate_sums(stage_of(i - 1), 1, U, V, G);
      }
      products(stage_of(i), 1, U, V, G);
    }
    if (n_iter > 0) {
      // The last step's pair 1 (no copy targets its stage: those are steps up to
      // n_iter - 1 + kR64Ahead).
      mfma_drain();
      gate_sums(stage_of(n_iter - 1), 1, U, V, G);
    }
  } else {
    for (int64_t i = 0; i < n_iter; ++i) {
      next_step(i);
#pragma unroll 1
      for (int pp = pp0; pp < kR64Pairs; pp += WPP) {
        products(stage_of(i), pp, U, V, G);
        mfma_drain();
        gate_sums(stage_of(i), pp, U, V, G);
      }
    }
  }
  wait_vmcnt<0>();  // the trailing copies (past the end: zeros) are done before LDS is reused
  mfma_drain();
  // acc_u / acc_v register i of lane (l32, hh): channel 32 cb + kord(i, hh), expanded row
  // 32 ec + l32; acc_o: expanded row 32 ec + kord(i, hh), channel 32 cb + l32.
  if constexpr (WPP == 2) {
    // The second wave of each chunk hands its sums to the first through LDS.
    __syncthreads();  // every wave is done with the stages
    float* cmb = reinterpret_cast<float*>(lds) + static_cast<size_t>(ec) * 96 * 64;
    if (pp0 == 1) {
#pragma unroll
      for (int cb = 0; cb < kBwdMB; ++cb)
#pragma unroll
        for (int i2 = 0; i2 < 16; ++i2) {
          cmb[((0 * kBwdMB + cb) * 16 + i2) * 64 + lane] = acc_u[cb][i2];
          cmb[((1 * kBwdMB + cb) * 16 + i2) * 64 + lane] = acc_v[cb][i2];
          cmb[((2 * kBwdMB + cb) * 16 + i2) * 64 + lane] = acc_o[cb][i2];
        }
    }
    __syncthreads();
    if (pp0 == 1) return;
#pragma unroll
    for (int cb = 0; cb < kBwdMB; ++cb)
#pragma unroll
      for (int i2 = 0; i2 < 16; ++i2) {
        acc_u[cb][i2] += cmb[((0 * kBwdMB + cb) * 16 + i2) * 64 + lane];
        acc_v[cb][i2] += cmb[((1 * kBwdMB + cb) * 16 + i2) * 64 + lane];
        acc_o[cb][i2] += cmb[((2 * kBwdMB + cb) * 16 + i2) * 64 + lane];
      }
  }
  float* out_u = a.partial + ((s0 * 3 + 0) * a.q_c + q) * (kBwdD * RD);
  float* out_v = a.partial + ((s0 * 3 + 1) * a.q_c + q) * (kBwdD * RD);
  float* out_o = a.partial + ((s0 * 3 + 2) * a.q_c + q) * (kBwdD * RD);
#pragma unroll
  for (int cb = 0; cb < kBwdMB; ++cb)
#pragma unroll
    for (int i2 = 0; i2 < 16; ++i2) {
      const int k = 32 * cb + 8 * (i2 >> 2) + 4 * hh + (i2 & 3);  // channel (u, v) / expanded row (o)
      out_u[k * RD + 32 * ec + l32] = acc_u[cb][i2];
      out_v[k * RD + 32 * ec + l32] = acc_v[cb][i2];
      out_o[(32 * ec + k - 32 * cb) * kBwdD + 32 * cb + l32] = acc_o[cb][i2];
    }
}

// Step ranges S of the reduction (partial rows S q_c; grid S q_c): about one workgroup of 8 waves
// per CU, at least one 2-pair step per range.
int64_t bwd_param_reduce64_ranges(int64_t pairs, int32_t q_c) {
  const int64_t steps = (pairs + kR64Pairs - 1) / kR64Pairs;
  int64_t ranges = static_cast<int64_t>(device_cus()) / q_c;
  if (ranges < 1) ranges = 1;
  return ranges > steps ? steps : ranges;
}

template <int RD>
int launch_param_reduce64(const ParamReduceArgs& a, int64_t grid, int32_t dtype, hipStream_t s) {
  const dim3 g(static_cast<unsigned>(grid));
  if (dtype == OW_DTYPE_BF16)
    hipLaunchKernelGGL((bwd_param_reduce64_kernel<BF16, RD>), g, dim3(64 * kR64Waves), 0, s, a);
  else
    hipLaunchKernelGGL((bwd_param_reduce64_kernel<F16, RD>), g, dim3(64 * kR64Waves), 0, s, a);
  return hip_status(hipGetLastError(), "bwd_param_reduce64_kernel launch");
}

// ---- Parameter-gradient reduction, d = 128 -----------------------------------------------
// dB_u'' = P_u^T dU', dB_v'' = P_v^T dV' ([128][rd]) and dB_o'' = Z^T dW' ([rd][128]), each a
// sum over the slots of one channel group, from the slot-major intermediates of
// ow_bwd_channel (P_u, P_v, dW' [q_c][slots][128]; Z, dU', dV' [q_c][slots][rd]).  Workgroup b
// takes group q = b % q_c, product t = (b / q_c) % 3 and 32-slot steps s, s + R, .. of that
// group (s = b / (3 q_c), R = gridDim.x / (3 q_c)): per step it needs 32 rows of the product's
// left tensor A (P_u, P_v or Z; MW channels) and of its right tensor B (dU', dV' or dW'; NW),
// which its 8 waves copy (buffer_load ... lds, untracked, 1 KB per copy) into one of
// kR2Stages LDS stages, kR2Stages - 1 steps ahead; one barrier per step.  A row keeps its 16-byte
// pieces swizzled (piece p of row r at slot p ^ 4 (r & 3)), so the transposed operand reads
// (ds_read_b64_tr_b16, four rows x 32 channels per 32 lanes) hit distinct banks.  Wave w owns a
// 2 x NB block rectangle of the [MW][NW] product (32x32 blocks, fp32 registers) and reads its
// 2 + NB operands per 16 slots.  The sums go to range s's partial row, laid out
// [3][q_c][128 rd], so that the sum of the rows over s (ow_sum_rows) is the [3][q_c][128 rd]
// gradient buffer.  Rows past the group's slots read as zero.
struct ParamReduce128Args {
  const uint16_t* pu;  // [q_c][slots][128]
  const uint16_t* pv;
  const uint16_t* dw;
  const uint16_t* z;   // [q_c][slots][rd]
  const uint16_t* du;
  const uint16_t* dv;
  float* partial;      // [ranges][3][q_c][128 * rd]
  int64_t slots;       // per group, a multiple of 16
  int32_t q_c;
};
constexpr int kR2D = 128;  // channel-group width d
constexpr int kR2Waves = 8;
constexpr int kR2Stages = 4;
constexpr int kR2Slots = 32;  // slots per step

// The LDS byte address of channel c of row r in a swizzled [rows][W] tile at base.
template <int W>
__device__ __forceinline__ uint32_t r2_at(uint32_t base, int r, int c) {
  return base + 2u * static_cast<uint32_t>(r * W + ((((c >> 3) ^ (4 * (r & 3)))) << 3) + (c & 7));
}

template <class Ty, int MW, int NW>
__device__ __forceinline__ void param_reduce128_product(const ParamReduce128Args& a, const uint16_t* A,
                                                        const uint16_t* B, uint32_t lds0, int q, int64_t s0,
                                                        int64_t sstep, float* out) {
  constexpr int STAGE = kR2Slots * (MW + NW) * 2;         // bytes per stage
  constexpr int COPIES = (MW + NW) * kR2Slots * 2 / 1024 / kR2Waves;  // per wave and step
  constexpr int ACH = MW * kR2Slots * 2 / 1024;            // copies of the A rows per step
  constexpr int NB = MW * NW / (1024 * kR2Waves * 2);      // n blocks per wave (m blocks: 2)
  constexpr int MP = MW / 64;                              // m-block pairs
  static_assert(COPIES * kR2Waves * 1024 == STAGE, "whole copies per wave");
  static_assert(NB >= 1 && (NW / 32) % NB == 0 && MP * (NW / 32 / NB) == kR2Waves, "block rectangles");
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hh = lane >> 5, l32 = lane & 31, l16 = lane & 15, half = (lane >> 4) & 1;
  const int mp = w % MP, np = w / MP;
  const int64_t steps = (a.slots + kR2Slots - 1) / kR2Slots;
  const int64_t n_iter = s0 < steps ? (steps - s0 + sstep - 1) / sstep : 0;  // same for every wave
  const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(A, static_cast<uint32_t>(a.q_c * a.slots * MW * 2));
  const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(B, static_cast<uint32_t>(a.q_c * a.slots * NW * 2));
  // This wave's copies per step: 1 KB pieces k = w + 8 c of the stage (k < ACH: A rows, else B
  // rows).  Lane -> row rr of the step and LDS slot sl of the row, which holds piece sl ^ 4 (rr & 3).
  uint32_t loff[COPIES], ldsk[COPIES];
  int lrow[COPIES];
  bool isa[COPIES];
#pragma unroll
  for (int c = 0; c < COPIES; ++c) {
    const int k = w + kR2Waves * c;
    isa[c] = k < ACH;
    const int width = isa[c] ? MW : NW, ppr = width / 8;  // 16-byte pieces per row
    const int kk = isa[c] ? k : k - ACH;
    const int rr = kk * (1024 / (2 * width)) + lane / ppr, sl = lane % ppr;
    lrow[c] = rr;
    loff[c] = static_cast<uint32_t>((rr * width + 8 * (sl ^ (4 * (rr & 3)))) * 2);
    ldsk[c] = static_cast<uint32_t>((isa[c] ? 0 : kR2Slots * MW * 2) + kk * 1024);
  }
  auto issue = [&](int64_t i) {
    const int64_t step = s0 + i * sstep;
    const int64_t slot0 = step * kR2Slots;
    const uint32_t stage = lds0 + static_cast<uint32_t>((i % kR2Stages) * STAGE);
    const uint32_t row0 = static_cast<uint32_t>(q * a.slots + slot0);
#pragma unroll
    for (int c = 0; c < COPIES; ++c) {
      const bool ok = step < steps && slot0 + lrow[c] < a.slots;
      const uint32_t voff = ok ? row0 * static_cast<uint32_t>((isa[c] ? MW : NW) * 2) + loff[c] : kOffOut;
      tile_copy_nt(isa[c] ? ra : rb, voff, stage + ldsk[c]);
    }
  };
  f32x16 acc[2][NB] = {};
#pragma unroll
  for (int i = 0; i < kR2Stages - 1; ++i) issue(i);
  for (int64_t i = 0; i < n_iter; ++i) {
    // This wave's copies of step i landed (those of steps i + 1 .. i + kR2Stages - 2 may be in
    // flight); the barrier makes every wave's visible and means every wave is done with stage
    // (i - 1) % kR2Stages, which step i + kR2Stages - 1 takes.
    wait_vmcnt<COPIES * (kR2Stages - 2)>();
    __syncthreads();
    issue(i + kR2Stages - 1);
    const uint32_t sa = lds0 + static_cast<uint32_t>((i % kR2Stages) * STAGE), sb = sa + kR2Slots * MW * 2;
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      // Lane (l32, hh) holds channel 32 blk + l32 of rows 16 g + 4 hh + 0..3 and 16 g + 8 + 4 hh
      // + 0..3 (the K order of both operands).
      const int r = 16 * g + 4 * hh + (l16 >> 2), cl = 16 * half + 4 * (l16 & 3);
      u32x4 av[2], bv[NB];
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const int c = 32 * (2 * mp + m) + cl;
        const u32x2 x = lds_read_tr16(r2_at<MW>(sa, r, c)), y = lds_read_tr16(r2_at<MW>(sa, r + 8, c));
        av[m] = u32x4{x[0], x[1], y[0], y[1]};
      }
#pragma unroll
      for (int n = 0; n < NB; ++n) {
        const int c = 32 * (NB * np + n) + cl;
        const u32x2 x = lds_read_tr16(r2_at<NW>(sb, r, c)), y = lds_read_tr16(r2_at<NW>(sb, r + 8, c));
        bv[n] = u32x4{x[0], x[1], y[0], y[1]};
      }
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int n = 0; n < NB; ++n) acc[m][n] = Ty::mma32(av[m], bv[n], acc[m][n]);
    }
  }
  wait_vmcnt<0>();  // the trailing copies (past the end: zeros) are done before the exit
  mfma_drain();
  // Accumulator register i of lane (l32, hh): row 32 mb + kord(i, hh), column 32 nb + l32.
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int n = 0; n < NB; ++n)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int row = 32 * (2 * mp + m) + 8 * (i >> 2) + 4 * hh + (i & 3), col = 32 * (NB * np + n) + l32;
        out[row * NW + col] = acc[m][n][i];
      }
}

template <class Ty, int RD>
__global__ void __launch_bounds__(64 * kR2Waves) bwd_param_reduce128_kernel(ParamReduce128Args a) {
  __shared__ __attribute__((aligned(16))) uint16_t st[kR2Stages][kR2Slots * (kR2D + RD)];
  const int q = blockIdx.x % a.q_c, t = (blockIdx.x / a.q_c) % 3;
  const int64_t s0 = blockIdx.x / (3 * a.q_c), sstep = gridDim.x / (3 * a.q_c);
  float* out = a.partial + ((s0 * 3 + t) * a.q_c + q) * (kR2D * RD);
  const uint32_t lds0 = lds_addr(&st[0][0]);
  if (t < 2)
    param_reduce128_product<Ty, kR2D, RD>(a, t == 0 ? a.pu : a.pv, t == 0 ? a.du : a.dv, lds0, q, s0, sstep, out);
  else
    param_reduce128_product<Ty, RD, kR2D>(a, a.z, a.dw, lds0, q, s0, sstep, out);
}

// Slot ranges R of the d = 128 reduction (grid 3 q_c R, partial rows R): at most one workgroup
// per CU, at least one 32-slot step per range.
int64_t bwd_param_reduce128_ranges(int64_t slots, int32_t q_c) {
  const int64_t steps = (slots + kR2Slots - 1) / kR2Slots;
  int64_t ranges = static_cast<int64_t>(device_cus()) / (3 * static_cast<int64_t>(q_c));
  if (ranges < 1) ranges = 1;
  return ranges > steps ? steps : ranges;
}

template <int RD>
int launch_param_reduce128(const ParamReduce128Args& a, int64_t grid, int32_t dtype, hipStream_t s) {
  const dim3 g(static_cast<unsigned>(grid));
  if (dtype == OW_DTYPE_BF16)
    hipLaunchKernelGGL((bwd_param_reduce128_kernel<BF16, RD>), g, dim3(64 * kR2Waves), 0, s, a);
  else
    hipLaunchKernelGGL((bwd_param_reduce128_kernel<F16, RD>), g, dim3(64 * kR2Waves), 0, s, a);
  return hip_status(hipGetLastError(), "bwd_param_reduce128_kernel launch");
}

// ---- Fixed-order sum of fp32 partial rows -------------------------------------------------
// out[c] = sum over r of p[r][c] (cols a multiple of 4, 16-byte aligned rows).  Workgroup b sums
// columns 256 b .. 256 b + 255 (lane: four of them); its W waves take rows w, w + W, .. in
// order and are then added in wave order, so the result depends on rows, cols and W only.
__global__ void __launch_bounds__(1024) sum_rows_kernel(const float4* __restrict__ p, int64_t rows, int64_t cols4,
                                                        float4* __restrict__ out, int W) {
  __shared__ float4 part[16][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t c = static_cast<int64_t>(blockIdx.x) * 64 + lane;
  float4 s = {0.0f, 0.0f, 0.0f, 0.0f};
  if (c < cols4) {
    int64_t r = w;
    for (; r + 3 * W < rows; r += 4 * W) {
      const float4 x0 = p[r * cols4 + c], x1 = p[(r + W) * cols4 + c];
      const float4 x2 = p[(r + 2 * W) * cols4 + c], x3 = p[(r + 3 * W) * cols4 + c];
      s += x0;
      s += x1;
      s += x2;
      s += x3;
    }
    for (; r < rows; r += W) s += p[r * cols4 + c];
  }
  if (W > 1) {
    part[w][lane] = s;
    __syncthreads();
    if (w == 0)
      for (int k = 1; k < W; ++k) s += part[k][lane];
  }
  if (w == 0 && c < cols4) out[c] = s;
}

// Waves per workgroup of sum_rows_kernel: enough rows in flight per column for few rows' latency.
int sum_rows_waves(int64_t rows) { return rows >= 128 ? 16 : rows >= 32 ? 8 : rows >= 8 ? 4 : 1; }

// ---- Channel side of the backward, d = 128: token side, U'/V'/dZ and the gate -------------
// Eight waves per workgroup, one workgroup per CU, persistent over units of 256 slots x one
// channel group (unit u: group u % q_c, slots 256 (u / q_c) + 32 wave .. for wave `wave`):
//   * P_u = A_u X', P_v = A_v X' from the wave's 32 X' rows, then dW' = A_o^T dY from its 32 dY
//     rows: the forward's block-diagonal token-side products (32x32x16 MFMAs), the X^T operands
//     by transposed LDS reads of the rows, which buffer_load ... lds copies into the wave's
//     swizzled tile (piece p of row r at slot p ^ tile128_swz(r)); P_u, P_v, dW' are stored;
//   * per 32-row chunk ec of the expanded dimension: U'^T = B_u''^T P_u^T, V'^T, dZ^T = B_o''
//     dW'^T (the chunk's 24 A-operand fragments of ow_pack_bwd_weights, shared by the eight
//     waves through three LDS buffers), the gate backward (as bwd_gate_kernel), and Z, dU', dV'
//     stored slot-major.
// The products that consume them (W' = Z B_o'', dP_u = dU' B_u''^T, dP_v = dV' B_v''^T, the
// slot reductions for dB and the token-matrix gradients) run after it.  Stores and copies are
// counted in vmcnt in issue order (explicit waits below).
constexpr int kB2D = 128;
constexpr int kB2KS = kB2D / 16;       // K steps over the channel group
constexpr int kB2FrA = 3 * kB2KS;      // A-operand fragments per chunk (24 KB)
constexpr int kB2Waves = 8;
constexpr int kB2Rows = 32 * kB2Waves;  // slots per unit
constexpr int kB2St = 40;               // staging row stride (elements) of the chunk outputs
static_assert(3 * 32 * kB2St <= 32 * kB2D, "the chunk outputs' staging fits in a wave's tile");

struct BwdChanArgs {
  const uint16_t* xt;   // [q_c][slots][128] X' tiles
  const uint16_t* dyt;  // [q_c][slots][128] dY tiles
  const float* a_u;     // [16][16] token matrices, fp32
  const float* a_v;
  const float* a_o;
  const uint16_t* packed;  // ow_pack_bwd_weights, d = 128
  uint16_t* pu;            // [q_c][slots][128]
  uint16_t* pv;
  uint16_t* dw;
  uint16_t* z;  // [q_c][slots][rd]
  uint16_t* du;
  uint16_t* dv;
  int64_t slots;
  int32_t q_c;
  // Routed rows (RT): x, dy [batch * n_tok][channels] read through the token table (group q is
  // channels 128 q .. 128 q + 127) instead of the xt, dyt tiles; the RMSNorm scales (rscale,
  // NULL: none) are folded into the token operands, as in the forward (A diag(r) x = A X').
  const uint16_t* x = nullptr;
  const uint16_t* dy = nullptr;
  const float* rscale = nullptr;
  const int32_t* tok = nullptr;  // [q_s * 16]
  int32_t q_s = 0, n_tok = 0, channels = 0;
};

// slot_row in 32-bit arithmetic, -1 also for sl >= slots (slots < 2^31 and batch * n_tok <
// 2^31: the callers check).
__device__ __forceinline__ int32_t slot_row32(const int32_t* tok, int64_t sl, int64_t slots, int32_t q_s,
                                              int32_t n_tok) {
  if (sl >= slots) return -1;
  const int32_t s32 = static_cast<int32_t>(sl), tg = s32 >> 4, b = tg / q_s, sg = tg - b * q_s;
  const int32_t tk = tok[sg * kG + (s32 & 15)];
  return (tk >= 0 && tk < n_tok) ? b * n_tok + tk : -1;
}

struct BwdChanLds {
  uint16_t x[kB2Waves][32 * kB2D];     // per wave: its 32 rows (X' or x, then dY)
  uint16_t w[3][kB2FrA * kFragElems];  // chunk buffers
  u32x4 tok[3][64];                    // A_u, A_v, A_o^T token-operand rows
  float rs[kB2Waves][32];              // RT: per wave, the RMSNorm scale of each slot
};

// out = the token-side product of one operand f (pair_token_side_mma for a single product).
template <class Ty, int KS>
__device__ __forceinline__ void token_side_one(const u32x4 (&xk)[KS / 2][2], u32x4 f, int lane, u32x4 (&out)[KS]) {
  const bool g0 = (lane & 16) == 0;
  const u32x4 f0 = keep_if(g0, f), f1 = keep_if(!g0, f);
  const f32x16 zero = {};
#pragma unroll
  for (int cb = 0; cb < KS / 2; ++cb) {
    f32x16 acc = Ty::mma32(xk[cb][0], f0, zero);
    acc = Ty::mma32(xk[cb][1], f1, acc);
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) out[2 * cb + s2] = pack_kstep<Ty>(acc, s2);
  }
}

template <class Ty, int RD, bool RT>
__global__ void __launch_bounds__(512) bwd_chan_d128_kernel(BwdChanArgs a, int32_t n_units) {
  constexpr int NCH = RD / 32;
  constexpr int CH = kB2FrA * kFragElems;                  // one chunk buffer (elements)
  constexpr int PACK_CH = bwd_frags(kB2D) * kFragElems;   // packed chunk stride (both operand halves)
  __shared__ __attribute__((aligned(16))) BwdChanLds sh;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hh = lane >> 5, l32 = lane & 31;
  const uint32_t lane16 = 16u * static_cast<uint32_t>(lane);
  const int64_t rows = a.slots * a.q_c;
  const uint32_t tbytes = static_cast<uint32_t>(rows * kB2D * 2), ebytes = static_cast<uint32_t>(rows * RD * 2);
  uint32_t xbytes = tbytes;  // RT: batch * n_tok * channels values of x and dy (below 2 GiB: host check)
  if constexpr (RT) xbytes = static_cast<uint32_t>(a.slots / (16 * a.q_s) * a.n_tok * a.channels * 2);
  const __amdgpu_buffer_rsrc_t rxt = buffer_rsrc(RT ? a.x : a.xt, xbytes), rdy = buffer_rsrc(RT ? a.dy : a.dyt, xbytes);
  const __amdgpu_buffer_rsrc_t rpu = buffer_rsrc(a.pu, tbytes), rpv = buffer_rsrc(a.pv, tbytes),
                               rdw = buffer_rsrc(a.dw, tbytes);
  const __amdgpu_buffer_rsrc_t rz = buffer_rsrc(a.z, ebytes), rdu = buffer_rsrc(a.du, ebytes),
                               rdv = buffer_rsrc(a.dv, ebytes);
  if (wave == 0) {
    sh.tok[0][lane] = token_frag<Ty, false>(a.a_u, lane);
    sh.tok[1][lane] = token_frag<Ty, false>(a.a_v, lane);
  } else if (wave == 1) {
    sh.tok[2][lane] = token_frag<Ty, true>(a.a_o, lane);
  }
  const uint32_t xlds = lds_addr(sh.x[wave]);

  for (int32_t u = blockIdx.x; u < n_units; u += gridDim.x) {
    const int q = u % a.q_c;
    const int64_t slot0 = static_cast<int64_t>(u / a.q_c) * kB2Rows + 32 * wave;
    const int64_t row0 = static_cast<int64_t>(q) * a.slots + slot0;
    // RT: the NHWC row of slot l32 (-1: pad) and its RMSNorm scale, for the wave's table.
    int32_t my_grow = -1;
    if constexpr (RT) {
      my_grow = slot_row32(a.tok, slot0 + l32, a.slots, a.q_s, a.n_tok);
      if (hh == 0) sh.rs[wave][l32] = (a.rscale && my_grow >= 0) ? a.rscale[my_grow] : 1.0f;
    }
    // Copy k: rows 4k .. 4k + 3 of the wave; lane -> row 4k + lane / 16, LDS slot lane % 16,
    // which holds the row's piece (lane % 16) ^ tile128_swz(row); rows past the slots read as zero.
    auto copy_tile = [&](__amdgpu_buffer_rsrc_t r) {
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int rr = 4 * k + (lane >> 4);
        const uint32_t piece = static_cast<uint32_t>((lane & 15) ^ tile128_swz(rr));
        uint32_t voff;
        if constexpr (RT) {
          const int32_t gr = __shfl(my_grow, rr);
          voff = gr >= 0 ? static_cast<uint32_t>(gr * a.channels + kB2D * q) * 2u + 16u * piece : kOffOut;
        } else {
          voff = slot0 + rr < a.slots
                     ? static_cast<uint32_t>(row0 + rr) * static_cast<uint32_t>(kB2D * 2) + 16u * piece
                     : kOffOut;
        }
        tile_copy(r, voff, xlds + static_cast<uint32_t>(4 * k * kB2D * 2));
      }
    };
    auto issue_chunk = [&](int ec) {
      const uint16_t* src = uniform_ptr(a.packed + (static_cast<size_t>(q) * NCH + ec) * PACK_CH);
      uint16_t* dst = sh.w[ec % 3];
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        const int f = wave + i * kB2Waves;
        copy_frag_to_lds(src + f * kFragElems, dst + f * kFragElems, lane16);
      }
    };
    auto at = [&](int r, int c) {
      return xlds + 2u * static_cast<uint32_t>(r * kB2D + (c ^ (8 * tile128_swz(r))));
    };
    // Lane (slot l32, hh) of K-step operand ks holds channels 16 ks + 4 hh + (0..3, 8..11).
    const int64_t my_row = row0 + l32;
    const bool my_ok = slot0 + l32 < a.slots;
    auto store_ops = [&](__amdgpu_buffer_rsrc_t r, const u32x4 (&v)[kB2KS]) {
#pragma unroll
      for (int ks = 0; ks < kB2KS; ++ks) {
        const uint32_t o = my_ok ? static_cast<uint32_t>(my_row * kB2D + 16 * ks + 4 * hh) * 2u : kOffOut;
        __builtin_amdgcn_raw_buffer_store_b64(u32x2{v[ks][0], v[ks][1]}, r, o, 0, 0);
        __builtin_amdgcn_raw_buffer_store_b64(u32x2{v[ks][2], v[ks][3]}, r, my_ok ? o + 16u : kOffOut, 0, 0);
      }
    };

    __syncthreads();  // the previous unit is done with the chunk buffers; tok is written
    copy_tile(rxt);    // 8 operations
    issue_chunk(0);    // 3
    issue_chunk(1);    // 3
    wait_vmcnt<6>();   // the X' rows (the chunk copies may be in flight)
    wave_lds_sync();
    u32x4 xk[kB2KS / 2][2];
    pair_xt_tr<kB2KS>(at, lane, xk);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the tile is read: the dY rows replace it
    copy_tile(rdy);  // 8
    u32x4 Pu[kB2KS], Pv[kB2KS], Dw[kB2KS];
    {
      u32x4 tu = sh.tok[0][lane], tv = sh.tok[1][lane];
      if constexpr (RT) {
        if (a.rscale) {  // A diag(r): the rows are x, not X'
          const float* r8 = &sh.rs[wave][16 * ((lane >> 4) & 1) + 4 * hh];
          tu = scale8<Ty>(tu, r8);
          tv = scale8<Ty>(tv, r8);
        }
      }
      pair_token_side_mma<Ty, kB2KS>(xk, tu, tv, lane, Pu, Pv);
    }
    store_ops(rpu, Pu);  // 16
    store_ops(rpv, Pv);  // 16
    wait_vmcnt<32>();    // the dY rows (and with them both chunk copies); the stores may be in flight
    wave_lds_sync();
    pair_xt_tr<kB2KS>(at, lane, xk);
    token_side_one<Ty, kB2KS>(xk, sh.tok[2][lane], lane, Dw);
    store_ops(rdw, Dw);  // 16

    // Chunk loop.  Step ec: [wait for chunk ec] [barrier] [copies of chunk ec + 2: 3] [products,
    // gate] [stores: 6].  Chunk ec >= 2 was copied at step ec - 2, and 6 + 3 + 6 operations
    // (6 + 6 without a copy at step ec - 1) were issued after it; chunks 0 and 1 landed before
    // the dY rows.
#pragma unroll 1
    for (int ec = 0; ec < NCH; ++ec) {
      if (ec >= 2) {
        if (ec + 1 < NCH)
          wait_vmcnt<15>();
        else
          wait_vmcnt<12>();
      }
      __syncthreads();  // chunk ec is in LDS for every wave; every wave is done with chunk ec - 1
      if (ec + 2 < NCH) issue_chunk(ec + 2);
      const u32x4* cf = reinterpret_cast<const u32x4*>(sh.w[ec % 3]);
      f32x16 U = {}, V = {}, G = {};
#pragma unroll
      for (int ks = 0; ks < kB2KS; ++ks) {
        U = Ty::mma32(cf[ks * (kFragElems / 8) + lane], Pu[ks], U);
        V = Ty::mma32(cf[(kB2KS + ks) * (kFragElems / 8) + lane], Pv[ks], V);
        G = Ty::mma32(cf[(2 * kB2KS + ks) * (kFragElems / 8) + lane], Dw[ks], G);
      }
      mfma_drain();
      f32x16 Z, DU, DV;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float up = U[i], vp = V[i], g = G[i];
        const float sg = gate_sigmoid(up);
        Z[i] = up * vp * sg;
        DU[i] = g * vp * sg * (1.0f - kLn2 * up * (1.0f - sg));
        DV[i] = g * up * sg;
      }
      // Registers 4b .. 4b + 3 are expanded rows 32 ec + 8b + 4hh + (0..3) of slot l32: staged
      // per wave as [32 slots][32 rows] (row stride kB2St) in the wave's tile, which the chunk
      // loop does not read, then stored as 64-byte row pieces (four lanes per slot).
      uint16_t* stg = sh.x[wave];
#pragma unroll
      for (int t = 0; t < 3; ++t) {
        const f32x16& m = t == 0 ? Z : t == 1 ? DU : DV;
#pragma unroll
        for (int b = 0; b < 4; ++b)
          *reinterpret_cast<u32x2*>(&stg[t * 32 * kB2St + l32 * kB2St + 8 * b + 4 * hh]) =
              u32x2{Ty::pack2(m[4 * b], m[4 * b + 1]), Ty::pack2(m[4 * b + 2], m[4 * b + 3])};
      }
      wave_lds_sync();
#pragma unroll
      for (int t = 0; t < 3; ++t) {
        const __amdgpu_buffer_rsrc_t r = t == 0 ? rz : t == 1 ? rdu : rdv;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int sl = 16 * h + (lane >> 2), part = lane & 3;
          const u32x4 v = *reinterpret_cast<const u32x4*>(&stg[t * 32 * kB2St + sl * kB2St + 8 * part]);
          const uint32_t o = slot0 + sl < a.slots
                                 ? static_cast<uint32_t>((row0 + sl) * RD + 32 * ec + 8 * part) * 2u
                                 : kOffOut;
          __builtin_amdgcn_raw_buffer_store_b128(v, r, o, 0, 0);
        }
      }
    }
  }
}

// ---- Channel side of the backward, d = 128, second part --------------------------------------
// Same units as bwd_chan_d128_kernel.  Per 32-slot pair (one per wave):
//   * pass 1 over the chunks of the expanded dimension: dP_u^T... as accumulators DPu[mb] +=
//     dU' B_u''^T, DPv[mb] += dV' B_v''^T (lane = channel 32 mb + l32, register i = slot
//     kord(i, hh)), the pair's dU', dV' chunk rows copied two chunks ahead into the wave's LDS
//     region (three buffers) and the chunk's B-operand fragments shared by the eight waves
//     (three LDS buffers);
//   * dX'^T = dP_u^T A_u + dP_v^T A_v with the operands swapped (lane = slot, registers =
//     channels), stored as 8-byte row pieces;
//   * dA_u += dP_u X'^T, dA_v += dP_v X'^T per 16-slot tile on 16x16x16 MFMAs over the channels:
//     dP rows by transposed LDS reads of dP staged channel-major, X' rows from memory;
//   * pass 2: W'[mb] += Z B_o'' from the Z chunk rows, then dA_o += dY W'^T the same way.
// The token-matrix gradients leave as per-workgroup fp32 partials (waves added in a fixed order).
struct BwdChan2Args {
  const uint16_t* xt;   // [q_c][slots][128]
  const uint16_t* dyt;
  const uint16_t* z;    // [q_c][slots][rd]
  const uint16_t* du;
  const uint16_t* dv;
  const float* a_u;     // [16][16] fp32
  const float* a_v;
  const uint16_t* packed;  // ow_pack_bwd_weights, d = 128
  uint16_t* dxt;           // [q_c][slots][128]
  float* partial;          // [gridDim][3][256]
  int64_t slots;
  int32_t q_c;
  // Routed (RT): X' and dY rows from x (times rscale, NULL: none, rounded as the gather) and dy
  // [batch * n_tok][channels], and dX' written to g, through the token table (group q is channels
  // 128 q .. 128 q + 127) instead of the xt, dyt, dxt tiles.
  const uint16_t* x = nullptr;
  const uint16_t* dy = nullptr;
  const float* rscale = nullptr;
  const int32_t* tok = nullptr;  // [q_s * 16]
  uint16_t* g = nullptr;
  int32_t q_s = 0, n_tok = 0, channels = 0;
};

constexpr int kB2FrB = 16;  // B-operand fragments of pass 1 per chunk (B_u''^T, B_v''^T)

// Rows in the wave's region are 64 bytes (32 values); their 16-byte pieces are XOR-swizzled so
// that the row-operand reads (one row per lane) and the staged dP / W' writes and transposed
// reads spread over the LDS banks: chunk rows (slot r) keep piece p at p ^ c2_rswz(r), the
// staged [128 channels][32 slots] set (channel c) at p ^ c2_sswz(c).
__device__ __forceinline__ int c2_rswz(int r) { return (r >> 2) & 3; }
__device__ __forceinline__ int c2_sswz(int c) { return (2 * ((c >> 2) & 1)) ^ ((c >> 3) & 1); }
constexpr int kB2RowBuf = 4096;  // bytes of one chunk-row buffer (pass 1: dU' then dV', 2 KB each)

struct BwdChan2Lds {
  uint16_t r[kB2Waves][3 * kB2RowBuf / 2];  // per wave: three chunk-row buffers; staged dP / W' in the first 8 KB
  uint16_t w[3][kB2FrB * kFragElems];      // chunk buffers
  u32x4 tok[2][64];                        // A_u^T, A_v^T token-operand rows
};
static_assert(kB2Waves * 3 * 256 * 4 <= sizeof(BwdChan2Lds::r), "the final dA sums fit in the row regions");

template <class Ty, int RD, bool RT>
__global__ void __launch_bounds__(512) bwd_chan2_d128_kernel(BwdChan2Args a, int32_t n_units) {
  constexpr int NCH = RD / 32;
  constexpr int MB = kB2D / 32;                            // 4 output blocks of 32 channels
  constexpr int PACK_CH = bwd_frags(kB2D) * kFragElems;   // packed chunk stride
  constexpr int OFF_BO = kB2FrA * kFragElems;              // B_o'' B operand within a packed chunk
  constexpr int OFF_BU = OFF_BO + 2 * MB * kFragElems;     // B_u''^T B operand (B_v''^T follows)
  __shared__ __attribute__((aligned(16))) BwdChan2Lds sh;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hh = lane >> 5, l32 = lane & 31, l16 = lane & 15, h4 = lane >> 4;
  const bool g0 = (lane & 16) == 0;
  const uint32_t lane16 = 16u * static_cast<uint32_t>(lane);
  const int64_t rows = a.slots * a.q_c;
  const uint32_t tbytes = static_cast<uint32_t>(rows * kB2D * 2), ebytes = static_cast<uint32_t>(rows * RD * 2);
  uint32_t gbytes = tbytes;  // RT: batch * n_tok * channels values of x, dy, g (below 2 GiB: host check)
  if constexpr (RT) gbytes = static_cast<uint32_t>(a.slots / (16 * a.q_s) * a.n_tok * a.channels * 2);
  const __amdgpu_buffer_rsrc_t rxt = buffer_rsrc(RT ? a.x : a.xt, gbytes), rdy = buffer_rsrc(RT ? a.dy : a.dyt, gbytes),
                               rdx = buffer_rsrc(RT ? a.g : a.dxt, gbytes);
  const __amdgpu_buffer_rsrc_t rz = buffer_rsrc(a.z, ebytes), rdu = buffer_rsrc(a.du, ebytes),
                               rdv = buffer_rsrc(a.dv, ebytes);
  if (wave == 0) {
    sh.tok[0][lane] = token_frag<Ty, true>(a.a_u, lane);
    sh.tok[1][lane] = token_frag<Ty, true>(a.a_v, lane);
  }
  const uint32_t rlds = lds_addr(sh.r[wave]);
  f32x4 dA[3] = {};

  for (int32_t u = blockIdx.x; u < n_units; u += gridDim.x) {
    const int q = u % a.q_c;
    const int64_t slot0 = static_cast<int64_t>(u / a.q_c) * kB2Rows + 32 * wave;
    const int64_t row0 = static_cast<int64_t>(q) * a.slots + slot0;
    const uint16_t* pk = a.packed + static_cast<size_t>(q) * NCH * PACK_CH;
    // Chunk rows of one [slots][RD] tensor (32 slots x 32 values, 2 KB) into the wave's region
    // at byte offset `at`: two copies, lane -> slot 16 c + lane / 4, LDS piece lane % 4 holding
    // the row's piece (lane % 4) ^ c2_rswz(slot).
    auto copy_rows = [&](__amdgpu_buffer_rsrc_t r, int ec, uint32_t at) {
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const int sl = 16 * c + (lane >> 2);
        const int pc = (lane & 3) ^ c2_rswz(sl);
        const uint32_t voff =
            slot0 + sl < a.slots ? static_cast<uint32_t>((row0 + sl) * RD + 32 * ec + 8 * pc) * 2u : kOffOut;
        tile_copy(r, voff, rlds + at + 1024u * c);
      }
    };
    // K-step operand s of a staged chunk (lane (slot l32, hh): values 16 s + 4 hh + 0..3 and + 8,
    // the 8-byte halves hh of pieces 2 s and 2 s + 1).
    auto row_op = [&](uint32_t at, int s2) {
      const uint16_t* base = sh.r[wave] + at / 2 + l32 * 32 + 4 * hh;
      const int sw = c2_rswz(l32);
      const u32x2 lo = *reinterpret_cast<const u32x2*>(base + 8 * ((2 * s2) ^ sw));
      const u32x2 hi = *reinterpret_cast<const u32x2*>(base + 8 * ((2 * s2 + 1) ^ sw));
      return u32x4{lo[0], lo[1], hi[0], hi[1]};
    };
    auto copy_w = [&](int ec, int off, int nfr) {  // nfr / 8 fragments per wave
      const uint16_t* src = uniform_ptr(pk + static_cast<size_t>(ec) * PACK_CH + off);
      uint16_t* dst = sh.w[ec % 3];
      for (int i = 0; i < nfr / kB2Waves; ++i) {
        const int f = wave + i * kB2Waves;
        copy_frag_to_lds(src + f * kFragElems, dst + f * kFragElems, lane16);
      }
    };
    // Stage an accumulator set (lane = channel 32 mb + l32, register 4b + k = slot 8b + 4hh + k)
    // channel-major: region [128 channels][32 slots], bf16.
    auto stage = [&](const f32x16 (&m)[MB]) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const int c = 32 * mb + l32;
#pragma unroll
        for (int b = 0; b < 4; ++b)
          *reinterpret_cast<u32x2*>(&sh.r[wave][c * 32 + 8 * (b ^ c2_sswz(c)) + 4 * hh]) =
              u32x2{Ty::pack2(m[mb][4 * b], m[mb][4 * b + 1]), Ty::pack2(m[mb][4 * b + 2], m[mb][4 * b + 3])};
      }
      wave_lds_sync();
    };
    // Rows 16 g + l16, channels 16 ks + 4 h4 .. + 3 of the staged set, by transposed reads (the
    // 16x16x16 operand: lane (t = l16, h4)); the lane's address: channel 16 ks + 4 h4 + l16 / 4,
    // slots 16 g + 4 (l16 % 4) .. + 3.
    auto staged_op = [&](int g, int ks) {
      const int c = 16 * ks + 4 * h4 + (l16 >> 2), sl = 16 * g + 4 * (l16 & 3);
      const uint32_t addr = rlds + 2u * static_cast<uint32_t>(c * 32 + 8 * ((sl >> 3) ^ c2_sswz(c)) + (sl & 7));
      return lds_read_tr16(addr);
    };
    // RT: the NHWC rows of the lane's slots 16 g + l16 (g < 2) and, for X', their RMSNorm scales.
    int32_t grow[2] = {-1, -1};
    float grs[2] = {1.0f, 1.0f};
    if constexpr (RT) {
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        grow[g] = slot_row32(a.tok, slot0 + 16 * g + l16, a.slots, a.q_s, a.n_tok);
        if (a.rscale && grow[g] >= 0) grs[g] = a.rscale[grow[g]];
      }
    }
    // Rows 16 g + l16 of a [slots][128] tensor, channels 16 ks + 4 h4 .. + 3 (zero past the slots);
    // RT: of x or dy (the loads only: x_scaled forms X' as the gather does).
    auto mem_op = [&](__amdgpu_buffer_rsrc_t r, int g, int ks) {
      uint32_t o;
      if constexpr (RT)
        o = grow[g] >= 0 ? static_cast<uint32_t>(grow[g] * a.channels + kB2D * q + 16 * ks + 4 * h4) * 2u : kOffOut;
      else
        o = slot0 + 16 * g + l16 < a.slots
                ? static_cast<uint32_t>((row0 + 16 * g + l16) * kB2D + 16 * ks + 4 * h4) * 2u
                : kOffOut;
      return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, o, 0, 0));
    };
    auto x_scaled = [&](u32x2 v, int g) {
      if constexpr (RT) {
        if (a.rscale) v = u32x2{scale2<Ty>(v[0], grs[g]), scale2<Ty>(v[1], grs[g])};
      }
      return v;
    };

    __syncthreads();  // the previous unit is done with every buffer; tok is written
    // Pass 1.  Step ec: [wait: chunk ec's rows and fragments] [barrier] [rows and fragments of
    // ec + 2: 4 + 2] [products].  Chunk ec + 1's copies may be in flight (6, none at the last step).
    copy_rows(rdu, 0, 0);
    copy_rows(rdv, 0, 2048);
    copy_w(0, OFF_BU, kB2FrB);
    if (NCH > 1) {
      copy_rows(rdu, 1, kB2RowBuf);
      copy_rows(rdv, 1, kB2RowBuf + 2048);
      copy_w(1, OFF_BU, kB2FrB);
    }
    f32x16 DPu[MB], DPv[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      DPu[mb] = f32x16{};
      DPv[mb] = f32x16{};
    }
#pragma unroll 1
    for (int ec = 0; ec < NCH; ++ec) {
      if (ec + 1 < NCH)
        wait_vmcnt<6>();
      else
        wait_vmcnt<0>();
      __syncthreads();  // chunk ec is in LDS for every wave; every wave is done with chunk ec - 1
      const uint32_t cur = kB2RowBuf * (ec % 3), nxt2 = kB2RowBuf * ((ec + 2) % 3);
      if (ec + 2 < NCH) {
        copy_rows(rdu, ec + 2, nxt2);
        copy_rows(rdv, ec + 2, nxt2 + 2048);
        copy_w(ec + 2, OFF_BU, kB2FrB);
      }
      const u32x4* cf = reinterpret_cast<const u32x4*>(sh.w[ec % 3]);
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        const u32x4 opu = row_op(cur, s2), opv = row_op(cur + 2048, s2);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          DPu[mb] = Ty::mma32(opu, cf[(2 * mb + s2) * (kFragElems / 8) + lane], DPu[mb]);
          DPv[mb] = Ty::mma32(opv, cf[(2 * MB + 2 * mb + s2) * (kFragElems / 8) + lane], DPv[mb]);
        }
      }
    }
    mfma_drain();

    // dX'^T = dP_u^T A_u + dP_v^T A_v: lane = slot l32, registers 4b .. 4b + 3 = channels 32 mb +
    // 8 b + 4 hh .. + 3.
    {
      const u32x4 tu = sh.tok[0][lane], tv = sh.tok[1][lane];
      const u32x4 tu0 = keep_if(g0, tu), tu1 = keep_if(!g0, tu);
      const u32x4 tv0 = keep_if(g0, tv), tv1 = keep_if(!g0, tv);
      const bool ok = slot0 + l32 < a.slots;
      // Byte offset of the lane's slot row in the output: dxt row, or (RT) the NHWC row of its
      // token at group q's columns (kOffOut for pad slots: the stores are dropped).
      uint32_t obase = kOffOut;
      if constexpr (RT) {
        const int32_t gr = slot_row32(a.tok, slot0 + l32, a.slots, a.q_s, a.n_tok);
        if (gr >= 0) obase = static_cast<uint32_t>(gr * a.channels + kB2D * q) * 2u;
      } else if (ok) {
        obase = static_cast<uint32_t>((row0 + l32) * kB2D) * 2u;
      }
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        f32x16 dx = Ty::mma32(pack_kstep<Ty>(DPu[mb], 0), tu0, f32x16{});
        dx = Ty::mma32(pack_kstep<Ty>(DPu[mb], 1), tu1, dx);
        dx = Ty::mma32(pack_kstep<Ty>(DPv[mb], 0), tv0, dx);
        dx = Ty::mma32(pack_kstep<Ty>(DPv[mb], 1), tv1, dx);
        mfma_drain();
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const uint32_t o = obase == kOffOut ? kOffOut : obase + 2u * static_cast<uint32_t>(32 * mb + 8 * b + 4 * hh);
          __builtin_amdgcn_raw_buffer_store_b64(u32x2{Ty::pack2(dx[4 * b], dx[4 * b + 1]), Ty::pack2(dx[4 * b + 2], dx[4 * b + 3])},
                                                rdx, o, 0, 0);
        }
      }
    }
    // dA_u, dA_v: the X rows requested before the staging of dP_u.
    u32x2 xo[2][kB2KS];
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int ks = 0; ks < kB2KS; ++ks) xo[g][ks] = mem_op(rxt, g, ks);
    stage(DPu);
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int ks = 0; ks < kB2KS; ++ks) xo[g][ks] = x_scaled(xo[g][ks], g);
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int ks = 0; ks < kB2KS; ++ks) dA[0] = Ty::mma16(staged_op(g, ks), xo[g][ks], dA[0]);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    stage(DPv);
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int ks = 0; ks < kB2KS; ++ks) dA[1] = Ty::mma16(staged_op(g, ks), xo[g][ks], dA[1]);
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");  // nothing in flight before pass 2's copies

    // Pass 2: W'[mb] += Z B_o''; [wait] [barrier] [Z rows and fragments of ec + 2: 2 + 1].
    __syncthreads();  // every wave is done with pass 1's chunk buffers
    copy_rows(rz, 0, 0);
    copy_w(0, OFF_BO, 2 * MB);
    if (NCH > 1) {
      copy_rows(rz, 1, kB2RowBuf);
      copy_w(1, OFF_BO, 2 * MB);
    }
    f32x16 W[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) W[mb] = f32x16{};
#pragma unroll 1
    for (int ec = 0; ec < NCH; ++ec) {
      if (ec + 1 < NCH)
        wait_vmcnt<3>();
      else
        wait_vmcnt<0>();
      __syncthreads();
      const uint32_t cur = kB2RowBuf * (ec % 3), nxt2 = kB2RowBuf * ((ec + 2) % 3);
      if (ec + 2 < NCH) {
        copy_rows(rz, ec + 2, nxt2);
        copy_w(ec + 2, OFF_BO, 2 * MB);
      }
      const u32x4* cf = reinterpret_cast<const u32x4*>(sh.w[ec % 3]);
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        const u32x4 opz = row_op(cur, s2);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) W[mb] = Ty::mma32(opz, cf[(2 * mb + s2) * (kFragElems / 8) + lane], W[mb]);
      }
    }
    mfma_drain();
    // dA_o = dY W'^T: A = dY rows from memory, B = staged W' rows.
    u32x2 yo[2][kB2KS];
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int ks = 0; ks < kB2KS; ++ks) yo[g][ks] = mem_op(rdy, g, ks);
    stage(W);
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int ks = 0; ks < kB2KS; ++ks) dA[2] = Ty::mma16(yo[g][ks], staged_op(g, ks), dA[2]);
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
  }

  // The workgroup's dA sums, waves added in order (in the row regions, which every wave is done
  // with after the barrier).
  mfma_drain();
  __syncthreads();
  float(*red)[3][256] = reinterpret_cast<float(*)[3][256]>(&sh.r[0][0]);
#pragma unroll
  for (int m = 0; m < 3; ++m)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[wave][m][(4 * h4 + i) * 16 + l16] = dA[m][i];
  __syncthreads();
  for (int e = threadIdx.x; e < 3 * 256; e += 512) {
    const int m = e >> 8, k = e & 255;
    float v = 0.0f;
    for (int w = 0; w < kB2Waves; ++w) v += red[w][m][k];
    a.partial[static_cast<int64_t>(blockIdx.x) * 768 + e] = v;
  }
}

template <int RD>
int launch_bwd_chan2_rd(const BwdChan2Args& a, int64_t grid, int32_t n_units, int32_t dtype, hipStream_t s) {
  const dim3 g(static_cast<unsigned>(grid));
  if (dtype == OW_DTYPE_BF16) {
    if (a.tok)
      hipLaunchKernelGGL((bwd_chan2_d128_kernel<BF16, RD, true>), g, dim3(512), 0, s, a, n_units);
    else
      hipLaunchKernelGGL((bwd_chan2_d128_kernel<BF16, RD, false>), g, dim3(512), 0, s, a, n_units);
  } else {
    if (a.tok)
      hipLaunchKernelGGL((bwd_chan2_d128_kernel<F16, RD, true>), g, dim3(512), 0, s, a, n_units);
    else
      hipLaunchKernelGGL((bwd_chan2_d128_kernel<F16, RD, false>), g, dim3(512), 0, s, a, n_units);
  }
  return hip_status(hipGetLastError(), "bwd_chan2_d128_kernel launch");
}

// Workgroups of the d = 128 backward kernels for `units` units: one per CU (a multiple of 8
// with more units than CUs), one per unit otherwise.
int64_t bwd_chan_grid(int64_t units) {
  int64_t grid = device_cus();
  if (grid >= units) return units;
  if (grid >= 8) grid -= grid % 8;
  return grid;
}

template <int RD>
int launch_bwd_chan_rd(const BwdChanArgs& a, int32_t n_units, int32_t dtype, hipStream_t s) {
  const dim3 g(static_cast<unsigned>(bwd_chan_grid(n_units)));
  if (dtype == OW_DTYPE_BF16) {
    if (a.tok)
      hipLaunchKernelGGL((bwd_chan_d128_kernel<BF16, RD, true>), g, dim3(512), 0, s, a, n_units);
    else
      hipLaunchKernelGGL((bwd_chan_d128_kernel<BF16, RD, false>), g, dim3(512), 0, s, a, n_units);
  } else {
    if (a.tok)
      hipLaunchKernelGGL((bwd_chan_d128_kernel<F16, RD, true>), g, dim3(512), 0, s, a, n_units);
    else
      hipLaunchKernelGGL((bwd_chan_d128_kernel<F16, RD, false>), g, dim3(512), 0, s, a, n_units);
  }
  return hip_status(hipGetLastError(), "bwd_chan_d128_kernel launch");
}

unsigned blocks_for(int64_t n) { return static_cast<unsigned>((n + 255) / 256); }

// out[b][i] = round(x[b][i] * scale[b]): the upstream gradient of the delta branch under
// per-sample drop-path (omniweave/models/block.py:99-107; the autograd of delta * keep_mask /
// keep_probability multiplies the gradient by the same per-image factor and rounds once).
// V = 8 elements per thread (16-bit types, 16-byte accesses) or V = 1.
template <class Ty, int V>
__global__ void __launch_bounds__(256) scale_samples_kernel(const uint16_t* x, const float* scale, uint16_t* out,
                                                            int64_t per_sample, int64_t total) {
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * V;
  if (i >= total) return;
  const float sc = scale[i / per_sample];
  if constexpr (V == 8) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(x + i);
    u32x4 o;
#pragma unroll
    for (int w = 0; w < 4; ++w) o[w] = Ty::pack2(Ty::to_f32(lo16(v[w])) * sc, Ty::to_f32(hi16(v[w])) * sc);
    *reinterpret_cast<u32x4*>(out + i) = o;
  } else {
    out[i] = Ty::from_f32(Ty::to_f32(x[i]) * sc);
  }
}

__global__ void __launch_bounds__(256) scale_samples_f32_kernel(const float* x, const float* scale, float* out,
                                                                int64_t per_sample, int64_t total) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < total) out[i] = x[i] * scale[i / per_sample];
}

}  // namespace
}  // namespace ow

extern "C" {

int ow_scale_samples(const void* x, const float* scale, void* out, int32_t batch, int64_t per_sample, int32_t dtype,
                     void* stream) {
  OW_CHECK_ARG(batch >= 0 && per_sample >= 0, "bad shape batch=%d per_sample=%lld", batch, (long long)per_sample);
  OW_CHECK_SUPPORTED(dtype == OW_DTYPE_BF16 || dtype == OW_DTYPE_F16 || dtype == OW_DTYPE_F32, "unsupported dtype %d",
                     dtype);
  const int64_t total = static_cast<int64_t>(batch) * per_sample;
  if (total == 0) {
    ow::clear_error();
    return OW_OK;
  }
  OW_CHECK_ARG(x && scale && out, "tensor pointer is NULL");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == OW_DTYPE_F32) {
    hipLaunchKernelGGL(ow::scale_samples_f32_kernel, dim3(ow::blocks_for(total)), dim3(256), 0, s,
                       static_cast<const float*>(x), scale, static_cast<float*>(out), per_sample, total);
  } else {
    const auto* xi = static_cast<const uint16_t*>(x);
    auto* oi = static_cast<uint16_t*>(out);
    const bool vec = per_sample % 8 == 0 && ow::aligned16(x) && ow::aligned16(out);
    const unsigned blocks = ow::blocks_for(vec ? total / 8 : total);
    if (dtype == OW_DTYPE_BF16) {
      if (vec)
        hipLaunchKernelGGL((ow::scale_samples_kernel<ow::BF16, 8>), dim3(blocks), dim3(256), 0, s, xi, scale, oi,
                           per_sample, total);
      else
        hipLaunchKernelGGL((ow::scale_samples_kernel<ow::BF16, 1>), dim3(blocks), dim3(256), 0, s, xi, scale, oi,
                           per_sample, total);
    } else {
      if (vec)
        hipLaunchKernelGGL((ow::scale_samples_kernel<ow::F16, 8>), dim3(blocks), dim3(256), 0, s, xi, scale, oi,
                           per_sample, total);
      else
        hipLaunchKernelGGL((ow::scale_samples_kernel<ow::F16, 1>), dim3(blocks), dim3(256), 0, s, xi, scale, oi,
                           per_sample, total);
    }
  }
  if (int rc = ow::hip_status(hipGetLastError(), "scale_samples_kernel launch")) return rc;
  ow::clear_error();
  return OW_OK;
}

int ow_bwd_gather(const void* x, const void* dy, const float* rscale, const int32_t* token_index,
                  const int32_t* channel_index, const OwPlan* plan, int32_t batch, int32_t dtype, void* xt, void* dyt,
                  void* stream) {
  int32_t q_s = 0, q_c = 0;
  if (int rc = ow_plan_dims(plan, &q_s, &q_c)) return rc;
  OW_CHECK_ARG(batch >= 0, "batch must be >= 0 (got %d)", batch);
  OW_CHECK_SUPPORTED(plan->spatial_tile == ow::kG, "unsupported spatial tile g=%d; expected 16", plan->spatial_tile);
  OW_CHECK_SUPPORTED(dtype == OW_DTYPE_BF16 || dtype == OW_DTYPE_F16 || dtype == OW_DTYPE_F32, "unsupported dtype %d",
                     dtype);
  if (batch == 0) {
    ow::clear_error();
    return OW_OK;
  }
  OW_CHECK_ARG(x && dy && token_index && channel_index && xt && dyt, "tensor pointer is NULL");
  if (dtype == OW_DTYPE_F32) {
    if (int rc = ow::bwd_gather_f32(static_cast<const float*>(x), static_cast<const float*>(dy), rscale, token_index,
                                    channel_index, static_cast<float*>(xt), static_cast<float*>(dyt),
                                    static_cast<int64_t>(batch) * q_s * ow::kG, plan->height * plan->width,
                                    plan->channels, q_s, q_c, plan->channel_tile, static_cast<hipStream_t>(stream)))
      return rc;
    ow::clear_error();
    return OW_OK;
  }
  OW_CHECK_SUPPORTED(plan->channel_tile % 8 == 0, "channel tile %d is not a multiple of 8", plan->channel_tile);
  OW_CHECK_ARG(ow::aligned16(xt) && ow::aligned16(dyt), "xt / dyt must be 16-byte aligned");
  const int32_t vec = plan->channels % 8 == 0 && ow::aligned16(x) && ow::aligned16(dy);
  ow::GatherArgs a{static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(dy), rscale, token_index,
                   channel_index, static_cast<uint16_t*>(xt), static_cast<uint16_t*>(dyt),
                   static_cast<int64_t>(batch) * q_s * ow::kG, plan->height * plan->width, plan->channels, q_s,
                   plan->channel_tile, vec};
  const int64_t total8 = static_cast<int64_t>(q_c) * a.slots * (a.d / 8);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == OW_DTYPE_BF16)
    hipLaunchKernelGGL(ow::bwd_gather_kernel<ow::BF16>, dim3(ow::blocks_for(total8)), dim3(256), 0, s, a, total8);
  else
    hipLaunchKernelGGL(ow::bwd_gather_kernel<ow::F16>, dim3(ow::blocks_for(total8)), dim3(256), 0, s, a, total8);
  if (int rc = ow::hip_status(hipGetLastError(), "bwd_gather_kernel launch")) return rc;
  ow::clear_error();
  return OW_OK;
}

int ow_bwd_gate(const void* u, const void* v, const void* dz, void* z, void* du, void* dv, int64_t n, int32_t dtype,
                void* stream) {
  OW_CHECK_ARG(n >= 0, "n must be >= 0");
  OW_CHECK_SUPPORTED(dtype == OW_DTYPE_BF16 || dtype == OW_DTYPE_F16 || dtype == OW_DTYPE_F32, "unsupported dtype %d",
                     dtype);
  if (n == 0) {
    ow::clear_error();
    return OW_OK;
  }
  OW_CHECK_ARG(u && v && dz && z && du && dv, "tensor pointer is NULL");
  if (dtype == OW_DTYPE_F32) {
    if (int rc = ow::bwd_gate_f32(static_cast<const float*>(u), static_cast<const float*>(v),
                                  static_cast<const float*>(dz), static_cast<float*>(z), static_cast<float*>(du),
                                  static_cast<float*>(dv), n, static_cast<hipStream_t>(stream)))
      return rc;
    ow::clear_error();
    return OW_OK;
  }
  OW_CHECK_ARG(n % 8 == 0, "n must be a multiple of 8 (got %lld)", (long long)n);
  OW_CHECK_ARG(ow::aligned16(u) && ow::aligned16(v) && ow::aligned16(dz) && ow::aligned16(z) && ow::aligned16(du) &&
                   ow::aligned16(dv),
               "gate buffers must be 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto cu = [](const void* p) { return static_cast<const uint16_t*>(p); };
  auto mu = [](void* p) { return static_cast<uint16_t*>(p); };
  const int64_t n8 = n / 8;
  if (dtype == OW_DTYPE_BF16)
    hipLaunchKernelGGL(ow::bwd_gate_kernel<ow::BF16>, dim3(ow::blocks_for(n8)), dim3(256), 0, s, cu(u), cu(v), cu(dz),
                       mu(z), mu(du), mu(dv), n8);
  else
    hipLaunchKernelGGL(ow::bwd_gate_kernel<ow::F16>, dim3(ow::blocks_for(n8)), dim3(256), 0, s, cu(u), cu(v), cu(dz),
                       mu(z), mu(du), mu(dv), n8);
  if (int rc = ow::hip_status(hipGetLastError(), "bwd_gate_kernel launch")) return rc;
  ow::clear_error();
  return OW_OK;
}

int ow_bwd_scatter(const void* dxt, const int32_t* token_index, const int32_t* channel_index, const OwPlan* plan,
                   int32_t batch, int32_t dtype, void* g, void* stream) {
  int32_t q_s = 0, q_c = 0;
  if (int rc = ow_plan_dims(plan, &q_s, &q_c)) return rc;
  OW_CHECK_ARG(batch >= 0, "batch must be >= 0 (got %d)", batch);
  OW_CHECK_SUPPORTED(dtype == OW_DTYPE_BF16 || dtype == OW_DTYPE_F16 || dtype == OW_DTYPE_F32, "unsupported dtype %d",
                     dtype);
  if (batch == 0) {
    ow::clear_error();
    return OW_OK;
  }
  OW_CHECK_ARG(dxt && token_index && channel_index && g, "tensor pointer is NULL");
  if (dtype == OW_DTYPE_F32) {
    if (int rc = ow::bwd_scatter_f32(static_cast<const float*>(dxt), token_index, channel_index, static_cast<float*>(g),
                                     static_cast<int64_t>(batch) * q_s * ow::kG, plan->height * plan->width,
                                     plan->channels, q_s, q_c, plan->channel_tile, static_cast<hipStream_t>(stream)))
      return rc;
    ow::clear_error();
    return OW_OK;
  }
  OW_CHECK_SUPPORTED(plan->channel_tile % 8 == 0, "channel tile %d is not a multiple of 8", plan->channel_tile);
  OW_CHECK_ARG(ow::aligned16(dxt), "dxt must be 16-byte aligned");
  const int64_t slots = static_cast<int64_t>(batch) * q_s * ow::kG;
  const int32_t d = plan->channel_tile;
  const int64_t total8 = static_cast<int64_t>(q_c) * slots * (d / 8);
  const int32_t vec = plan->channels % 8 == 0 && ow::aligned16(g);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint16_t* src = static_cast<const uint16_t*>(dxt);
  const int32_t n_tok = plan->height * plan->width;
  hipLaunchKernelGGL(ow::bwd_scatter_kernel, dim3(ow::blocks_for(total8)), dim3(256), 0, s, src, token_index,
                     channel_index, static_cast<uint16_t*>(g), slots, n_tok, plan->channels, q_s, d, vec, total8);
  if (int rc = ow::hip_status(hipGetLastError(), "bwd_scatter_kernel launch")) return rc;
  ow::clear_error();
  return OW_OK;
}

int ow_bwd_rmsnorm(const void* x, const void* g, const float* rscale, const void* dout, void* dx, int64_t rows,
                   int32_t channels, int32_t residual, int32_t dtype, void* stream) {
  OW_CHECK_ARG(rows >= 0 && channels >= 1, "bad shape rows=%lld channels=%d", (long long)rows, channels);
  OW_CHECK_SUPPORTED(dtype == OW_DTYPE_BF16 || dtype == OW_DTYPE_F16 || dtype == OW_DTYPE_F32, "unsupported dtype %d",
                     dtype);
  if (rows == 0) {
    ow::clear_error();
    return OW_OK;
  }
  OW_CHECK_ARG(x && g && dx && (!residual || dout), "tensor pointer is NULL");
  if (dtype == OW_DTYPE_F32) {
    if (int rc = ow::bwd_rmsnorm_f32(static_cast<const float*>(x), static_cast<const float*>(g), rscale,
                                     static_cast<const float*>(dout),
                                     static_cast<float*>(dx), rows, channels, residual,
                                     static_cast<hipStream_t>(stream)))
      return rc;
    ow::clear_error();
    return OW_OK;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto cu = [](const void* p) { return static_cast<const uint16_t*>(p); };
  uint16_t* out = static_cast<uint16_t*>(dx);
  const bool vec = channels % 8 == 0 && ow::aligned16(x) && ow::aligned16(g) && ow::aligned16(dx) &&
                   (!residual || ow::aligned16(dout));
  if (!vec) {
    const unsigned blocks = static_cast<unsigned>((rows + 3) / 4);
    if (dtype == OW_DTYPE_BF16)
      hipLaunchKernelGGL(ow::bwd_rmsnorm_scalar_kernel<ow::BF16>, dim3(blocks), dim3(256), 0, s, cu(x), cu(g), rscale,
                         cu(dout), out, rows, channels, residual);
    else
      hipLaunchKernelGGL(ow::bwd_rmsnorm_scalar_kernel<ow::F16>, dim3(blocks), dim3(256), 0, s, cu(x), cu(g), rscale,
                         cu(dout), out, rows, channels, residual);
  } else {
    int32_t lpr = 1;
    while (lpr < 64 && lpr * 8 < channels) lpr *= 2;
    const int64_t rows_per_block = 4 * (64 / lpr);
    const unsigned blocks = static_cast<unsigned>((rows + rows_per_block - 1) / rows_per_block);
    if (dtype == OW_DTYPE_BF16)
      hipLaunchKernelGGL(ow::bwd_rmsnorm_kernel<ow::BF16>, dim3(blocks), dim3(256), 0, s, cu(x), cu(g), rscale, cu(dout),
                         out, rows, channels, residual, lpr);
    else
      hipLaunchKernelGGL(ow::bwd_rmsnorm_kernel<ow::F16>, dim3(blocks), dim3(256), 0, s, cu(x), cu(g), rscale, cu(dout),
                         out, rows, channels, residual, lpr);
  }
  if (int rc = ow::hip_status(hipGetLastError(), "bwd_rmsnorm_kernel launch")) return rc;
  ow::clear_error();
  return OW_OK;
}

int ow_fold_weights(const void* b_u, const void* b_v, const void* b_o, int32_t weight_dtype, const float* norm_weight,
                    const float* gamma, const int32_t* channel_index, int32_t channels, int32_t q_c, int32_t d,
                    int32_t rd, int32_t compute_dtype, void* bu, void* bu_t, void* bv, void* bv_t, void* bo,
                    void* bo_t, void* stream) {
  OW_CHECK_ARG(b_u && b_v && b_o && channel_index && bu && bu_t && bv && bv_t && bo && bo_t, "tensor pointer is NULL");
  OW_CHECK_ARG(q_c >= 1 && d >= 1 && rd >= 1 && channels >= 1, "bad shape q_c=%d d=%d rd=%d C=%d", q_c, d, rd, channels);
  OW_CHECK_ARG(weight_dtype >= OW_DTYPE_F32 && weight_dtype <= OW_DTYPE_F16, "unknown weight dtype %d", weight_dtype);
  OW_CHECK_SUPPORTED(compute_dtype == OW_DTYPE_BF16 || compute_dtype == OW_DTYPE_F16 || compute_dtype == OW_DTYPE_F32,
                     "unsupported compute dtype %d", compute_dtype);
  if (compute_dtype == OW_DTYPE_F32) {
    auto mf = [](void* p) { return static_cast<float*>(p); };
    if (int rc = ow::fold_weights_f32(b_u, b_v, b_o, weight_dtype, norm_weight, gamma, channel_index, channels, q_c, d,
                                      rd, mf(bu), mf(bu_t), mf(bv), mf(bv_t), mf(bo), mf(bo_t),
                                      static_cast<hipStream_t>(stream)))
      return rc;
    ow::clear_error();
    return OW_OK;
  }
  auto mu = [](void* p) { return static_cast<uint16_t*>(p); };
  ow::FoldArgs a{b_u, b_v, b_o, norm_weight, gamma, channel_index, mu(bu), mu(bu_t), mu(bv), mu(bv_t), mu(bo), mu(bo_t),
                 weight_dtype, q_c, d, rd, channels};
  const int64_t total = static_cast<int64_t>(q_c) * d * rd;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (compute_dtype == OW_DTYPE_BF16)
    hipLaunchKernelGGL(ow::fold_weights_kernel<ow::BF16>, dim3(ow::blocks_for(total)), dim3(256), 0, s, a, total);
  else
    hipLaunchKernelGGL(ow::fold_weights_kernel<ow::F16>, dim3(ow::blocks_for(total)), dim3(256), 0, s, a, total);
  if (int rc = ow::hip_status(hipGetLastError(), "fold_weights_kernel launch")) return rc;
  ow::clear_error();
  return OW_OK;
}

int ow_tile_mix(const void* in1, const float* m1, const void* in2, const float* m2, void* out, int64_t n_tiles,
                int32_t d, int32_t dtype, void* stream) {
  OW_CHECK_ARG(n_tiles >= 0, "bad tile count %lld", (long long)n_tiles);
  OW_CHECK_SUPPORTED(d == 64 || d == 128, "unsupported channel tile d=%d; expected 64 or 128", d);
  OW_CHECK_SUPPORTED(dtype == OW_DTYPE_BF16 || dtype == OW_DTYPE_F16 || dtype == OW_DTYPE_F32, "unsupported dtype %d",
                     dtype);
  if (n_tiles == 0) {
    ow::clear_error();
    return OW_OK;
  }
  OW_CHECK_ARG(in1 && m1 && out && (!in2 == !m2), "tensor pointer is NULL");
  if (dtype == OW_DTYPE_F32) {
    if (int rc = ow::tile_mix_f32(static_cast<const float*>(in1), m1, static_cast<const float*>(in2), m2,
                                  static_cast<float*>(out), n_tiles, d, static_cast<hipStream_t>(stream)))
      return rc;
    ow::clear_error();
    return OW_OK;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const unsigned blocks = static_cast<unsigned>((n_tiles + 3) / 4);
  auto cu = [](const void* p) { return static_cast<const uint16_t*>(p); };
  uint16_t* o = static_cast<uint16_t*>(out);
#define OW_TILE_MIX(TY, TWO, NB)                                                                               \
  hipLaunchKernelGGL((ow::tile_mix_kernel<TY, TWO, NB>), dim3(blocks), dim3(256), 0, s, cu(in1), m1, cu(in2), m2, o, \
                     n_tiles)
  if (dtype == OW_DTYPE_BF16) {
    if (d == 64) {
      if (in2) OW_TILE_MIX(ow::BF16, true, 4); else OW_TILE_MIX(ow::BF16, false, 4);
    } else {
      if (in2) OW_TILE_MIX(ow::BF16, true, 8); else OW_TILE_MIX(ow::BF16, false, 8);
    }
  } else {
    if (d == 64) {
      if (in2) OW_TILE_MIX(ow::F16, true, 4); else OW_TILE_MIX(ow::F16, false, 4);
    } else {
      if (in2) OW_TILE_MIX(ow::F16, true, 8); else OW_TILE_MIX(ow::F16, false, 8);
    }
  }
#undef OW_TILE_MIX
  if (int rc = ow::hip_status(hipGetLastError(), "tile_mix_kernel launch")) return rc;
  ow::clear_error();
  return OW_OK;
}

int ow_tile_outer(const void* in1, const void* in2, float* partial, int32_t n_waves, int64_t n_tiles, int32_t d,
                  int32_t dtype, void* stream) {
  OW_CHECK_ARG(n_tiles >= 0 && d >= 16 && d % 16 == 0, "bad shape n_tiles=%lld d=%d", (long long)n_tiles, d);
  OW_CHECK_ARG(n_waves >= 4 && n_waves % 4 == 0, "n_waves must be a positive multiple of 4 (got %d)", n_waves);
  OW_CHECK_SUPPORTED(dtype == OW_DTYPE_BF16 || dtype == OW_DTYPE_F16 || dtype == OW_DTYPE_F32, "unsupported dtype %d",
                     dtype);
  OW_CHECK_ARG(partial && (n_tiles == 0 || (in1 && in2)), "tensor pointer is NULL");
  if (dtype == OW_DTYPE_F32) {
    if (int rc = ow::tile_outer_f32(static_cast<const float*>(in1), static_cast<const float*>(in2), partial, n_waves,
                                    n_tiles, d, static_cast<hipStream_t>(stream)))
      return rc;
    ow::clear_error();
    return OW_OK;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto cu = [](const void* p) { return static_cast<const uint16_t*>(p); };
  const int32_t vec = ow::aligned16(in1) && ow::aligned16(in2) ? 1 : 0;  // 16-byte row loads
  if (dtype == OW_DTYPE_BF16)
    hipLaunchKernelGGL(ow::tile_outer_kernel<ow::BF16>, dim3(n_waves / 4), dim3(256), 0, s, cu(in1), cu(in2), partial,
                       n_tiles, d, vec);
  else
    hipLaunchKernelGGL(ow::tile_outer_kernel<ow::F16>, dim3(n_waves / 4), dim3(256), 0, s, cu(in1), cu(in2), partial,
                       n_tiles, d, vec);
  if (int rc = ow::hip_status(hipGetLastError(), "tile_outer_kernel launch")) return rc;
  ow::clear_error();
  return OW_OK;
}

size_t ow_bwd_packed_bytes(int32_t q_c, int32_t d, int32_t rd) {
  if (q_c < 1 || (d != 64 && d != 128) || (rd != 128 && rd != 256)) return 0;
  return static_cast<size_t>(q_c) * (rd / 32) * ow::bwd_frags(d) * ow::kFragElems * 2;
}

int ow_pack_bwd_weights(const void* b_u, const void* b_v, const void* b_o, int32_t weight_dtype, const float* norm_weight,
                        const float* gamma, const int32_t* channel_index, int32_t channels, int32_t q_c, int32_t d,
                        int32_t rd, int32_t compute_dtype, void* packed, void* stream) {
  OW_CHECK_ARG(b_u && b_v && b_o && channel_index && packed, "tensor pointer is NULL");
  OW_CHECK_SUPPORTED((d == 64 || d == 128) && (rd == 128 || rd == 256),
                     "packed backward weights need d in {64, 128}, rd in {128, 256}");
  OW_CHECK_ARG(q_c >= 1 && channels >= 1, "bad shape q_c=%d C=%d", q_c, channels);
  OW_CHECK_ARG(weight_dtype >= OW_DTYPE_F32 && weight_dtype <= OW_DTYPE_F16, "unknown weight dtype %d", weight_dtype);
  OW_CHECK_SUPPORTED(compute_dtype == OW_DTYPE_BF16 || compute_dtype == OW_DTYPE_F16, "unsupported compute dtype %d",
                     compute_dtype);
  const int64_t total = static_cast<int64_t>(ow_bwd_packed_bytes(q_c, d, rd) / 2);
  ow::BwdPackArgs p{b_u, b_v, b_o, norm_weight, gamma, channel_index, static_cast<uint16_t*>(packed),
                    weight_dtype, q_c, rd, channels, total, d};
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (compute_dtype == OW_DTYPE_BF16)
    hipLaunchKernelGGL(ow::pack_bwd_kernel<ow::BF16>, dim3(ow::blocks_for(total)), dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(ow::pack_bwd_kernel<ow::F16>, dim3(ow::blocks_for(total)), dim3(256), 0, s, p);
  if (int rc = ow::hip_status(hipGetLastError(), "pack_bwd_kernel launch")) return rc;
  ow::clear_error();
  return OW_OK;
}

int64_t ow_bwd_param_reduce64_partials(int64_t slots, int32_t q_c, int32_t rd) {
  if (q_c < 1 || slots <= 0 || slots % 32 || (rd != 128 && rd != 256)) return 0;
  return ow::bwd_param_reduce64_ranges(slots / 32, q_c) * q_c;
}

int ow_bwd_param_reduce64(const void* pu, const void* pv, const void* dw, const void* packed, size_t packed_bytes,
                          float* partial, int64_t n_partial, int64_t slots, int32_t q_c, int32_t rd, int32_t dtype,
                          void* stream) {
  OW_CHECK_SUPPORTED(rd == 128 || rd == 256, "parameter reduction needs rd in {128, 256} (got %d)", rd);
  OW_CHECK_SUPPORTED(dtype == OW_DTYPE_BF16 || dtype == OW_DTYPE_F16, "unsupported dtype %d", dtype);
  OW_CHECK_ARG(q_c >= 1 && slots >= 0 && slots % 32 == 0, "bad shape q_c=%d slots=%lld (multiple of 32)", q_c,
               (long long)slots);
  OW_CHECK_ARG(packed && packed_bytes == ow_bwd_packed_bytes(q_c, ow::kBwdD, rd),
               "packed backward weights hold %zu bytes", packed_bytes);
  if (slots == 0) {
    ow::clear_error();
    return OW_OK;
  }
  const int64_t rows = ow_bwd_param_reduce64_partials(slots, q_c, rd);
  OW_CHECK_ARG(n_partial == rows, "partial holds %lld rows; %lld needed (ow_bwd_param_reduce64_partials)",
               (long long)n_partial, (long long)rows);
  OW_CHECK_ARG(static_cast<int64_t>(q_c) * slots * ow::kBwdD * 2 < (int64_t(1) << 31),
               "intermediates of %lld slots exceed 2 GiB (buffer addressing)", (long long)slots);
  OW_CHECK_ARG(pu && pv && dw && partial, "tensor pointer is NULL");
  for (const void* p : {pu, pv, dw, packed})
    OW_CHECK_ARG(ow::aligned16(p), "intermediates and packed weights must be 16-byte aligned");
  auto cu = [](const void* p) { return static_cast<const uint16_t*>(p); };
  ow::ParamReduceArgs a{cu(pu), cu(pv), cu(dw), cu(packed), partial, slots / 32, q_c};
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int rc = rd == 128 ? ow::launch_param_reduce64<128>(a, rows, dtype, s)
                           : ow::launch_param_reduce64<256>(a, rows, dtype, s);
  if (rc == OW_OK) ow::clear_error();
  return rc;
}

int64_t ow_bwd_param_reduce128_partials(int64_t slots, int32_t q_c, int32_t rd) {
  if (q_c < 1 || slots <= 0 || slots % 16 || (rd != 128 && rd != 256)) return 0;
  return ow::bwd_param_reduce128_ranges(slots, q_c) * q_c;
}

int ow_bwd_param_reduce128(const void* pu, const void* pv, const void* dw, const void* z, const void* du,
                           const void* dv, float* partial, int64_t n_partial, int64_t slots, int32_t q_c, int32_t rd,
                           int32_t dtype, void* stream) {
  OW_CHECK_SUPPORTED(rd == 128 || rd == 256, "parameter reduction needs rd in {128, 256} (got %d)", rd);
  OW_CHECK_SUPPORTED(dtype == OW_DTYPE_BF16 || dtype == OW_DTYPE_F16, "unsupported dtype %d", dtype);
  OW_CHECK_ARG(q_c >= 1 && slots >= 0 && slots % 16 == 0, "bad shape q_c=%d slots=%lld (multiple of 16)", q_c,
               (long long)slots);
  if (slots == 0) {
    ow::clear_error();
    return OW_OK;
  }
  const int64_t rows = ow_bwd_param_reduce128_partials(slots, q_c, rd);
  OW_CHECK_ARG(n_partial == rows, "partial holds %lld rows; %lld needed (ow_bwd_param_reduce128_partials)",
               (long long)n_partial, (long long)rows);
  OW_CHECK_ARG(static_cast<int64_t>(q_c) * slots * rd * 2 < (int64_t(1) << 31),
               "intermediates of %lld slots exceed 2 GiB (buffer addressing)", (long long)slots);
  OW_CHECK_ARG(pu && pv && dw && z && du && dv && partial, "tensor pointer is NULL");
  for (const void* p : {pu, pv, dw, z, du, dv})
    OW_CHECK_ARG(ow::aligned16(p), "intermediate buffers must be 16-byte aligned");
  auto cu = [](const void* p) { return static_cast<const uint16_t*>(p); };
  ow::ParamReduce128Args a{cu(pu), cu(pv), cu(dw), cu(z), cu(du), cu(dv), partial, slots, q_c};
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t grid = 3 * rows;
  const int rc = rd == 128 ? ow::launch_param_reduce128<128>(a, grid, dtype, s)
                           : ow::launch_param_reduce128<256>(a, grid, dtype, s);
  if (rc == OW_OK) ow::clear_error();
  return rc;
}

int ow_sum_rows(const float* partial, int64_t rows, int64_t cols, float* out, void* stream) {
  OW_CHECK_ARG(rows >= 1 && cols >= 0 && cols % 4 == 0, "bad shape rows=%lld cols=%lld (cols a multiple of 4)",
               (long long)rows, (long long)cols);
  if (cols == 0) {
    ow::clear_error();
    return OW_OK;
  }
  OW_CHECK_ARG(partial && out, "tensor pointer is NULL");
  OW_CHECK_ARG(ow::aligned16(partial) && ow::aligned16(out), "partial and out must be 16-byte aligned");
  const int64_t cols4 = cols / 4, blocks = (cols4 + 63) / 64;
  OW_CHECK_ARG(blocks < (int64_t(1) << 31), "too many columns (%lld)", (long long)cols);
  const int W = ow::sum_rows_waves(rows);
  hipLaunchKernelGGL(ow::sum_rows_kernel, dim3(static_cast<unsigned>(blocks)), dim3(64 * W), 0,
                     static_cast<hipStream_t>(stream), reinterpret_cast<const float4*>(partial), rows, cols4,
                     reinterpret_cast<float4*>(out), W);
  if (int rc = ow::hip_status(hipGetLastError(), "sum_rows_kernel launch")) return rc;
  ow::clear_error();
  return OW_OK;
}

// Workgroups (and partial rows) of ow_bwd_fused: rd = 128 about one resident-weights workgroup
// per CU; rd = 256 rounds of four pairs, grid-strided over at most kBwdFusedGrid workgroups, so
// the dA partials stay few.
int64_t ow_bwd_fused_partials(int64_t slots, int32_t q_c, int32_t rd) {
  if (q_c < 1 || slots <= 0 || slots % 32 || (rd != 128 && rd != 256)) return 0;
  if (rd == 128) return ow::bwd_fused_res_grid(slots / 32, q_c);
  const int64_t rounds = static_cast<int64_t>(q_c) * ((slots / 32 + 3) / 4);
  return rounds < ow::kBwdFusedGrid ? rounds : ow::kBwdFusedGrid;
}

int ow_bwd_fused(const void* xt, const void* dyt, const float* a_u, const float* a_v, const float* a_o,
                 const void* packed, size_t packed_bytes, void* pu, void* pv, void* dw, void* dxt, float* partial,
                 int64_t n_partial, int64_t slots, int32_t q_c, int32_t d, int32_t rd, int32_t dtype, void* stream) {
  OW_CHECK_SUPPORTED(d == ow::kBwdD && (rd == 128 || rd == 256), "fused backward needs d = 64, rd in {128, 256}");
  OW_CHECK_SUPPORTED(dtype == OW_DTYPE_BF16 || dtype == OW_DTYPE_F16, "unsupported dtype %d", dtype);
  OW_CHECK_ARG(q_c >= 1 && slots >= 0 && slots % 32 == 0, "bad shape q_c=%d slots=%lld (multiple of 32)", q_c,
               (long long)slots);
  OW_CHECK_ARG(packed && packed_bytes == ow_bwd_packed_bytes(q_c, d, rd), "packed backward weights hold %zu bytes",
               packed_bytes);
  if (slots == 0) {
    ow::clear_error();
    return OW_OK;
  }
  const int64_t grid = ow_bwd_fused_partials(slots, q_c, rd);
  OW_CHECK_ARG(n_partial == grid, "partial holds %lld workgroup rows; %lld needed (ow_bwd_fused_partials)",
               (long long)n_partial, (long long)grid);
  OW_CHECK_ARG(static_cast<int64_t>(q_c) * slots * ow::kBwdD * 2 < (int64_t(1) << 31),
               "tiles of %lld slots exceed 2 GiB (buffer addressing)", (long long)slots);
  OW_CHECK_ARG(xt && dyt && a_u && a_v && a_o && pu && pv && dw && dxt && partial, "tensor pointer is NULL");
  for (const void* p : {xt, dyt, packed, static_cast<const void*>(pu), static_cast<const void*>(pv),
                        static_cast<const void*>(dw), static_cast<const void*>(dxt)})
    OW_CHECK_ARG(ow::aligned16(p), "tiles and packed weights must be 16-byte aligned");
  auto cu = [](const void* p) { return static_cast<const uint16_t*>(p); };
  auto mu = [](void* p) { return static_cast<uint16_t*>(p); };
  ow::BwdFusedArgs a{cu(xt), cu(dyt), a_u, a_v, a_o, cu(packed), mu(pu), mu(pv), mu(dw), mu(dxt), partial, slots,
                     slots / 32, 0, q_c};
  a.rounds = static_cast<int64_t>(q_c) * ((a.pairs_per_q + 3) / 4);
  return ow::launch_bwd_fused<false>(a, grid, rd, dtype, static_cast<hipStream_t>(stream));
}

namespace ow {
namespace {
// ow_bwd_channel and its routed form (r.tok, r.x, r.dy set; xt, dyt NULL).
int bwd_channel(const void* xt, const void* dyt, const float* a_u, const float* a_v, const float* a_o,
                const void* packed, size_t packed_bytes, void* pu, void* pv, void* dw, void* z, void* du, void* dv,
                int64_t slots, int32_t q_c, int32_t d, int32_t rd, int32_t dtype, const BwdChanArgs& r,
                void* stream) {
  OW_CHECK_SUPPORTED(d == ow::kB2D && (rd == 128 || rd == 256), "backward channel kernel needs d = 128, rd in {128, 256}");
  OW_CHECK_SUPPORTED(dtype == OW_DTYPE_BF16 || dtype == OW_DTYPE_F16, "unsupported dtype %d", dtype);
  OW_CHECK_ARG(q_c >= 1 && slots >= 0 && slots % 16 == 0, "bad shape q_c=%d slots=%lld (multiple of 16)", q_c,
               (long long)slots);
  OW_CHECK_ARG(packed && packed_bytes == ow_bwd_packed_bytes(q_c, d, rd), "packed backward weights hold %zu bytes",
               packed_bytes);
  if (slots == 0) {
    ow::clear_error();
    return OW_OK;
  }
  OW_CHECK_ARG(static_cast<int64_t>(q_c) * slots * rd * 2 < (int64_t(1) << 31), "tiles of %lld slots exceed 2 GiB",
               (long long)slots);
  const void* xs = r.tok ? static_cast<const void*>(r.x) : xt;
  const void* ys = r.tok ? static_cast<const void*>(r.dy) : dyt;
  OW_CHECK_ARG(xs && ys && a_u && a_v && a_o && pu && pv && dw && z && du && dv, "tensor pointer is NULL");
  for (const void* p : {xs, ys, packed, static_cast<const void*>(pu), static_cast<const void*>(pv),
                        static_cast<const void*>(dw), static_cast<const void*>(z), static_cast<const void*>(du),
                        static_cast<const void*>(dv)})
    OW_CHECK_ARG(ow::aligned16(p), "tiles and packed weights must be 16-byte aligned");
  auto cu = [](const void* p) { return static_cast<const uint16_t*>(p); };
  auto mu = [](void* p) { return static_cast<uint16_t*>(p); };
  ow::BwdChanArgs a = r;
  a.xt = cu(xt);
  a.dyt = cu(dyt);
  a.a_u = a_u;
  a.a_v = a_v;
  a.a_o = a_o;
  a.packed = cu(packed);
  a.pu = mu(pu);
  a.pv = mu(pv);
  a.dw = mu(dw);
  a.z = mu(z);
  a.du = mu(du);
  a.dv = mu(dv);
  a.slots = slots;
  a.q_c = q_c;
  const int64_t units = static_cast<int64_t>(q_c) * ((slots + ow::kB2Rows - 1) / ow::kB2Rows);
  OW_CHECK_ARG(units < (int64_t(1) << 31), "too many units");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int rc = rd == 256 ? ow::launch_bwd_chan_rd<256>(a, static_cast<int32_t>(units), dtype, s)
                           : ow::launch_bwd_chan_rd<128>(a, static_cast<int32_t>(units), dtype, s);
  if (rc == OW_OK) ow::clear_error();
  return rc;
}

// The routing of ow_bwd_channel_routed / ow_bwd_channel2_routed: plan checks, and the row
// tables of the kernels' routed mode (slots = batch * q_s * 16).
struct Routed128 {
  int64_t slots = 0;
  int32_t q_c = 0, d = 0, q_s = 0, n_tok = 0, channels = 0;
};
int routed128(const OwPlan* plan, int32_t batch, const void* x, const void* dy, const int32_t* token_index,
              Routed128& r) {
  if (int rc = ow_plan_dims(plan, &r.q_s, &r.q_c)) return rc;
  r.d = plan->channel_tile;
  r.channels = plan->channels;
  OW_CHECK_SUPPORTED(plan->spatial_tile == kG, "unsupported spatial tile g=%d; expected 16", plan->spatial_tile);
  OW_CHECK_SUPPORTED(r.d == kB2D && r.channels == r.q_c * kB2D && (plan->radix_level == 0 || r.q_c == 1),
                     "routed backward needs the identity channel order with C = q_c * 128");
  OW_CHECK_ARG(batch >= 0 && static_cast<int64_t>(batch) * r.q_s < (int64_t(1) << 27), "bad batch %d", batch);
  OW_CHECK_ARG(static_cast<int64_t>(batch) * plan->height * plan->width * r.channels * 2 < (int64_t(1) << 31),
               "x, dy and g must be below 2 GiB (buffer addressing)");
  OW_CHECK_ARG(x && dy && token_index, "tensor pointer is NULL");
  r.slots = static_cast<int64_t>(batch) * r.q_s * kG;
  r.n_tok = plan->height * plan->width;
  return OW_OK;
}
}  // namespace
}  // namespace ow

int ow_bwd_channel(const void* xt, const void* dyt, const float* a_u, const float* a_v, const float* a_o,
                   const void* packed, size_t packed_bytes, void* pu, void* pv, void* dw, void* z, void* du, void* dv,
                   int64_t slots, int32_t q_c, int32_t d, int32_t rd, int32_t dtype, void* stream) {
  return ow::bwd_channel(xt, dyt, a_u, a_v, a_o, packed, packed_bytes, pu, pv, dw, z, du, dv, slots, q_c, d, rd, dtype,
                         ow::BwdChanArgs{}, stream);
}

int ow_bwd_channel_routed(const void* x, const void* dy, const float* rscale, const int32_t* token_index,
                          const OwPlan* plan, int32_t batch, const float* a_u, const float* a_v, const float* a_o,
                          const void* packed, size_t packed_bytes, void* pu, void* pv, void* dw, void* z, void* du,
                          void* dv, int32_t rd, int32_t dtype, void* stream) {
  ow::Routed128 rt;
  if (int rc = ow::routed128(plan, batch, x, dy, token_index, rt)) return rc;
  ow::BwdChanArgs r{};
  r.x = static_cast<const uint16_t*>(x);
  r.dy = static_cast<const uint16_t*>(dy);
  r.rscale = rscale;
  r.tok = token_index;
  r.q_s = rt.q_s;
  r.n_tok = rt.n_tok;
  r.channels = rt.channels;
  return ow::bwd_channel(nullptr, nullptr, a_u, a_v, a_o, packed, packed_bytes, pu, pv, dw, z, du, dv, rt.slots,
                         rt.q_c, rt.d, rd, dtype, r, stream);
}

int64_t ow_bwd_channel_partials(int64_t slots, int32_t q_c) {
  if (q_c < 1 || slots <= 0 || slots % 16) return 0;
  return ow::bwd_chan_grid(static_cast<int64_t>(q_c) * ((slots + ow::kB2Rows - 1) / ow::kB2Rows));
}

namespace ow {
namespace {
// ow_bwd_channel2 and its routed form: r.tok / r.g set (and dxt NULL) for the routed one.
int bwd_channel2(const void* xt, const void* dyt, const void* z, const void* du, const void* dv, const float* a_u,
                 const float* a_v, const void* packed, size_t packed_bytes, void* dxt, float* partial, int64_t n_partial,
                 int64_t slots, int32_t q_c, int32_t d, int32_t rd, int32_t dtype, const BwdChan2Args& r,
                 void* stream) {
  OW_CHECK_SUPPORTED(d == ow::kB2D && (rd == 128 || rd == 256), "backward channel kernel needs d = 128, rd in {128, 256}");
  OW_CHECK_SUPPORTED(dtype == OW_DTYPE_BF16 || dtype == OW_DTYPE_F16, "unsupported dtype %d", dtype);
  OW_CHECK_ARG(q_c >= 1 && slots >= 0 && slots % 16 == 0, "bad shape q_c=%d slots=%lld (multiple of 16)", q_c,
               (long long)slots);
  OW_CHECK_ARG(packed && packed_bytes == ow_bwd_packed_bytes(q_c, d, rd), "packed backward weights hold %zu bytes",
               packed_bytes);
  if (slots == 0) {
    ow::clear_error();
    return OW_OK;
  }
  const int64_t grid = ow_bwd_channel_partials(slots, q_c);
  OW_CHECK_ARG(n_partial == grid, "partial holds %lld workgroup rows; %lld needed (ow_bwd_channel_partials)",
               (long long)n_partial, (long long)grid);
  OW_CHECK_ARG(static_cast<int64_t>(q_c) * slots * rd * 2 < (int64_t(1) << 31), "tiles of %lld slots exceed 2 GiB",
               (long long)slots);
  OW_CHECK_ARG(xt && dyt && z && du && dv && a_u && a_v && (dxt || r.g) && partial, "tensor pointer is NULL");
  for (const void* p : {xt, dyt, z, du, dv, packed, r.g ? static_cast<const void*>(r.g) : dxt})
    OW_CHECK_ARG(ow::aligned16(p), "tiles and packed weights must be 16-byte aligned");
  auto cu = [](const void* p) { return static_cast<const uint16_t*>(p); };
  ow::BwdChan2Args a = r;
  a.xt = cu(xt);
  a.dyt = cu(dyt);
  a.z = cu(z);
  a.du = cu(du);
  a.dv = cu(dv);
  a.a_u = a_u;
  a.a_v = a_v;
  a.packed = cu(packed);
  a.dxt = static_cast<uint16_t*>(dxt);
  a.partial = partial;
  a.slots = slots;
  a.q_c = q_c;
  const int64_t units = static_cast<int64_t>(q_c) * ((slots + ow::kB2Rows - 1) / ow::kB2Rows);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int rc = rd == 256 ? ow::launch_bwd_chan2_rd<256>(a, grid, static_cast<int32_t>(units), dtype, s)
                           : ow::launch_bwd_chan2_rd<128>(a, grid, static_cast<int32_t>(units), dtype, s);
  if (rc == OW_OK) ow::clear_error();
  return rc;
}
}  // namespace
}  // namespace ow

int ow_bwd_channel2(const void* xt, const void* dyt, const void* z, const void* du, const void* dv, const float* a_u,
                    const float* a_v, const void* packed, size_t packed_bytes, void* dxt, float* partial,
                    int64_t n_partial, int64_t slots, int32_t q_c, int32_t d, int32_t rd, int32_t dtype, void* stream) {
  OW_CHECK_ARG(dxt, "tensor pointer is NULL");
  return ow::bwd_channel2(xt, dyt, z, du, dv, a_u, a_v, packed, packed_bytes, dxt, partial, n_partial, slots, q_c, d,
                          rd, dtype, ow::BwdChan2Args{}, stream);
}

int ow_bwd_channel2_routed(const void* x, const void* dy, const float* rscale, const void* z, const void* du,
                           const void* dv, const float* a_u, const float* a_v, const void* packed, size_t packed_bytes,
                           const int32_t* token_index, const OwPlan* plan, int32_t batch, void* g, float* partial,
                           int64_t n_partial, int32_t rd, int32_t dtype, void* stream) {
  ow::Routed128 rt;
  if (int rc = ow::routed128(plan, batch, x, dy, token_index, rt)) return rc;
  OW_CHECK_ARG(g, "tensor pointer is NULL");
  ow::BwdChan2Args r{};
  r.x = static_cast<const uint16_t*>(x);
  r.dy = static_cast<const uint16_t*>(dy);
  r.rscale = rscale;
  r.tok = token_index;
  r.g = static_cast<uint16_t*>(g);
  r.q_s = rt.q_s;
  r.n_tok = rt.n_tok;
  r.channels = rt.channels;
  return ow::bwd_channel2(x, dy, z, du, dv, a_u, a_v, packed, packed_bytes, nullptr, partial, n_partial, rt.slots,
                          rt.q_c, rt.d, rd, dtype, r, stream);
}

int ow_bwd_fused_routed(const void* x, const void* dy, const float* rscale, const int32_t* token_index,
                        const OwPlan* plan, int32_t batch, const float* a_u, const float* a_v, const float* a_o,
                        const void* packed, size_t packed_bytes, void* pu, void* pv, void* dw, void* g,
                        float* partial, int64_t n_partial, int32_t rd, int32_t dtype, void* stream) {
  int32_t q_s = 0, q_c = 0;
  if (int rc = ow_plan_dims(plan, &q_s, &q_c)) return rc;
  const int32_t d = plan->channel_tile, c = plan->channels, n = plan->height * plan->width;
  OW_CHECK_SUPPORTED(d == ow::kBwdD && (rd == 128 || rd == 256), "fused backward needs d = 64, rd in {128, 256}");
  OW_CHECK_SUPPORTED(dtype == OW_DTYPE_BF16 || dtype == OW_DTYPE_F16, "unsupported dtype %d", dtype);
  OW_CHECK_SUPPORTED(plan->spatial_tile == ow::kG, "unsupported spatial tile g=%d; expected 16", plan->spatial_tile);
  OW_CHECK_SUPPORTED(c == q_c * ow::kBwdD && (plan->radix_level == 0 || q_c == 1),
                     "routed backward needs the identity channel order with C = q_c * 64");
  OW_CHECK_ARG(batch >= 0 && static_cast<int64_t>(batch) * q_s < (int64_t(1) << 31), "bad batch %d", batch);
  OW_CHECK_ARG(static_cast<int64_t>(batch) * plan->height * plan->width * c * 2 < (int64_t(1) << 31),
               "x and dy must be below 2 GiB (buffer addressing)");
  OW_CHECK_ARG(packed && packed_bytes == ow_bwd_packed_bytes(q_c, d, rd), "packed backward weights hold %zu bytes",
               packed_bytes);
  const int64_t slots = static_cast<int64_t>(batch) * q_s * ow::kG;
  if (slots == 0) {
    ow::clear_error();
    return OW_OK;
  }
  const int64_t grid = ow_bwd_fused_partials(slots, q_c, rd);
  OW_CHECK_ARG(n_partial == grid, "partial holds %lld workgroup rows; %lld needed (ow_bwd_fused_partials)",
               (long long)n_partial, (long long)grid);
  OW_CHECK_ARG(x && dy && token_index && a_u && a_v && a_o && pu && pv && dw && g && partial,
               "tensor pointer is NULL");
  for (const void* p : {x, dy, packed, static_cast<const void*>(pu), static_cast<const void*>(pv),
                        static_cast<const void*>(dw), static_cast<const void*>(g)})
    OW_CHECK_ARG(ow::aligned16(p), "tensors and packed weights must be 16-byte aligned");
  auto cu = [](const void* p) { return static_cast<const uint16_t*>(p); };
  auto mu = [](void* p) { return static_cast<uint16_t*>(p); };
  ow::BwdFusedArgs a{nullptr, nullptr, a_u, a_v, a_o, cu(packed), mu(pu), mu(pv), mu(dw), nullptr, partial, slots,
                     slots / 32, 0, q_c};
  a.rounds = static_cast<int64_t>(q_c) * ((a.pairs_per_q + 3) / 4);
  a.x = cu(x);
  a.dy = cu(dy);
  a.rscale = rscale;
  a.tok = token_index;
  a.g = mu(g);
  a.batch = batch;
  a.n_tok = n;
  a.q_s = q_s;
  a.channels = c;
  return ow::launch_bwd_fused<true>(a, grid, rd, dtype, static_cast<hipStream_t>(stream));
}

int ow_small_to_f32(const void* const* src, const int32_t* dtype, const int64_t* count, int32_t n, float* dst,
                    void* stream) {
  OW_CHECK_ARG(n >= 1 && n <= 8, "between 1 and 8 sources (got %d)", n);
  OW_CHECK_ARG(src && dtype && count && dst, "argument pointer is NULL");
  ow::SmallF32Args a{};
  a.n = n;
  a.dst = dst;
  a.off[0] = 0;
  for (int k = 0; k < n; ++k) {
    OW_CHECK_ARG(dtype[k] >= OW_DTYPE_F32 && dtype[k] <= OW_DTYPE_F16, "unknown dtype %d of source %d", dtype[k], k);
    OW_CHECK_ARG(count[k] >= 0, "bad count %lld of source %d", (long long)count[k], k);
    OW_CHECK_ARG(src[k] || count[k] == 0, "source %d is NULL", k);
    a.src[k] = src[k];
    a.dtype[k] = dtype[k];
    a.off[k + 1] = a.off[k] + count[k];
  }
  for (int k = n + 1; k < 9; ++k) a.off[k] = a.off[n];
  const int64_t total = a.off[n];
  if (total > 0) {
    OW_CHECK_ARG(total < (int64_t(1) << 31), "too many values (%lld)", (long long)total);
    hipLaunchKernelGGL(ow::small_to_f32_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), a);
    if (int rc = ow::hip_status(hipGetLastError(), "small_to_f32_kernel launch")) return rc;
  }
  ow::clear_error();
  return OW_OK;
}

int ow_bwd_params(const void* b_u, const void* b_v, const void* b_o, int32_t weight_dtype, const float* norm_weight,
                  const float* gamma, const int32_t* channel_index, int32_t channels, int32_t q_c, int32_t d, int32_t rd,
                  const float* dbu, const float* dbv, const float* dbo, float* g_bu, float* g_bv, float* g_bo,
                  float* g_gamma, float* g_norm_weight, void* stream) {
  OW_CHECK_ARG(b_u && b_v && b_o && channel_index && dbu && dbv && dbo && g_bu && g_bv && g_bo && g_gamma,
               "tensor pointer is NULL");
  OW_CHECK_ARG(!norm_weight == !g_norm_weight, "norm_weight and its gradient go together");
  OW_CHECK_ARG(q_c >= 1 && d >= 1 && rd >= 1 && channels >= 1, "bad shape q_c=%d d=%d rd=%d C=%d", q_c, d, rd, channels);
  OW_CHECK_ARG(weight_dtype >= OW_DTYPE_F32 && weight_dtype <= OW_DTYPE_F16, "unknown weight dtype %d", weight_dtype);
  ow::ParamArgs a{b_u, b_v, b_o, norm_weight, gamma, channel_index, dbu, dbv, dbo, g_bu, g_bv, g_bo, g_gamma,
                  g_norm_weight, weight_dtype, q_c, d, rd, channels};
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t n_a = (static_cast<int64_t>(q_c) * d + 3) / 4;
  const int64_t n_b = static_cast<int64_t>(q_c) * ((d + ow::kParamC - 1) / ow::kParamC);
  OW_CHECK_ARG(n_a + n_b < (int64_t(1) << 31), "too many channels (q_c=%d d=%d)", q_c, d);
  hipLaunchKernelGGL(ow::bwd_params_kernel, dim3(static_cast<unsigned>(n_a + n_b)), dim3(256), 0, s, a,
                     static_cast<int32_t>(n_a));
  if (int rc = ow::hip_status(hipGetLastError(), "bwd_params_kernel launch")) return rc;
  ow::clear_error();
  return OW_OK;
}

}  // extern "C"
