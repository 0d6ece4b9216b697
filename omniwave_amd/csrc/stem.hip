// Stem of the OmniWeave backbone as one gather-GEMM (omniweave/models/backbone.py:121,173-176):
// NCHW image [B, 3, H, W] -> space_to_depth(4) -> Linear(48, N, bias=False) -> NHWC
// [B, H/4, W/4, N], without materialising the permuted image.
//
// The 48-deep contraction runs on 32x32x16 MFMAs.  Any K order works if the weight and the
// image operand agree, so K runs over (input channel, row offset, column offset): K step c is
// input channel c, and the 8 K slots of lane half hh are the 4x2 pixels of patch rows 2hh and
// 2hh + 1 — two 8-byte vectors read straight from the NCHW image.  The weight (K order (row
// offset, column offset, channel), as nn.Linear holds it after space_to_depth) is gathered
// into that order once per workgroup and stays in registers.  The product is computed
// transposed (output channels x pixels, weight rows as the A operand) and leaves through LDS
// as whole 16-byte vectors: the 32 pixels of a wave are 32 contiguous NHWC rows.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "ow_device.h"

namespace ow {
namespace {

constexpr int kStemIn = 3;                         // image channels
constexpr int kStemF = 4;                          // patch size (space_to_depth factor)
constexpr int kStemK = kStemIn * kStemF * kStemF;  // 48
constexpr int kStemThreads = 128;                  // two waves, 32 output pixels each
constexpr int kStemPix = 64;                       // output pixels per unit

struct StemArgs {
  const uint16_t* img;  // [B, 3, H, W]
  const uint16_t* w;    // [N, 48]
  uint16_t* out;        // [B, H/4, W/4, N]
  int32_t height, width;
  int32_t ho, wo;       // output rows and columns
  int32_t wblocks;      // 64-pixel blocks per output row
  int64_t units;        // B * ho * wblocks
};

template <class Ty, int NB>
__global__ void __attribute__((amdgpu_flat_work_group_size(kStemThreads, kStemThreads))) stem_kernel(StemArgs a) {
  constexpr int N = 32 * NB;
  constexpr int LDO = N + 8;  // padded LDS row stride (elements)
  __shared__ __attribute__((aligned(16))) uint16_t ot[2][32 * LDO];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int hh = lane >> 5, l32 = lane & 31;

  // A operand of output-channel block cb, K step c: row 32 cb + l32 of the weight, slot j =
  // patch pixel (row 2 hh + j / 4, column j % 4) of input channel c.
  u32x4 wa[NB][kStemIn];
#pragma unroll
  for (int cb = 0; cb < NB; ++cb)
#pragma unroll
    for (int c = 0; c < kStemIn; ++c) {
      const uint16_t* wr = a.w + (32 * cb + l32) * kStemK;
      auto tap = [&](int j) -> uint32_t {
        return wr[(2 * hh + j / 4) * (kStemF * kStemIn) + (j % 4) * kStemIn + c];
      };
      wa[cb][c] = u32x4{tap(0) | (tap(1) << 16), tap(2) | (tap(3) << 16), tap(4) | (tap(5) << 16),
                        tap(6) | (tap(7) << 16)};
    }

  uint16_t* o = ot[wave];
  auto load_unit = [&](int64_t u, u32x4 (&xb)[kStemIn]) {
    const int32_t pb = static_cast<int32_t>(u % a.wblocks);
    const int64_t bi = u / a.wblocks;
    const int32_t i = static_cast<int32_t>(bi % a.ho);
    const int64_t b = bi / a.ho;
    const int32_t p = pb * kStemPix + wave * 32 + l32;
    const bool valid = u < a.units && p < a.wo;
#pragma unroll
    for (int c = 0; c < kStemIn; ++c) {
      const uint16_t* src =
          a.img + ((b * kStemIn + c) * a.height + kStemF * i + 2 * hh) * static_cast<int64_t>(a.width) + kStemF * p;
      u32x2 r0 = {0u, 0u}, r1 = {0u, 0u};
      if (valid) {
        r0 = *reinterpret_cast<const u32x2*>(src);
        r1 = *reinterpret_cast<const u32x2*>(src + a.width);
      }
      xb[c] = u32x4{r0.x, r0.y, r1.x, r1.y};
    }
  };
  u32x4 xn[kStemIn];
  load_unit(blockIdx.x, xn);
  for (int64_t u = blockIdx.x; u < a.units; u += gridDim.x) {
    const int32_t pb = static_cast<int32_t>(u % a.wblocks);
    const int64_t bi = u / a.wblocks;  // b * ho + i
    const int32_t p0 = pb * kStemPix + wave * 32;  // first output pixel of this wave
    u32x4 xb[kStemIn];
#pragma unroll
    for (int c = 0; c < kStemIn; ++c) xb[c] = xn[c];
    load_unit(u + gridDim.x, xn);
    f32x16 acc[NB];
#pragma unroll
    for (int cb = 0; cb < NB; ++cb) {
      acc[cb] = f32x16{};
#pragma unroll
      for (int c = 0; c < kStemIn; ++c) acc[cb] = Ty::mma32(wa[cb][c], xb[c], acc[cb]);
    }
    mfma_drain();

    // Accumulator lane (pixel l32, hh) register 4q + r = channel 32 cb + 8q + 4hh + r.
#pragma unroll
    for (int cb = 0; cb < NB; ++cb)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<u32x2*>(&o[l32 * LDO + 32 * cb + 8 * q + 4 * hh]) =
            u32x2{Ty::pack2(acc[cb][4 * q], acc[cb][4 * q + 1]), Ty::pack2(acc[cb][4 * q + 2], acc[cb][4 * q + 3])};
    wave_lds_sync();

    // Output pixels p0 .. p0 + 31 of row (b, i): 32 contiguous NHWC rows of N channels.
    uint16_t* dst = a.out + (bi * a.wo + p0) * N;
    constexpr int VPR = N / 8;
    constexpr int NV = 32 * VPR / 64;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int idx = lane + 64 * v;
      const int r = idx / VPR, cv = idx % VPR;
      if (p0 + r < a.wo)
        *reinterpret_cast<u32x4*>(dst + r * N + cv * 8) = *reinterpret_cast<const u32x4*>(&o[r * LDO + cv * 8]);
    }
    wave_lds_sync();
  }
}

// Persistent over units (the weight operands are gathered once per workgroup), with exactly as
// many workgroups as fit on the device at once: a grid beyond that leaves a second, partial
// wave of workgroups that each run a full share of units after the first ones finish.
template <class Ty, int NB>
int launch_stem_nb(const StemArgs& a, hipStream_t stream) {
  static int per_cu[64] = {0};
  int dev = 0;
  if (int rc = hip_status(hipGetDevice(&dev), "hipGetDevice")) return rc;
  int fit = dev >= 0 && dev < 64 ? per_cu[dev] : 0;
  if (fit == 0) {
    if (int rc = hip_status(hipOccupancyMaxActiveBlocksPerMultiprocessor(&fit, stem_kernel<Ty, NB>, kStemThreads, 0),
                            "hipOccupancyMaxActiveBlocksPerMultiprocessor"))
      return rc;
    fit = fit > 0 ? fit : 1;
    if (dev >= 0 && dev < 64) per_cu[dev] = fit;
  }
  const int64_t slots = static_cast<int64_t>(device_cus()) * fit;
  const unsigned grid = static_cast<unsigned>(a.units < slots ? a.units : slots);
  hipLaunchKernelGGL((stem_kernel<Ty, NB>), dim3(grid), dim3(kStemThreads), 0, stream, a);
  return hip_status(hipGetLastError(), "stem_kernel launch");
}

template <class Ty>
int launch_stem(const StemArgs& a, int32_t n_out, hipStream_t stream) {
  switch (n_out / 32) {
    case 1: return launch_stem_nb<Ty, 1>(a, stream);
    case 2: return launch_stem_nb<Ty, 2>(a, stream);
    case 3: return launch_stem_nb<Ty, 3>(a, stream);
    case 4: return launch_stem_nb<Ty, 4>(a, stream);
    case 6: return launch_stem_nb<Ty, 6>(a, stream);
    case 8: return launch_stem_nb<Ty, 8>(a, stream);
    default: return fail(OW_ERR_UNSUPPORTED, "stem: %d output channels; expected 32, 64, 96, 128, 192 or 256", n_out);
  }
}

}  // namespace
}  // namespace ow

extern "C" {

int ow_stem_fwd(const void* image, const void* weight, void* out, int32_t batch, int32_t height, int32_t width,
                int32_t n_out, int32_t dtype, void* stream) {
  OW_CHECK_ARG(batch >= 0 && height >= 0 && width >= 0, "negative size (batch %d, height %d, width %d)", batch,
               height, width);
  OW_CHECK_SUPPORTED(dtype == OW_DTYPE_BF16 || dtype == OW_DTYPE_F16, "stem: dtype %d; expected bf16 or f16", dtype);
  OW_CHECK_ARG(height % ow::kStemF == 0 && width % ow::kStemF == 0,
               "height %d and width %d must be divisible by 4", height, width);
  OW_CHECK_SUPPORTED(n_out > 0 && n_out % 32 == 0 && n_out <= 256 && n_out != 160 && n_out != 224,
                     "stem: %d output channels; expected 32, 64, 96, 128, 192 or 256", n_out);
  const int64_t pixels = static_cast<int64_t>(batch) * (height / ow::kStemF) * (width / ow::kStemF);
  if (pixels == 0) {
    ow::clear_error();
    return OW_OK;
  }
  OW_CHECK_ARG(image && weight && out, "tensor pointer is NULL");
  OW_CHECK_ARG(reinterpret_cast<uintptr_t>(image) % 8 == 0 && ow::aligned16(out) &&
                   reinterpret_cast<uintptr_t>(weight) % 2 == 0,
               "image must be 8-byte and out 16-byte aligned");
  OW_CHECK_ARG(static_cast<int64_t>(batch) * ow::kStemIn * height * width < (int64_t(1) << 40) &&
                   pixels * n_out < (int64_t(1) << 40),
               "tensor too large");
  ow::StemArgs a{};
  a.img = static_cast<const uint16_t*>(image);
  a.w = static_cast<const uint16_t*>(weight);
  a.out = static_cast<uint16_t*>(out);
  a.height = height;
  a.width = width;
  a.ho = height / ow::kStemF;
  a.wo = width / ow::kStemF;
  a.wblocks = (a.wo + ow::kStemPix - 1) / ow::kStemPix;
  a.units = static_cast<int64_t>(batch) * a.ho * a.wblocks;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int rc = dtype == OW_DTYPE_BF16 ? ow::launch_stem<ow::BF16>(a, n_out, s) : ow::launch_stem<ow::F16>(a, n_out, s);
  if (rc == OW_OK) ow::clear_error();
  return rc;
}

}  // extern "C"
