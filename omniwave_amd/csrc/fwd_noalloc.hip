// ow_bigemm_fwd without caller-provided device memory beyond its inputs and outputs.
//
// The only scratch buffer of the forward is the RMSNorm row-scale buffer (batch * H * W fp32)
// of launches whose statistics come from a separate pass (fp32 activations, element access of
// ragged or unaligned rows, channel counts the in-kernel statistics do not cover).  Here it is
// a file-scope device array, so a caller that cannot allocate (graph capture, a serving loop
// with a fixed footprint) still gets every code path.  Each GPU holds its own copy of the array
// for the life of the process; its device address is looked up once per device, with that
// device current, on the first call there.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>

#include "ow_device.h"

namespace ow {
// Rows of RMSNorm scales the array holds (4 MiB): OmniWeave-T's largest stage, 56 x 56 tokens,
// at batch 334; 14 x 14 at batch 5349.
constexpr int64_t kScratchRows = int64_t(1) << 20;
}  // namespace ow

static __device__ __align__(256) float scratch[ow::kScratchRows];

namespace ow {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
float* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device (looked up once per device).
int scratch_address(float** out) {
  int dev = -1;
  if (int rc = hip_status(hipGetDevice(&dev), "hipGetDevice")) return rc;
  if (dev < 0 || dev >= kMaxDevices) return fail(OW_ERR_UNSUPPORTED, "device id %d is out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    if (int rc = hip_status(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)")) return rc;
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_ptr[dev];
  return OW_OK;
}

}  // namespace
}  // namespace ow

extern "C" {

int ow_bigemm_fwd_noalloc(const void* x, void* out, float eps, const void* packed, size_t packed_bytes,
                          const int32_t* token_index, const int32_t* channel_index, const OwPlan* plan,
                          int32_t batch, int32_t rd, int32_t dtype, int32_t flags, void* stream) {
  OW_CHECK_ARG(plan, "plan is NULL");
  OW_CHECK_ARG(batch >= 0, "batch must be >= 0 (got %d)", batch);
  // Rejected before any device call when the launch would need more row scales than the array
  // holds.
  const int64_t rows = static_cast<int64_t>(batch) * plan->height * plan->width;
  const bool needs = ow::fwd_needs_scale_buffer(x, out, plan, rd, dtype, flags, false, batch);
  OW_CHECK_SUPPORTED(!needs || rows <= ow::kScratchRows,
                     "batch * H * W = %lld rows of RMSNorm scales exceed the %lld rows of the library's scratch",
                     (long long)rows, (long long)ow::kScratchRows);
  float* ptr = nullptr;
  if (batch > 0) {
    if (int rc = ow::scratch_address(&ptr)) return rc;
  }
  return ow_bigemm_fwd(x, out, eps, packed, packed_bytes, token_index, channel_index, plan, batch, rd, dtype, flags,
                       ptr, static_cast<size_t>(ow::kScratchRows) * sizeof(float), stream);
}

}  // extern "C"
