// rtq_noalloc.hip — rtq_linear_forward_noalloc_d (include/rtq.h): Linear::forward on device
// pointers for callers that cannot allocate device memory (code under HIP graph capture, tight
// serving loops, harnesses that forbid hipMalloc).  The forward's workspace (the quantised
// activation fragments, their scales and the LoRA-down partials) lives in `scratch`, a file-scope
// device array of kScratchBytes that every GPU holds from the library's set-up until the process
// ends, instead of the context's hipMalloc'd workspace.  Nothing on this path allocates.
//
// Host code never passes `scratch` itself to a kernel (that name is a host-side stand-in, not a
// device address): rtq_scratch_setup resolves the array's address on each device once, with that
// device current, and the entry point hands that address to the kernels.
#include <hip/hip_runtime.h>

#include <mutex>

#include "rtq_internal.h"

namespace {
constexpr size_t kScratchBytes = size_t(64) << 20;  // the largest forward workspace this entry point serves
constexpr int kMaxDevices = 64;

std::mutex g_mu;
void* g_scratch[kMaxDevices] = {};  // the array's device address on each device (null: not set up)
}  // namespace

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

// called by rtq_ctx_create with `device` current; once per device
rtq_status rtq_scratch_setup(int device) {
  if (device < 0 || device >= kMaxDevices) return rtq_fail(RTQ_ERR_INVALID, "device %d out of range", device);
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_scratch[device]) return RTQ_OK;
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p)
    return rtq_fail(RTQ_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", device, hipGetErrorString(e));
  g_scratch[device] = p;
  return RTQ_OK;
}

extern "C" rtq_status rtq_linear_forward_noalloc_d(rtq_ctx* ctx, const rtq_weight* w, const float* bias,
                                                   const rtq_lora* lora, const float* x, int64_t t, float* y,
                                                   void* stream) {
  const int dev = rtq_ctx_device_id(ctx);
  if (dev < 0 || dev >= kMaxDevices) return rtq_fail(RTQ_ERR_INVALID, "null context");
  void* p = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    p = g_scratch[dev];
  }
  if (!p) return rtq_fail(RTQ_ERR_INVALID, "scratch of device %d is not set up", dev);
  return rtq_linear_forward_ws_d(ctx, w, bias, lora, x, t, y, stream, p, kScratchBytes);
}
