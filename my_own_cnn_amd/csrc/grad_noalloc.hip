// miq_grad_nhwc_f32_noalloc: the ordered fp32 filter gradient (miq_grad_nhwc_f32_ws) with its
// split partial sums in a file-scope device array, for callers that cannot allocate device
// memory (code under HIP graph capture, serving loops, harnesses that forbid hipMalloc).
//
// `scratch` is one array per device, held from the library's first use on that device until
// the process ends.  On the host its name is only a handle: the device address of this
// device's copy comes from hipGetSymbolAddress, called once per device (with that device
// current) on the entry point's first call there, and only that address is handed to the
// kernels.  Every call on a device shares its copy, so calls that overlap on one device
// (other streams, other threads) race; nothing in it needs clearing between calls, because
// each call writes every partial entry before its summing pass reads it.

#include <mutex>

#include "miq_qconv.h"
#include "qconv_internal.h"

constexpr size_t kScratchBytes = size_t{32} << 20;  // 32 MiB per device

static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

namespace {

constexpr int kMaxDevices = 64;
std::once_flag g_once[kMaxDevices];
void* g_scratch[kMaxDevices];
hipError_t g_status[kMaxDevices];

int scratch_of_current_device(void** out) {
  *out = nullptr;
  int dev = 0;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return miq::report_error(MIQ_ERR_HIP, std::string("hipGetDevice: ") + hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return miq::report_error(MIQ_ERR_UNSUPPORTED, "device index beyond 63");
  std::call_once(g_once[dev], [dev]() {
    void* ptr = nullptr;
    g_status[dev] = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    g_scratch[dev] = g_status[dev] == hipSuccess ? ptr : nullptr;
  });
  if (g_status[dev] != hipSuccess || g_scratch[dev] == nullptr) {
    return miq::report_error(MIQ_ERR_HIP, std::string("hipGetSymbolAddress of the grad scratch array: ") +
                                              hipGetErrorString(g_status[dev]));
  }
  *out = g_scratch[dev];
  return MIQ_OK;
}

}  // namespace

extern "C" int miq_grad_nhwc_f32_noalloc(const float* x, const float* dy, float* dw, int32_t n, int32_t h,
                                         int32_t wdt, int32_t c, int32_t r, int32_t s, int32_t k,
                                         const miq_conv2d_params* p, int32_t algo, void* stream) {
  size_t need = 0;
  const int st = miq::grad_f32_check(x, dy, dw, n, h, wdt, c, r, s, k, p, algo, &need);
  if (st != MIQ_OK) return st;
  if (need > kScratchBytes) {
    return miq::report_error(MIQ_ERR_UNSUPPORTED, "fp32 grad needs " + std::to_string(need) +
                                                      " bytes of split partial sums; the allocation-free entry point "
                                                      "holds at most 33554432 (use miq_grad_nhwc_f32_ws)");
  }
  void* ws = nullptr;
  if (need > 0) {
    const int e = scratch_of_current_device(&ws);
    if (e != MIQ_OK) return e;
  }
  return miq_grad_nhwc_f32_ws(x, dy, dw, n, h, wdt, c, r, s, k, p, algo, ws, need > 0 ? kScratchBytes : 0, stream);
}
