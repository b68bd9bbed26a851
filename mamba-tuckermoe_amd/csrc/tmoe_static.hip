// The workspace of tmoe_forward_static: one file-scope device array per GPU,
// so that a forward can run without any allocation (callers under HIP graph
// capture or in serving loops that may not call hipMalloc). Each GPU the
// library runs on holds its copy until the process ends. Host code never uses
// the array's name as an address: its device address on the current GPU comes
// from hipGetSymbolAddress, looked up once per device and kept.
#include <hip/hip_runtime.h>

#include <mutex>

#include "tmoe_internal.h"

namespace {

static __device__ __align__(256) unsigned char scratch[tmoe::kStaticScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices];   // device address of `scratch` on each GPU (null: not looked up)

}  // namespace

namespace tmoe {

hipError_t static_scratch(hipStream_t stream, void** ptr) {
  *ptr = nullptr;
  int cur = -1;
  if (hipError_t e = hipGetDevice(&cur); e != hipSuccess) return e;
  // the device the forward's kernels run on: the stream's (the null stream: the
  // current device's)
  int dev = cur;
  if (stream) {
    hipDevice_t d = -1;
    if (hipError_t e = hipStreamGetDevice(stream, &d); e != hipSuccess) return e;
    dev = (int)d;
  }
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_ptr[dev]) {
    // with `dev` current: the address of that GPU's copy
    if (dev != cur)
      if (hipError_t e = hipSetDevice(dev); e != hipSuccess) return e;
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (dev != cur) {
      const hipError_t r = hipSetDevice(cur);
      if (e == hipSuccess) e = r;
    }
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    g_ptr[dev] = p;
  }
  *ptr = g_ptr[dev];
  return hipSuccess;
}

}  // namespace tmoe
