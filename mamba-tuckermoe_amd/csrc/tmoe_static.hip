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

hipError_t static_scratch(void** ptr) {
  *ptr = nullptr;
  int dev = -1;
  if (hipError_t e = hipGetDevice(&dev); e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_ptr[dev]) {
    void* p = nullptr;
    // with `dev` current: the address of this GPU's copy
    if (hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)); e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    g_ptr[dev] = p;
  }
  *ptr = g_ptr[dev];
  return hipSuccess;
}

}  // namespace tmoe
