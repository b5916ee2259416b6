// noalloc.hip -- the fixed device workspace of wgx_mm_noalloc (include/wgx.h).
//
// One array per GPU, in the code object's own device memory: it exists from
// the moment the library's code object is loaded on a device until the
// process ends, so using it allocates nothing.  In host code the name
// `scratch` is only a host-side stand-in; its device address comes from
// hipGetSymbolAddress, looked up once per device with that device current
// (each GPU holds its own copy of the array at its own address), and only
// that address is ever handed to a kernel.
#include <mutex>

#include "internal.h"

static __device__ __align__(256) unsigned char scratch[WGX_NOALLOC_SCRATCH_BYTES];

namespace wgx {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices];
hipError_t g_err[kMaxDevices];
bool g_done[kMaxDevices];

}  // namespace

hipError_t noalloc_scratch(int device, void** out) {
  *out = nullptr;
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_done[device]) {
    int cur = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e == hipSuccess && cur != device) e = hipSetDevice(device);
    void* p = nullptr;
    if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e == hipSuccess && p == nullptr) e = hipErrorInvalidSymbol;
    if (cur >= 0 && cur != device) {
      const hipError_t r = hipSetDevice(cur);  // the caller's device back
      if (e == hipSuccess) e = r;
    }
    g_ptr[device] = e == hipSuccess ? p : nullptr;
    g_err[device] = e;
    g_done[device] = true;
  }
  *out = g_ptr[device];
  return g_err[device];
}

}  // namespace wgx
