// The scratch array of rtg_forward_cached_noalloc and its per-device address.
//
// In host code the name `scratch` is only a host-side stand-in for the
// device symbol: passing it to a kernel would fault. Host code therefore uses
// the address hipGetSymbolAddress returns for the device, never the name.
// Every device holds its own copy of the array until the process ends; calls
// on one device share it and take scratch_lock(device) for the whole pass.
#include "scratch.h"

#include <mutex>

namespace rtg {

static __device__ __align__(256) float scratch[kScratchHeadFloats + kScratchFloats];

float* scratch_device_ptr(int device, hipError_t* err) {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static float* ptrs[kMaxDevices] = {};
  std::lock_guard<std::mutex> g(mu);
  if (device < 0 || device >= kMaxDevices) {
    *err = hipErrorInvalidDevice;
    return nullptr;
  }
  if (!ptrs[device]) {
    int cur = 0;
    hipError_t e = hipGetDevice(&cur);
    if (e == hipSuccess && cur != device) e = hipSetDevice(device);
    void* p = nullptr;
    if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e == hipSuccess) e = hipMemset(p, 0, kScratchHeadFloats * sizeof(float));
    if (cur != device) {
      const hipError_t r = hipSetDevice(cur);
      if (e == hipSuccess) e = r;
    }
    if (e != hipSuccess) {
      *err = e;
      return nullptr;
    }
    ptrs[device] = static_cast<float*>(p);
  }
  *err = hipSuccess;
  return ptrs[device];
}

std::mutex& scratch_lock(int device) {
  static std::mutex locks[64];
  return locks[(unsigned)device % 64u];
}

}  // namespace rtg
