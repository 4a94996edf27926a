// w4a16_scratch.hip -- the static device scratch of the allocation-free entry
// point (w4a16_linear_noalloc).  One file-scope array per GPU the library runs on,
// held until the process ends; its device address is looked up once per device
// with hipGetSymbolAddress (the array's name is only a host-side stand-in) and
// cached.  Calls that share a GPU share its array.
#include <hip/hip_runtime.h>

#include <mutex>

#include "w4a16_launch.h"

namespace {

__device__ __attribute__((aligned(256))) unsigned char scratch[W4L_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices] = {};

}  // namespace

hipError_t w4l_scratch(void** ptr) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (p == nullptr) return hipErrorInvalidSymbol;
    g_ptr[dev] = p;
  }
  *ptr = g_ptr[dev];
  return hipSuccess;
}
