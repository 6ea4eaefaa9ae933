// Fixed device scratch of ponni_forward_no_alloc.
//
// One file-scope device array, `scratch`, of kStaticScratchBytes.  Every GPU
// the library runs on holds its own copy from the first use on that GPU until
// the process ends.  The array's name is a host-side stand-in in host code,
// not a device address: its address on a device comes from
// hipGetSymbolAddress, called once per device with that device current, and
// only that address is ever handed to kernels.
#include <hip/hip_runtime.h>

#include <mutex>

#include "plan.h"

namespace ponni_hip {
namespace {

__device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_mutex;
void* g_scratch[kMaxDevices] = {};  // device address of `scratch`, per device

}  // namespace

hipError_t static_scratch(int device, void** out) {
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_mutex);
  if (g_scratch[device] == nullptr) {
    int current = -1;
    hipError_t e = hipGetDevice(&current);
    if (e != hipSuccess) return e;
    if (current != device) return hipErrorInvalidDevice;
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (p == nullptr) return hipErrorInvalidSymbol;
    g_scratch[device] = p;
  }
  *out = g_scratch[device];
  return hipSuccess;
}

}  // namespace ponni_hip
