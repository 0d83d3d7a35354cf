// gmoe_noalloc.hip — the device scratch of the allocation-free forward
// (gmoe_ffn_forward_noalloc): one file-scope array per GPU, sized once, that the library
// never allocates or frees at call time. Its address on a device is looked up once, with
// that device current, and kept; host code passes that address (never the array's name,
// which on the host is only a stand-in) to kernels and copies.
#include <hip/hip_runtime.h>

#include <mutex>

#include "gmoe_internal.h"

namespace {

static __device__ __align__(256) uint8_t scratch[gmoe::kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices] = {};

}  // namespace

namespace gmoe {

// Address of `scratch` on `device`, which must be the current device. Looked up on the
// first call for the device and kept.
hipError_t noalloc_scratch(int device, void** out) {
  *out = nullptr;
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> g(g_mu);
  if (!g_ptr[device]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    g_ptr[device] = p;
  }
  *out = g_ptr[device];
  return hipSuccess;
}

}  // namespace gmoe
