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
// Per device: an event recorded after each call's work on the scratch (on the call's
// stream), which the next call's stream waits for, and a lock held while a call queues its
// wait, launches and record. Every call on a GPU, from any context and on any stream, then
// runs after the previous one has finished with the shared array.
hipEvent_t g_ev[kMaxDevices] = {};
std::mutex g_dev_mu[kMaxDevices];

}  // namespace

namespace gmoe {

// Address of `scratch` on `device`, which must be the current device, and the device's
// ordering event: looked up and created on the first call for the device (set-up, from
// gmoe_init), then kept.
hipError_t noalloc_scratch(int device, void** out) {
  *out = nullptr;
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> g(g_mu);
  if (!g_ptr[device]) {
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    e = hipEventCreateWithFlags(&g_ev[device], hipEventDisableTiming);
    if (e != hipSuccess) return e;
    g_ptr[device] = p;
  }
  *out = g_ptr[device];
  return hipSuccess;
}

// Brackets one call's work on `st`: the returned lock is held until noalloc_end. A call
// being captured into a graph neither waits nor records (its replays are ordered by
// whoever launches the graph); any other waits for the previous call on the device.
std::unique_lock<std::mutex> noalloc_begin(int device, hipStream_t st, hipError_t* err) {
  std::unique_lock<std::mutex> lk(g_dev_mu[device]);
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  *err = hipStreamIsCapturing(st, &cs);
  if (*err == hipSuccess && cs == hipStreamCaptureStatusNone) *err = hipStreamWaitEvent(st, g_ev[device], 0);
  return lk;
}

hipError_t noalloc_end(int device, hipStream_t st) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(st, &cs);
  if (e == hipSuccess && cs == hipStreamCaptureStatusNone) e = hipEventRecord(g_ev[device], st);
  return e;
}

}  // namespace gmoe
