// rwkvmoe_forward_noalloc: the LoRA-MoE ChannelMix forward with its scratch
// memory in a device array the library owns, for callers that cannot
// allocate (code under HIP graph capture, serving loops, harnesses that
// forbid hipMalloc).  It launches exactly the kernels rwkvmoe_forward
// launches; only the workspace differs.
//
// The array lives in this translation unit's code object.  Its host-side
// name is a stand-in, not a device address: the device address is looked up
// with hipGetSymbolAddress once per device, on the first call made outside a
// graph capture with that device current (each device holds its own copy at
// its own address, until the process ends), and only that address is used.
// Calls captured into a HIP graph after that first call replay correctly:
// the forward issues no memset and no allocation.
//
// Every call on one device shares that device's array and leaves the last
// call's contents in it.  The forward needs no part of its workspace to start
// at zero (every region is written before it is read within a call; the loss
// ticket is reset by the router pass of the same call), so nothing is
// cleared here.  Two calls that overlap on one device (different streams, or
// host threads racing) race on the array.
#include <atomic>
#include <mutex>

#include "../../include/rwkvmoe.h"
#include "internal.h"

namespace rwkvmoe {

int forward_check(const rwkvmoe_desc* desc, const rwkvmoe_tensors* t);  // api.hip

namespace {

constexpr size_t kScratchBytes = (size_t)RWKVMOE_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

static __device__ __attribute__((aligned(256))) unsigned char scratch[kScratchBytes];

struct DeviceScratch {
  std::mutex mu;
  std::atomic<void*> ptr{nullptr};
};
DeviceScratch g_scratch[kMaxDevices];

// Device address of `scratch` on the current device, looked up on the first
// call made with that device current and kept for the process.  The lookup
// is not a stream operation and may load the code object, so it is not made
// while `s` is being captured into a graph: a first call under capture
// returns hipErrorStreamCaptureUnsupported (make one call outside the capture
// first).  A failed lookup is not kept: the next call tries again.
hipError_t scratch_ptr(hipStream_t s, void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  DeviceScratch& d = g_scratch[dev];
  if (void* p = d.ptr.load(std::memory_order_acquire)) {
    *out = p;
    return hipSuccess;
  }
  std::lock_guard<std::mutex> lock(d.mu);
  if (void* p = d.ptr.load(std::memory_order_acquire)) {
    *out = p;
    return hipSuccess;
  }
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  e = hipStreamIsCapturing(s, &cs);
  if (e != hipSuccess) return e;
  if (cs != hipStreamCaptureStatusNone) return hipErrorStreamCaptureUnsupported;
  void* p = nullptr;
  e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return e;
  if (p == nullptr || ((uintptr_t)p % 256) != 0) return hipErrorInvalidSymbol;
  d.ptr.store(p, std::memory_order_release);
  *out = p;
  return hipSuccess;
}

}  // namespace
}  // namespace rwkvmoe

extern "C" int rwkvmoe_forward_noalloc(const rwkvmoe_desc* desc, const rwkvmoe_tensors* t, void* stream) {
  using namespace rwkvmoe;
  // host-only checks first: argument errors never reach a HIP call
  const int st = forward_check(desc, t);
  if (st != RWKVMOE_OK) return st;
  size_t need = 0;
  if (rwkvmoe_workspace_bytes(desc, &need) != RWKVMOE_OK || need > kScratchBytes) return RWKVMOE_ERR_SCRATCH;
  void* ws = nullptr;
  const hipError_t e = scratch_ptr((hipStream_t)stream, &ws);
  if (e != hipSuccess) return (int)e;
  return rwkvmoe_forward(desc, t, ws, kScratchBytes, stream);
}
