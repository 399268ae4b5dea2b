// noalloc.hip -- the device scratch of the entry points that allocate nothing
// (nve_amd_dedup_gather_noalloc): a file-scope device array, one copy per GPU,
// reached from host code only through the address hipGetSymbolAddress returns
// for the current device (the array's name in host code is a host-side
// stand-in, not a device address).
//
// Calls on one GPU share its array, so they are put in one order: each call
// issues its work under the device's host lock, makes its stream wait for the
// completion event of the call issued before it (on whatever stream that was)
// and records the event again behind its own work.  The event is made once
// per device, at set-up, next to the symbol lookup; no call after that makes
// or frees anything.
#include <hip/hip_runtime.h>

#include <mutex>

#include "noalloc_launch.hpp"

namespace nve_amd {

static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;

struct DeviceSlot {
  std::mutex mu;             // held from begin() to end(): one caller issues at a time
  void* ptr = nullptr;       // this device's copy of `scratch`
  hipEvent_t done = nullptr; // recorded behind the last call's work
  bool recorded = false;     // done has been recorded at least once
};
DeviceSlot g_slots[kMaxDevices];

bool capturing(hipStream_t s) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(s, &st) == hipSuccess && st == hipStreamCaptureStatusActive;
}
}  // namespace

hipError_t NoAllocSession::begin(hipStream_t s) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  DeviceSlot& slot = g_slots[dev];
  std::unique_lock<std::mutex> lk(slot.mu);
  if (slot.ptr == nullptr) {
    // set-up, once per device with that device current: its own copy of the
    // array, and the event that orders the calls
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (p == nullptr) return hipErrorInvalidSymbol;
    e = hipEventCreateWithFlags(&slot.done, hipEventDisableTiming);
    if (e != hipSuccess) return e;
    slot.ptr = p;
  }
  // under graph capture the captured stream's own order is the only order
  // (an event recorded outside the capture cannot be waited on inside it)
  order_ = !capturing(s);
  if (order_ && slot.recorded) {
    e = hipStreamWaitEvent(s, slot.done, 0);
    if (e != hipSuccess) return e;
  }
  dev_ = dev;
  stream_ = s;
  scratch_ = slot.ptr;
  lock_ = std::move(lk);
  return hipSuccess;
}

hipError_t NoAllocSession::end() {
  if (dev_ < 0) return hipSuccess;
  DeviceSlot& slot = g_slots[dev_];
  hipError_t e = hipSuccess;
  if (order_) {
    e = hipEventRecord(slot.done, stream_);
    if (e == hipSuccess) slot.recorded = true;
  }
  dev_ = -1;
  lock_.unlock();
  return e;
}

NoAllocSession::~NoAllocSession() {
  // a call that failed part way still orders what it issued before the next
  if (dev_ >= 0) (void)end();
}

}  // namespace nve_amd
