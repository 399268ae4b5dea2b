// noalloc_launch.hpp -- device scratch of the allocation-free entry points.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <mutex>

namespace nve_amd {

// Bytes of the per-GPU scratch array (enough for the dedup-ordered gather of
// kNoAllocMaxKeys keys).
constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;
constexpr int64_t kNoAllocMaxKeys = 262144;

// One allocation-free call on the current GPU.  begin(s) takes the GPU's
// host lock, sets the GPU up on its first call (the scratch array's device
// address from hipGetSymbolAddress, one completion event) and makes s wait
// for the previous call's work on that GPU, on any stream; device_scratch() is then
// this GPU's array.  end() records the completion event behind the work just
// issued on s and releases the lock (the destructor does so too, for a call
// that throws).  So calls on one GPU run one after another in the order they
// were issued, from any thread or stream.  Under graph capture of s the
// event is neither waited for nor recorded: the graph's own stream order
// applies, and replays that overlap other calls on the GPU race.
class NoAllocSession {
 public:
  NoAllocSession() = default;
  NoAllocSession(const NoAllocSession&) = delete;
  NoAllocSession& operator=(const NoAllocSession&) = delete;
  ~NoAllocSession();
  hipError_t begin(hipStream_t s);
  void* device_scratch() const { return scratch_; }
  hipError_t end();

 private:
  int dev_ = -1;
  bool order_ = false;
  hipStream_t stream_ = nullptr;
  void* scratch_ = nullptr;
  std::unique_lock<std::mutex> lock_;
};

}  // namespace nve_amd
