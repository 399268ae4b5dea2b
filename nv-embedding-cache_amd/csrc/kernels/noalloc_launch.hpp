// noalloc_launch.hpp -- device scratch of the allocation-free entry points.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace nve_amd {

// Bytes of the per-GPU scratch array (enough for the dedup-ordered gather of
// kNoAllocMaxKeys keys).
constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;
constexpr int64_t kNoAllocMaxKeys = 262144;

// Device address of the current GPU's scratch array (looked up once per
// device, then cached).  Callers on one GPU share it: calls that overlap race.
hipError_t noalloc_scratch(void** out);

}  // namespace nve_amd
