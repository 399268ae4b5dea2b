// uvm_gather_launch.hpp -- the two alternative miss paths of a cached lookup
// over a host-resident backing table (uvm_gather.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "launch.hpp"

namespace nve_amd {

// SortGather step 1: one sort key per lookup key -- misses first, then hits,
// each in ascending key order: ((hit << bits) | k), k the key clamped to all
// ones in `bits` (keys that resolve to no row too); pos[i] = i.  Adds the
// misses to *miss_counter and *call_misses (either may be null).
hipError_t launch_sortgather_keys(const void* keys, int64_t n, int key_bytes, const RowSource& src,
                                  int bits, uint64_t* sort_key, uint32_t* pos,
                                  unsigned long long* miss_counter,
                                  unsigned long long* call_misses, hipStream_t stream);
// out[j] = keys[pos[j]] in the key type.
hipError_t launch_permute_keys(const void* keys, int key_bytes, const uint32_t* pos, int64_t n,
                               void* out, hipStream_t stream);
// out + pos[j]*out_stride <- staging + j*row_bytes, for j < count (the
// staging rows and positions may be pinned host memory).
hipError_t launch_scatter_rows(const uint8_t* staging, const uint32_t* pos, int64_t count,
                               uint64_t row_bytes, uint8_t* out, int64_t out_stride,
                               hipStream_t stream);

}  // namespace nve_amd
