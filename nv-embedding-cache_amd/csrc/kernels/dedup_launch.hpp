// dedup_launch.hpp -- host launchers of the dedup kernels (dedup.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nve_amd {

// k64[i] = key i as an unsigned sort key (sign bit flipped when flip != 0), v[i] = i.
hipError_t launch_dedup_prep(const void* keys, int key_bytes, int64_t n, int flip, uint64_t* k64,
                             uint32_t* v, hipStream_t stream);
hipError_t launch_dedup_outputs(const uint64_t* ks, const uint32_t* vs, const uint32_t* scan,
                                int64_t n, int key_bytes, void* unique, void* inverse,
                                void* offsets, uint32_t* start, uint32_t* pos_key,
                                hipStream_t stream);
// counts[u] for u < u_n, or for u < *u_dev when u_dev is given (u_n an upper bound).
hipError_t launch_dedup_counts(const uint32_t* start, uint32_t u_n, const uint32_t* u_dev,
                               int key_bytes, void* counts, hipStream_t stream);

}  // namespace nve_amd
