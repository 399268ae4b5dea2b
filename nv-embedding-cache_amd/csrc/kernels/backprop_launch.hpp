// backprop_launch.hpp -- host launchers of the training backprop helper kernels (backprop.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nve_amd {

// how a key position weighs its gradient row
enum { kBackpropConcat = 0, kBackpropSum = 1, kBackpropWSum = 2, kBackpropMean = 3, kBackpropWMean = 4 };

hipError_t launch_bag_denom(const void* offsets, int key_bytes, int64_t num_bags, int64_t hotness,
                            const void* weights, int wdt, int wmean, float* denom,
                            hipStream_t stream);
hipError_t launch_backprop_prep(const void* inverse, int key_bytes, int64_t n, int mode,
                                const void* offsets, int64_t num_bags, int64_t hotness,
                                const void* weights, int wdt, const float* denom, int64_t none_row,
                                void* rowkey, float* nw, hipStream_t stream);
hipError_t launch_run_count(const void* counts, int key_bytes, int64_t u, int64_t max_run,
                            uint32_t* nruns, hipStream_t stream);
hipError_t launch_run_write(const void* doff, int key_bytes, int64_t u, int64_t n, int64_t max_run,
                            const uint32_t* run_scan, uint32_t total, void* run_off, void* key_run_off,
                            hipStream_t stream);

}  // namespace nve_amd
