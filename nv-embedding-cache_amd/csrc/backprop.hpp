// backprop.hpp -- training backprop: sparse gradient of a lookup (device buffers, caller workspace).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstddef>

namespace nve_amd {

size_t backprop_workspace_bytes(int64_t n, int64_t num_bags, int64_t dim);

// Unique keys ascending into unique_out (key type) and one gradient row per
// unique key into grads_out (dim values of the gradient type); returns the
// number of unique keys (synchronizes the stream).  grads_in: one row per bag
// (pooled) or per key position (pooling == NVE_POOL_CONCATENATE).
int64_t pooling_backprop_run(int key_bytes, int64_t n, const void* keys, int pooling, int sparse,
                             const void* offsets, int64_t num_bags, int64_t hotness,
                             const void* weights, int wdt, const void* grads_in, int gdt,
                             int64_t dim, void* unique_out, void* grads_out, void* ws,
                             size_t ws_bytes, hipStream_t s, bool exact = false);

}  // namespace nve_amd
