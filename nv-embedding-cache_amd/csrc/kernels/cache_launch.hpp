// cache_launch.hpp -- host launchers of the cache maintenance and modify kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nve_amd {

hipError_t launch_fill_tags(void* tags, int64_t count, int key_bytes, int64_t sentinel,
                            hipStream_t stream);
hipError_t launch_fill_u32(uint32_t* p, int64_t count, uint32_t v, hipStream_t stream);
hipError_t launch_fill_u64(uint64_t* p, int64_t count, uint64_t v, hipStream_t stream);
// *host_total = sum of words[0..n) (host_total: pinned host memory, written by
// the kernel); reset != 0 also zeroes the words.  One wave.
hipError_t launch_counter_total(unsigned long long* words, int n, unsigned long long* host_total, int reset,
                                hipStream_t stream);
// host_dst[0..bytes) = dev_src[0..bytes), bytes <= 64 (host_dst: pinned host
// memory, written by the kernel, one byte per lane).
hipError_t launch_small_read(void* host_dst, const void* dev_src, int bytes, hipStream_t stream);
hipError_t launch_cache_erase(void* tags, const void* keys, int64_t n, int key_bytes,
                              uint64_t num_sets, int64_t sentinel, hipStream_t stream);

}  // namespace nve_amd
