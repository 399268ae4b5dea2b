// cache.hip -- maintenance kernels of the 8-way set-associative cache:
// tag fill (init / clear), invalidate (erase) and a u64 fill used to zero
// counters without a memset node (safe under HIP graph capture).
//
// Reference: call_fill_tags (ec_set_associative.cuh:590-595),
// SetUpdateDataKernel<invalidate_only> + invalidate_tag_kernel
// (ec_set_associative_modify.cuh:516-561, ec_set_associative.cuh:240-261).
#include "device_common.cuh"
#include "cache_launch.hpp"

namespace nve_amd {

template <typename T>
__global__ __launch_bounds__(256) void fill_kernel(T* p, int64_t n, T v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// One lane per key: every way of the key's set whose rebuilt key equals the
// key gets the sentinel tag.
template <typename K, typename UK>
__global__ __launch_bounds__(256) void erase_kernel(K* tags, const K* keys, int64_t n, UK num_sets,
                                                    K sentinel) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const K key = keys[i];
  const UK set = (UK)key % num_sets;
  K* t = tags + (uint64_t)set * 8;
#pragma unroll
  for (int w = 0; w < 8; ++w) {
    const K tw = t[w];
    if ((K)((UK)tw * num_sets + set) == key) t[w] = sentinel;
  }
}

hipError_t launch_fill_tags(void* tags, int64_t count, int key_bytes, int64_t sentinel,
                            hipStream_t stream) {
  if (count <= 0) return hipSuccess;
  const int64_t grid = (count + 255) / 256;
  if (key_bytes == 4)
    hipLaunchKernelGGL(fill_kernel<int32_t>, dim3(grid), dim3(256), 0, stream, (int32_t*)tags,
                       count, (int32_t)sentinel);
  else
    hipLaunchKernelGGL(fill_kernel<int64_t>, dim3(grid), dim3(256), 0, stream, (int64_t*)tags,
                       count, (int64_t)sentinel);
  return hipGetLastError();
}

hipError_t launch_fill_u32(uint32_t* p, int64_t count, uint32_t v, hipStream_t stream) {
  if (count <= 0) return hipSuccess;
  hipLaunchKernelGGL(fill_kernel<uint32_t>, dim3((count + 255) / 256), dim3(256), 0, stream, p,
                     count, v);
  return hipGetLastError();
}

hipError_t launch_fill_u64(uint64_t* p, int64_t count, uint64_t v, hipStream_t stream) {
  if (count <= 0) return hipSuccess;
  hipLaunchKernelGGL(fill_kernel<uint64_t>, dim3((count + 255) / 256), dim3(256), 0, stream, p,
                     count, v);
  return hipGetLastError();
}

// *total = the sum of the counter's words, stored straight into pinned host
// memory (no copy operation behind the kernel); with reset, the words
// become 0 for the next count.
__global__ __launch_bounds__(64) void counter_total_kernel(unsigned long long* words, int n,
                                                           unsigned long long* total, int reset) {
  unsigned long long t = 0;
  for (int i = (int)threadIdx.x; i < n; i += 64) {
    t += words[i];
    if (reset) words[i] = 0;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) t += __shfl_xor(t, o);
  if (threadIdx.x == 0) *total = t;
}

hipError_t launch_counter_total(unsigned long long* words, int n, unsigned long long* host_total, int reset,
                                hipStream_t stream) {
  hipLaunchKernelGGL(counter_total_kernel, dim3(1), dim3(64), 0, stream, words, n, host_total, reset);
  return hipGetLastError();
}

// A readback of a few bytes (counts and spans between the launches of an
// insert or a dedup): one wave stores them into pinned host memory, which
// costs less than a copy-engine transfer queued behind the kernels.
__global__ __launch_bounds__(64) void small_read_kernel(const uint8_t* src, uint8_t* dst, int bytes) {
  const int i = (int)threadIdx.x;
  if (i < bytes) dst[i] = src[i];
}

hipError_t launch_small_read(void* host_dst, const void* dev_src, int bytes, hipStream_t stream) {
  if (bytes <= 0 || bytes > 64) return hipErrorInvalidValue;
  hipLaunchKernelGGL(small_read_kernel, dim3(1), dim3(64), 0, stream, static_cast<const uint8_t*>(dev_src),
                     static_cast<uint8_t*>(host_dst), bytes);
  return hipGetLastError();
}

hipError_t launch_cache_erase(void* tags, const void* keys, int64_t n, int key_bytes,
                              uint64_t num_sets, int64_t sentinel, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  const int64_t grid = (n + 255) / 256;
  if (key_bytes == 4)
    hipLaunchKernelGGL((erase_kernel<int32_t, uint32_t>), dim3(grid), dim3(256), 0, stream,
                       (int32_t*)tags, (const int32_t*)keys, n, (uint32_t)num_sets,
                       (int32_t)sentinel);
  else
    hipLaunchKernelGGL((erase_kernel<int64_t, uint64_t>), dim3(grid), dim3(256), 0, stream,
                       (int64_t*)tags, (const int64_t*)keys, n, (uint64_t)num_sets, sentinel);
  return hipGetLastError();
}

}  // namespace nve_amd
