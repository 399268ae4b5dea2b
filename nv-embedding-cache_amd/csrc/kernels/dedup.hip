// dedup.hip -- key deduplication on the GPU (Deduper::dedup, deduper.cuh:136-221)
// and the dedup-ordered gather.
//
// dedup: stable radix sort of (key, position) -> run heads -> exclusive scan
// -> per run: unique key, start offset; per position: inverse = original
// position in key order; counts from consecutive starts.  Outputs match the
// reference's: unique keys ascending (signed order), counts, the stable
// inverse map and exclusive offsets.
#include "device_common.cuh"
#include "dedup_launch.hpp"

namespace nve_amd {

__global__ __launch_bounds__(256) void dedup_prep_kernel(const void* keys, int key_bytes, int64_t n,
                                                         int flip, uint64_t* k64, uint32_t* v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    const int64_t k = load_key(keys, key_bytes, i);
    k64[i] = flip ? flip_key(k, key_bytes) : (uint64_t)k;
    v[i] = (uint32_t)i;
  }
}

// inverse[i] = position of the i-th key in key order; at a run head:
// unique[u] = key, offsets[u] = i (= start[u]); start[U] = n.
__global__ __launch_bounds__(256) void dedup_outputs_kernel(const uint64_t* ks, const uint32_t* vs,
                                                            const uint32_t* scan, int64_t n,
                                                            int key_bytes, void* unique,
                                                            void* inverse, void* offsets,
                                                            uint32_t* start, uint32_t* pos_key) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  store_key(inverse, key_bytes, i, (int64_t)vs[i]);
  const bool head = (i == 0 || ks[i] != ks[i - 1]);
  if (pos_key != nullptr) pos_key[i] = head ? scan[i] : scan[i] - 1u;  // unique index of position i
  if (head) {
    const uint32_t u = scan[i];
    store_key(unique, key_bytes, u, unflip_key(ks[i], key_bytes));
    store_key(offsets, key_bytes, u, i);
    start[u] = (uint32_t)i;
  }
  if (i == n - 1) start[scan[i] + (head ? 1u : 0u)] = (uint32_t)n;
}

// u_dev (optional): the unique count in device memory, for a grid sized by an
// upper bound without reading the count back first.
__global__ __launch_bounds__(256) void dedup_counts_kernel(const uint32_t* start, uint32_t u_n,
                                                           const uint32_t* u_dev, int key_bytes,
                                                           void* counts) {
  const uint32_t u = blockIdx.x * blockDim.x + threadIdx.x;
  const uint32_t m = u_dev != nullptr ? *u_dev : u_n;
  if (u < m) store_key(counts, key_bytes, u, (int64_t)(start[u + 1] - start[u]));
}

hipError_t launch_dedup_prep(const void* keys, int key_bytes, int64_t n, int flip, uint64_t* k64,
                             uint32_t* v, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(dedup_prep_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, keys, key_bytes,
                     n, flip, k64, v);
  return hipGetLastError();
}

hipError_t launch_dedup_outputs(const uint64_t* ks, const uint32_t* vs, const uint32_t* scan,
                                int64_t n, int key_bytes, void* unique, void* inverse,
                                void* offsets, uint32_t* start, uint32_t* pos_key,
                                hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(dedup_outputs_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, ks, vs, scan,
                     n, key_bytes, unique, inverse, offsets, start, pos_key);
  return hipGetLastError();
}

hipError_t launch_dedup_counts(const uint32_t* start, uint32_t u_n, const uint32_t* u_dev,
                               int key_bytes, void* counts, hipStream_t stream) {
  if (u_n == 0) return hipSuccess;
  hipLaunchKernelGGL(dedup_counts_kernel, dim3((u_n + 255) / 256), dim3(256), 0, stream, start, u_n,
                     u_dev, key_bytes, counts);
  return hipGetLastError();
}

}  // namespace nve_amd
