// sort.hip -- stable LSD radix sort of (uint64 key, uint32 value) pairs, an
// exclusive scan and a key-span reduction: the sorting primitives behind the
// cache insert (histogram and set grouping) and dedup.
//
// The reference uses CUB (cub::DeviceRadixSort::SortPairs[Descending],
// DeviceRunLengthEncode::Encode, DeviceScan::ExclusiveSum; deduper.cuh:157-200,
// gather_keys_data_ptrs.cuh:154-183, ec_set_associative_modify.cuh:472-497).
// Only the mathematical results matter (a stable sort; descending sorts are
// expressed by the caller as ascending sorts of a complemented key).
//
// One pass per 8-bit digit, three kernels per pass:
//   hist     each 256-thread workgroup counts the digits of its 2048-key tile
//            into LDS and writes the 256 counts digit-major;
//   scan     one workgroup turns the digit-major counts into exclusive offsets
//            (digit d of tile t lands after every smaller digit and after
//            digit d of tiles < t: this is what makes the pass stable);
//   scatter  each workgroup ranks its keys stably: a wave finds the lanes
//            sharing its digit with eight ballots, ranks by popcount of the
//            lower lanes, and adds the counts of earlier waves and rounds.
#include "device_common.cuh"
#include "sort_launch.hpp"

namespace nve_amd {

constexpr int kSortThreads = 256;
constexpr int kSortItems = 8;
constexpr int kSortTile = kSortThreads * kSortItems;

__global__ __launch_bounds__(256) void radix_hist_kernel(const uint64_t* keys, int64_t n, int shift,
                                                         uint32_t* counts, int nblocks) {
  __shared__ uint32_t h[256];
  const int tid = threadIdx.x;
  h[tid] = 0;
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * kSortTile;
#pragma unroll
  for (int r = 0; r < kSortItems; ++r) {
    const int64_t i = base + r * kSortThreads + tid;
    if (i < n) atomicAdd(&h[(keys[i] >> shift) & 255u], 1u);
  }
  __syncthreads();
  counts[(int64_t)tid * nblocks + blockIdx.x] = h[tid];
}

// Exclusive scan of m uint32 in place by one 1024-thread workgroup: thread t
// owns a contiguous chunk, chunks are summed, the chunk sums scanned in LDS,
// then each chunk rewritten with its running prefix.  Also writes the total.
__global__ __launch_bounds__(1024) void scan_kernel(uint32_t* data, int64_t m, uint32_t* total) {
  __shared__ uint32_t sums[1024];
  const int tid = threadIdx.x;
  const int64_t chunk = (m + 1023) / 1024;
  const int64_t b = tid * chunk;
  const int64_t e = b + chunk < m ? b + chunk : m;
  uint32_t s = 0;
  for (int64_t i = b; i < e; ++i) s += data[i];
  sums[tid] = s;
  __syncthreads();
  // Hillis-Steele inclusive scan of the 1024 chunk sums
  for (int o = 1; o < 1024; o <<= 1) {
    const uint32_t v = tid >= o ? sums[tid - o] : 0u;
    __syncthreads();
    sums[tid] += v;
    __syncthreads();
  }
  uint32_t run = tid > 0 ? sums[tid - 1] : 0u;
  for (int64_t i = b; i < e; ++i) {
    const uint32_t v = data[i];
    data[i] = run;
    run += v;
  }
  if (tid == 1023 && total != nullptr) *total = sums[1023];
}

__global__ __launch_bounds__(256) void radix_scatter_kernel(const uint64_t* keys, const uint32_t* vals,
                                                            uint64_t* ko, uint32_t* vo, int64_t n,
                                                            int shift, const uint32_t* offsets,
                                                            int nblocks) {
  __shared__ uint32_t run[256];
  __shared__ uint32_t wcnt[4][256];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  run[tid] = offsets[(int64_t)tid * nblocks + blockIdx.x];
#pragma unroll
  for (int w = 0; w < 4; ++w) wcnt[w][tid] = 0;
  __syncthreads();
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const int64_t base = (int64_t)blockIdx.x * kSortTile;
  for (int r = 0; r < kSortItems; ++r) {
    const int64_t i = base + r * kSortThreads + tid;
    const bool valid = i < n;
    const uint64_t k = valid ? keys[i] : 0ull;
    const uint32_t v = valid ? vals[i] : 0u;
    const uint32_t d = (uint32_t)(k >> shift) & 255u;
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const uint64_t m = __ballot((d >> b) & 1u);
      peers &= ((d >> b) & 1u) ? m : ~m;
    }
    const uint32_t rank = (uint32_t)__popcll(peers & lt_mask);
    const bool leader = valid && (peers & lt_mask) == 0;
    if (leader) wcnt[wave][d] = (uint32_t)__popcll(peers);
    __syncthreads();
    if (valid) {
      uint32_t pos = run[d] + rank;
      for (int w = 0; w < wave; ++w) pos += wcnt[w][d];
      ko[pos] = k;
      vo[pos] = v;
    }
    __syncthreads();
    run[tid] += wcnt[0][tid] + wcnt[1][tid] + wcnt[2][tid] + wcnt[3][tid];
#pragma unroll
    for (int w = 0; w < 4; ++w) wcnt[w][tid] = 0;
    __syncthreads();
  }
}

// OR over i of keys[i] ^ keys[0]: the bits where keys differ.
__global__ __launch_bounds__(256) void key_span_kernel(const uint64_t* keys, int64_t n,
                                                       unsigned long long* out) {
  const uint64_t k0 = keys[0];
  uint64_t acc = 0;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    acc |= keys[i] ^ k0;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) acc |= __shfl_xor(acc, o);
  if ((threadIdx.x & 63) == 0 && acc) atomicOr(out, (unsigned long long)acc);
}

// ---------------------------------------------------------------------------
size_t radix_sort_temp_bytes(int64_t n) {
  const int64_t nblocks = (n + kSortTile - 1) / kSortTile;
  return (size_t)(nblocks > 0 ? nblocks : 1) * 256 * sizeof(uint32_t) + 256;
}

hipError_t radix_sort_pairs(uint64_t* keys, uint32_t* vals, uint64_t* keys_alt, uint32_t* vals_alt,
                            int64_t n, int begin_bit, int end_bit, void* temp, int* result_in_alt,
                            hipStream_t stream) {
  *result_in_alt = 0;
  if (n <= 1 || end_bit <= begin_bit) return hipSuccess;
  const int64_t nblocks = (n + kSortTile - 1) / kSortTile;
  if (nblocks > 0x7fffffff) return hipErrorInvalidValue;
  uint32_t* counts = static_cast<uint32_t*>(temp);
  uint64_t* ki = keys;
  uint32_t* vi = vals;
  uint64_t* ka = keys_alt;
  uint32_t* va = vals_alt;
  for (int shift = begin_bit; shift < end_bit; shift += 8) {
    hipLaunchKernelGGL(radix_hist_kernel, dim3(nblocks), dim3(kSortThreads), 0, stream, ki, n,
                       shift, counts, (int)nblocks);
    hipLaunchKernelGGL(scan_kernel, dim3(1), dim3(1024), 0, stream, counts, nblocks * 256,
                       (uint32_t*)nullptr);
    hipLaunchKernelGGL(radix_scatter_kernel, dim3(nblocks), dim3(kSortThreads), 0, stream, ki, vi,
                       ka, va, n, shift, counts, (int)nblocks);
    std::swap(ki, ka);
    std::swap(vi, va);
    *result_in_alt ^= 1;
  }
  return hipGetLastError();
}

hipError_t exclusive_scan_u32(uint32_t* data, int64_t m, uint32_t* total, hipStream_t stream) {
  if (m <= 0) return hipSuccess;
  hipLaunchKernelGGL(scan_kernel, dim3(1), dim3(1024), 0, stream, data, m, total);
  return hipGetLastError();
}

hipError_t key_span(const uint64_t* keys, int64_t n, unsigned long long* out, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  int64_t grid = (n + 255) / 256;
  if (grid > 1024) grid = 1024;
  hipLaunchKernelGGL(key_span_kernel, dim3(grid), dim3(256), 0, stream, keys, n, out);
  return hipGetLastError();
}

}  // namespace nve_amd
