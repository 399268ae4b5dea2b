// backprop.hip -- helper kernels of the training backprop (the sparse gradient
// of a lookup): bag denominators, the gradient row and weight of every key
// position in dedup order, and the cutting of each unique key's positions
// into runs.  The gradient sums themselves run on pool_kernel (CSR, one lane
// group per run, key order), see csrc/backprop.cpp.
//
// Reference behaviour restated: GradientCalculator::compute_gradients
// (cuda_ops/gradient_calculator.cuh:238-301): compute_normalized_weights
// (:29-63), compute_pooling_inverse_mapping (:65-82), compute_pooling_gradients
// (:84-135); GradientDedup (cuda_ops/dedup_grads_kernel.cuh:57-107).
#include "backprop_launch.hpp"
#include "device_common.cuh"

namespace nve_amd {

namespace {

// [s, e) of bag b (Fixed: b*hotness; CSR: the caller's offsets)
__device__ __forceinline__ void bag_range(const void* offsets, int key_bytes, int64_t hotness,
                                          int64_t b, int64_t* s, int64_t* e) {
  if (offsets == nullptr) {
    *s = b * hotness;
    *e = *s + hotness;
  } else {
    *s = load_key(offsets, key_bytes, b);
    *e = load_key(offsets, key_bytes, b + 1);
  }
}

// Mean: the bag's key count; WeightedMean: its weights added in position order.
__global__ __launch_bounds__(256) void bag_denom_kernel(const void* offsets, int key_bytes,
                                                        int64_t num_bags, int64_t hotness,
                                                        const void* weights, int wdt, int wmean,
                                                        float* denom) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= num_bags) return;
  int64_t s, e;
  bag_range(offsets, key_bytes, hotness, b, &s, &e);
  if (!wmean) {
    denom[b] = (float)(e - s);
    return;
  }
  float acc = 0.0f;
  for (int64_t p = s; p < e; ++p) acc += load_weight(weights, wdt, p);
  denom[b] = acc;
}

// bag holding position p, or -1 (Fixed: p / hotness; CSR: binary search for
// the last b with offsets[b] <= p, valid when p < offsets[b + 1])
__device__ __forceinline__ int64_t bag_of(int64_t p, const void* offsets, int key_bytes,
                                          int64_t num_bags, int64_t hotness) {
  if (offsets == nullptr) {
    const int64_t b = hotness > 0 ? p / hotness : -1;
    return (b >= 0 && b < num_bags) ? b : -1;
  }
  if (num_bags <= 0 || load_key(offsets, key_bytes, 0) > p) return -1;
  int64_t lo = 0, hi = num_bags;
  while (hi - lo > 1) {
    const int64_t mid = (lo + hi) >> 1;
    if (load_key(offsets, key_bytes, mid) <= p) lo = mid;
    else hi = mid;
  }
  return p < load_key(offsets, key_bytes, lo + 1) ? lo : -1;
}

// For dedup position j (key position p = inverse[j]): the gradient row it
// reads (Concatenate: p; pooled: its bag, or none_row outside every bag) and
// its weight (1, w[p], 1 / count or w[p] / sum of the bag's weights).
__global__ __launch_bounds__(256) void backprop_prep_kernel(
    const void* inverse, int key_bytes, int64_t n, int mode, const void* offsets, int64_t num_bags,
    int64_t hotness, const void* weights, int wdt, const float* denom, int64_t none_row,
    void* rowkey, float* nw) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= n) return;
  const int64_t p = load_key(inverse, key_bytes, j);
  int64_t row = p;
  float w = 1.0f;
  if (mode != kBackpropConcat) {
    const int64_t b = bag_of(p, offsets, key_bytes, num_bags, hotness);
    row = b < 0 ? none_row : b;
    if (b >= 0) {
      if (mode == kBackpropWSum) w = load_weight(weights, wdt, p);
      else if (mode == kBackpropMean) w = 1.0f / denom[b];
      else if (mode == kBackpropWMean) w = load_weight(weights, wdt, p) / denom[b];
    }
  }
  store_key(rowkey, key_bytes, j, row);
  nw[j] = w;
}

__global__ __launch_bounds__(256) void run_count_kernel(const void* counts, int key_bytes, int64_t u,
                                                        int64_t max_run, uint32_t* nruns) {
  const int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= u) return;
  const int64_t c = load_key(counts, key_bytes, k);
  nruns[k] = (uint32_t)((c + max_run - 1) / max_run);
}

// run_off: run r covers dedup positions [run_off[r], run_off[r + 1]);
// key_run_off: key k owns runs [key_run_off[k], key_run_off[k + 1]).  One
// thread per run (its key found by binary search in the exclusive scan of
// the run counts, every key owning at least one run) and per key.
__global__ __launch_bounds__(256) void run_write_kernel(const void* doff, int key_bytes, int64_t u,
                                                        int64_t n, int64_t max_run,
                                                        const uint32_t* run_scan, uint32_t total,
                                                        void* run_off, void* key_run_off) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < (int64_t)total) {
    int64_t lo = 0, hi = u;  // last k with run_scan[k] <= i
    while (hi - lo > 1) {
      const int64_t mid = (lo + hi) >> 1;
      if ((int64_t)run_scan[mid] <= i) lo = mid;
      else hi = mid;
    }
    store_key(run_off, key_bytes, i, load_key(doff, key_bytes, lo) + (i - (int64_t)run_scan[lo]) * max_run);
  }
  if (i < u) store_key(key_run_off, key_bytes, i, run_scan[i]);
  if (i == 0) {
    store_key(run_off, key_bytes, total, n);
    store_key(key_run_off, key_bytes, u, total);
  }
}

}  // namespace

hipError_t launch_bag_denom(const void* offsets, int key_bytes, int64_t num_bags, int64_t hotness,
                            const void* weights, int wdt, int wmean, float* denom,
                            hipStream_t stream) {
  if (num_bags <= 0) return hipSuccess;
  hipLaunchKernelGGL(bag_denom_kernel, dim3((unsigned)((num_bags + 255) / 256)), dim3(256), 0, stream,
                     offsets, key_bytes, num_bags, hotness, weights, wdt, wmean, denom);
  return hipGetLastError();
}

hipError_t launch_backprop_prep(const void* inverse, int key_bytes, int64_t n, int mode,
                                const void* offsets, int64_t num_bags, int64_t hotness,
                                const void* weights, int wdt, const float* denom, int64_t none_row,
                                void* rowkey, float* nw, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(backprop_prep_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                     inverse, key_bytes, n, mode, offsets, num_bags, hotness, weights, wdt, denom,
                     none_row, rowkey, nw);
  return hipGetLastError();
}

hipError_t launch_run_count(const void* counts, int key_bytes, int64_t u, int64_t max_run,
                            uint32_t* nruns, hipStream_t stream) {
  if (u <= 0) return hipSuccess;
  hipLaunchKernelGGL(run_count_kernel, dim3((unsigned)((u + 255) / 256)), dim3(256), 0, stream, counts,
                     key_bytes, u, max_run, nruns);
  return hipGetLastError();
}

hipError_t launch_run_write(const void* doff, int key_bytes, int64_t u, int64_t n, int64_t max_run,
                            const uint32_t* run_scan, uint32_t total, void* run_off, void* key_run_off,
                            hipStream_t stream) {
  if (u <= 0) return hipSuccess;
  const int64_t m = (int64_t)total > u ? (int64_t)total : u;
  hipLaunchKernelGGL(run_write_kernel, dim3((unsigned)((m + 255) / 256)), dim3(256), 0, stream, doff,
                     key_bytes, u, n, max_run, run_scan, total, run_off, key_run_off);
  return hipGetLastError();
}

}  // namespace nve_amd
