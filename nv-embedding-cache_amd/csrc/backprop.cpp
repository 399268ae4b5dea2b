// backprop.cpp -- training backprop: the sparse gradient of a lookup with
// respect to the table (the reference's GradientCalculator::compute_gradients,
// cuda_ops/gradient_calculator.cuh:238-301, reached from pynve's
// concat_backprop / pooling_backprop, python/pynve/bindings/binding_layers.hpp:131-250).
//
//   keys -> dedup (unique keys ascending, stable inverse, runs)      dedup.cpp
//        -> per dedup position: the gradient row it reads (its bag, or
//           its own position for Concatenate) and its weight           backprop.hip
//        -> each key's positions cut into runs of at most kMaxRun
//        -> pool 1: one fp32 partial row per run (CSR over the runs, one lane
//           group per run, positions in order: acc + g, or fma(g, w, acc))
//        -> pool 2: the partials of each key added in run order, rounded
//           once to the gradient type                                  pool_kernel
// Deterministic, and bit-exact with the CPU oracle's statement of the same
// order.  The reference splits runs at 1024 positions and adds the pieces
// with atomics (its order is not fixed) and accumulates fp16 gradients in
// fp16; here every sum is fp32, rounded once.
#include <algorithm>

#include "backprop.hpp"
#include "dedup.hpp"
#include "kernels/backprop_launch.hpp"
#include "kernels/launch.hpp"
#include "kernels/sort_launch.hpp"
#include "layers.hpp"

namespace nve_amd {

namespace {

constexpr int64_t kMaxRun = 64;  // positions per run

size_t pad(size_t b) { return (b + 255) / 256 * 256; }

struct BackpropBufs {
  uint8_t* dedup_ws;
  size_t dedup_bytes;
  void *counts, *inverse, *doff, *rowkey, *run_off, *key_run_off;
  float *denom, *nw, *partials;
  uint32_t* nruns;
};

BackpropBufs carve(void* ws, int64_t n, int64_t num_bags, int64_t dim) {
  uint8_t* p = static_cast<uint8_t*>(ws);
  BackpropBufs b;
  const size_t un = (size_t)std::max<int64_t>(n, 1);
  b.dedup_ws = p;
  b.dedup_bytes = dedup_workspace_bytes(n);
  p += pad(b.dedup_bytes);
  b.counts = p;
  p += pad(8 * un);
  b.inverse = p;
  p += pad(8 * un);
  b.doff = p;
  p += pad(8 * (un + 1));
  b.rowkey = p;
  p += pad(8 * un);
  b.run_off = p;
  p += pad(8 * (un + 1));
  b.key_run_off = p;
  p += pad(8 * (un + 1));
  b.nruns = reinterpret_cast<uint32_t*>(p);
  p += pad(4 * (un + 1));
  b.denom = reinterpret_cast<float*>(p);
  p += pad(4 * (size_t)std::max<int64_t>(num_bags, 1));
  b.nw = reinterpret_cast<float*>(p);
  p += pad(4 * un);
  b.partials = reinterpret_cast<float*>(p);
  return b;
}

}  // namespace

size_t backprop_workspace_bytes(int64_t n, int64_t num_bags, int64_t dim) {
  const size_t un = (size_t)std::max<int64_t>(n, 1);
  return pad(dedup_workspace_bytes(n)) + 3 * pad(8 * un) + 3 * pad(8 * (un + 1)) +
         pad(4 * (un + 1)) + pad(4 * (size_t)std::max<int64_t>(num_bags, 1)) + pad(4 * un) +
         pad(4 * un * (size_t)std::max<int64_t>(dim, 1));
}

int64_t pooling_backprop_run(int key_bytes, int64_t n, const void* keys, int pooling, int sparse,
                             const void* offsets, int64_t num_bags, int64_t hotness,
                             const void* weights, int wdt, const void* grads_in, int gdt,
                             int64_t dim, void* unique_out, void* grads_out, void* ws,
                             size_t ws_bytes, hipStream_t s) {
  if (n <= 0) return 0;
  NVE_CHECK_ARG(key_bytes == 4 || key_bytes == 8, "Unsupported key size ", key_bytes);
  NVE_CHECK_ARG(gdt == kF32 || gdt == kF16, "Gradients must be float32 or float16");
  NVE_CHECK_ARG(dim > 0, "Invalid embedding width");
  NVE_CHECK_ARG(keys && grads_in && unique_out && grads_out, "keys and gradient buffers must not be NULL");
  NVE_CHECK_ARG(ws != nullptr && ws_bytes >= backprop_workspace_bytes(n, num_bags, dim), "Workspace too small");
  const bool concat = pooling == NVE_POOL_CONCATENATE;
  int mode = kBackpropConcat;
  if (!concat) {
    NVE_CHECK_ARG(num_bags >= 0, "Invalid number of bags");
    if (sparse == NVE_SPARSE_CSR) NVE_CHECK_ARG(offsets != nullptr, "CSR offsets must not be NULL");
    else NVE_CHECK_ARG(hotness > 0, "Fixed hotness must be positive");
    switch (pooling) {
      case NVE_POOL_SUM: mode = kBackpropSum; break;
      case NVE_POOL_WEIGHTED_SUM: mode = kBackpropWSum; break;
      case NVE_POOL_MEAN: mode = kBackpropMean; break;
      case NVE_POOL_WEIGHTED_MEAN: mode = kBackpropWMean; break;
      default: NVE_CHECK_ARG(false, "Unsupported pooling type ", pooling);
    }
    if (mode == kBackpropWSum || mode == kBackpropWMean) {
      NVE_CHECK_ARG(weights != nullptr, "Weighted pooling needs weights");
      NVE_CHECK_ARG(wdt == kF32 || wdt == kF16, "Weights must be float32 or float16");
    }
  }
  const void* csr = (!concat && sparse == NVE_SPARSE_CSR) ? offsets : nullptr;
  BackpropBufs b = carve(ws, n, num_bags, dim);

  // (1) dedup: unique keys straight into the caller's buffer
  const int64_t u = dedup_run(key_bytes, n, keys, unique_out, b.counts, b.inverse, b.doff, b.dedup_ws,
                              b.dedup_bytes, s);

  // (2) gradient row and weight per dedup position
  if (mode == kBackpropMean || mode == kBackpropWMean)
    NVE_HIP(launch_bag_denom(csr, key_bytes, num_bags, hotness, weights, wdt, mode == kBackpropWMean,
                             b.denom, s));
  const int64_t grad_rows = concat ? n : num_bags;
  NVE_HIP(launch_backprop_prep(b.inverse, key_bytes, n, mode, csr, num_bags, hotness, weights, wdt,
                               b.denom, grad_rows, b.rowkey, b.nw, s));

  // (3) runs of at most kMaxRun positions per unique key
  uint32_t* total = reinterpret_cast<uint32_t*>(b.dedup_ws);  // dedup's scratch is free again
  void* scan_tmp = b.dedup_ws + 256;
  NVE_HIP(launch_run_count(b.counts, key_bytes, u, kMaxRun, b.nruns, s));
  NVE_HIP(exclusive_scan_u32(b.nruns, u, total, scan_tmp, s));
  const uint32_t runs = read_back(total, s);
  NVE_HIP(launch_run_write(b.doff, key_bytes, u, n, kMaxRun, b.nruns, runs, b.run_off, b.key_run_off, s));

  const int ges = gdt == kF16 ? 2 : 4;
  // (4) one fp32 partial row per run, positions in order
  PoolLaunch p1{};
  p1.keys = b.rowkey;
  p1.key_bytes = key_bytes;
  p1.num_keys = n;
  p1.offsets = b.run_off;
  p1.num_bags = runs;
  p1.weighted = (mode == kBackpropWSum || mode == kBackpropMean || mode == kBackpropWMean) ? 1 : 0;
  p1.weights = b.nw;
  p1.weight_dtype = kF32;
  p1.src.table = static_cast<const uint8_t*>(grads_in);
  p1.src.row_bytes = (uint64_t)(dim * ges);
  p1.src.load_indices = 1;
  p1.src.num_rows = (uint64_t)grad_rows;  // positions in no bag read nothing
  p1.stored_dtype = gdt;
  p1.count = dim;
  p1.out = b.partials;
  p1.out_stride = dim * 4;
  p1.out_dtype = kF32;
  p1.force_split = -1;  // one lane group per run: position order
  NVE_HIP(launch_pool(p1, s));

  // (5) each key's partials added in run order, rounded once
  PoolLaunch p2{};
  p2.key_bytes = key_bytes;
  p2.num_keys = runs;
  p2.offsets = b.key_run_off;
  p2.num_bags = u;
  p2.src.table = reinterpret_cast<const uint8_t*>(b.partials);
  p2.src.row_bytes = (uint64_t)(dim * 4);
  p2.src.load_indices = 0;  // row = run index
  p2.src.num_rows = runs;
  p2.stored_dtype = kF32;
  p2.count = dim;
  p2.out = grads_out;
  p2.out_stride = dim * ges;
  p2.out_dtype = gdt;
  p2.force_split = -1;
  NVE_HIP(launch_pool(p2, s));
  return u;
}

}  // namespace nve_amd
