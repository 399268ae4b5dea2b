// backprop.cpp -- training backprop: the sparse gradient of a lookup with
// respect to the table (the reference's GradientCalculator::compute_gradients,
// cuda_ops/gradient_calculator.cuh:238-301, reached from pynve's
// concat_backprop / pooling_backprop, python/pynve/bindings/binding_layers.hpp:131-250).
//
//   keys -> dedup (unique keys ascending, stable inverse, the unique index of
//           every dedup position)                                  dedup.cpp
//        -> per dedup position: the gradient row it reads (its bag, or
//           its own position for Concatenate) and its weight        backprop.hip
//        -> piece_pool_kernel: each block of kPieceBlock dedup positions added
//           per key in position order (fp32); keys inside a block finished
//           there, pieces of keys crossing a block edge kept as fp32 rows and
//           each crossing key recorded in the block where it starts
//        -> piece_combine_kernel: each crossing key from its pieces (kPieceFanIn
//           sub-sequences, each in order, then their sums in order), rounded once
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
#include "runtime.hpp"

namespace nve_amd {

namespace {

size_t pad(size_t b) { return (b + 255) / 256 * 256; }

struct BackpropBufs {
  uint8_t* dedup_ws;
  size_t dedup_bytes;
  void *counts, *inverse, *doff;
  uint32_t *kidx, *rows, *cross;
  float *denom, *nw, *slots;
};

size_t slot_bytes(int64_t n, int64_t dim) {
  const int64_t blocks = (std::max<int64_t>(n, 1) + kPieceBlock - 1) / kPieceBlock;
  return pad(2 * (size_t)blocks * 4 * (size_t)std::max<int64_t>(dim, 1));
}

BackpropBufs carve(void* ws, int64_t n, int64_t num_bags) {
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
  b.kidx = reinterpret_cast<uint32_t*>(p);
  p += pad(4 * un);
  b.rows = reinterpret_cast<uint32_t*>(p);
  p += pad(4 * un);
  b.nw = reinterpret_cast<float*>(p);
  p += pad(4 * un);
  b.denom = reinterpret_cast<float*>(p);
  p += pad(4 * (size_t)std::max<int64_t>(num_bags, 1));
  b.cross = reinterpret_cast<uint32_t*>(p);  // one entry per block
  p += pad(4 * (un / kPieceBlock + 2));
  b.slots = reinterpret_cast<float*>(p);
  return b;
}

}  // namespace

size_t backprop_workspace_bytes(int64_t n, int64_t num_bags, int64_t dim) {
  const size_t un = (size_t)std::max<int64_t>(n, 1);
  return pad(dedup_workspace_bytes(n)) + 2 * pad(8 * un) + pad(8 * (un + 1)) + 3 * pad(4 * un) +
         pad(4 * (size_t)std::max<int64_t>(num_bags, 1)) + pad(4 * (un / kPieceBlock + 2)) +
         slot_bytes(n, dim);
}

int64_t pooling_backprop_run(int key_bytes, int64_t n, const void* keys, int pooling, int sparse,
                             const void* offsets, int64_t num_bags, int64_t hotness,
                             const void* weights, int wdt, const void* grads_in, int gdt,
                             int64_t dim, void* unique_out, void* grads_out, void* ws,
                             size_t ws_bytes, hipStream_t s, bool exact) {
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
  NVE_CHECK_ARG(dim <= INT32_MAX, "Invalid embedding width");
  NVE_CHECK_ARG(concat || num_bags < (int64_t)kNoGradRow, "Too many bags");
  const void* csr = (!concat && sparse == NVE_SPARSE_CSR) ? offsets : nullptr;
  BackpropBufs b = carve(ws, n, num_bags);

  // (1) bag denominators (Mean modes), then the dedup: unique keys straight
  // into the caller's buffer, and (2) on the way the gradient row and weight
  // of every dedup position (the unique count is read once everything is
  // queued: no stall in between)
  if (mode == kBackpropMean || mode == kBackpropWMean)
    NVE_HIP(launch_bag_denom(csr, key_bytes, num_bags, hotness, weights, wdt, mode == kBackpropWMean,
                             b.denom, s));
  const PositionGrad pg{mode, csr, key_bytes, num_bags, hotness, weights, wdt, b.denom, b.rows, b.nw};
  const DedupHead* head_dev = nullptr;
  dedup_run(key_bytes, n, keys, unique_out, b.counts, b.inverse, b.doff, b.dedup_ws, b.dedup_bytes, s,
            b.kidx, &head_dev, exact, &pg);

  // (3) pieces, then the keys that cross a block edge
  PieceArgs a{};
  a.kidx = b.kidx;
  a.rows = b.rows;
  a.nw = b.nw;
  a.doff = b.doff;
  a.counts = b.counts;
  a.grads = static_cast<const uint8_t*>(grads_in);
  a.slots = b.slots;
  a.cross = b.cross;
  a.out = static_cast<uint8_t*>(grads_out);
  a.n = n;
  a.dim = (int32_t)dim;
  a.key_bytes = key_bytes;
  const int f16 = gdt == kF16 ? 1 : 0;
  const int weighted = (mode == kBackpropWSum || mode == kBackpropMean || mode == kBackpropWMean) ? 1 : 0;
  NVE_HIP(launch_piece_pool(a, f16, weighted, s));
  NVE_HIP(launch_piece_combine(a, f16, s));
  const DedupHead h = read_back(head_dev, s);
  if (!exact && dedup_spec_failed(h))  // keys differ above the speculated sort bits: all again, exactly
    return pooling_backprop_run(key_bytes, n, keys, pooling, sparse, offsets, num_bags, hotness, weights, wdt,
                                grads_in, gdt, dim, unique_out, grads_out, ws, ws_bytes, s, true);
  return (int64_t)h.total;
}

}  // namespace nve_amd
