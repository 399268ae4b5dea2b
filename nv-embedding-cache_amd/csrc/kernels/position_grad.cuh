// position_grad.cuh -- the gradient row and weight of one key position of a
// training backprop, shared by backprop_prep_kernel and the dedup's run
// outputs (which compute them on the way when the backprop asks).
//
// Reference behaviour restated: compute_normalized_weights and
// compute_pooling_inverse_mapping (cuda_ops/gradient_calculator.cuh:29-82).
#pragma once

#include "backprop_launch.hpp"
#include "device_common.cuh"

namespace nve_amd {

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

// For dedup position j holding key position p: rows[j] = the gradient row it
// reads (Concatenate: p; pooled: its bag, or kNoGradRow outside every bag),
// nw[j] = its weight (1, w[p], 1 / count or w[p] / sum of the bag's weights).
__device__ __forceinline__ void position_grad(const PositionGrad& g, int64_t j, int64_t p) {
  uint32_t row = (uint32_t)p;
  float w = 1.0f;
  if (g.mode != kBackpropConcat) {
    const int64_t b = bag_of(p, g.offsets, g.key_bytes, g.num_bags, g.hotness);
    row = b < 0 ? kNoGradRow : (uint32_t)b;
    if (b >= 0) {
      if (g.mode == kBackpropWSum) w = load_weight(g.weights, g.wdt, p);
      else if (g.mode == kBackpropMean) w = 1.0f / g.denom[b];
      else if (g.mode == kBackpropWMean) w = load_weight(g.weights, g.wdt, p) / g.denom[b];
    }
  }
  g.rows[j] = row;
  g.nw[j] = w;
}

}  // namespace nve_amd
