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
// Dedup positions outside every bag read no gradient row.
constexpr uint32_t kNoGradRow = 0xffffffffu;
// Positions per block of the summation order (a piece is one key's positions
// inside one block), and the number of sub-sequences a key's pieces are added
// in before their sums are added.
constexpr int kPieceBlock = 32;
constexpr int kPieceFanIn = 8;
constexpr int kCombineBlocks = 8;  // block entries per combine workgroup
constexpr int kLightPieces = 32;   // a crossing key of more pieces is added by a whole workgroup

// What the backprop needs per key position: how its gradient row and weight
// follow from its position (the bags, weights and bag denominators), and
// where they go (rows / nw, one entry per dedup position; rows null: none).
struct PositionGrad {
  int mode;             // kBackprop*
  const void* offsets;  // CSR offsets of the key type, or null (Fixed hotness)
  int key_bytes;
  int64_t num_bags;
  int64_t hotness;
  const void* weights;
  int wdt;
  const float* denom;   // Mean / WeightedMean: per bag
  uint32_t* rows;
  float* nw;
};

// rows / nw of every dedup position j from inverse[j] (its key position).
hipError_t launch_backprop_prep(const void* inverse, int key_bytes, int64_t n, const PositionGrad& g,
                                hipStream_t stream);

struct PieceArgs {
  const uint32_t* kidx;  // unique index of each dedup position
  const uint32_t* rows;  // gradient row of each dedup position (kNoGradRow: none)
  const float* nw;       // weight of each dedup position (weighted modes)
  const void* doff;      // first dedup position of each unique key (key type)
  const void* counts;    // positions of each unique key (key type)
  const uint8_t* grads;  // gradient rows, dim elements of the gradient type
  float* slots;          // two fp32 rows per block
  uint32_t* cross;       // per block: the key that starts in it and crosses out, or none
  uint8_t* out;          // one row per unique key, of the gradient type
  int64_t n;
  int32_t dim;
  int32_t key_bytes;
};

// Pieces: rows of keys inside one block, fp32 partial rows of the others.
hipError_t launch_piece_pool(const PieceArgs& a, int f16, int weighted, hipStream_t stream);
// The keys that cross a block edge, from their pieces.
hipError_t launch_piece_combine(const PieceArgs& a, int f16, hipStream_t stream);

}  // namespace nve_amd
