// dedup.hpp -- key dedup and dedup-ordered gather (device buffers, caller workspace).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstddef>

#include "kernels/backprop_launch.hpp"

namespace nve_amd {

size_t dedup_workspace_bytes(int64_t n);

// The unique count and the key span of a dedup, side by side at the start of
// its workspace so that one readback fetches both.
struct DedupHead {
  uint32_t total;           // unique keys
  uint32_t pad;
  unsigned long long span;  // OR over the keys of key ^ key[0] (sort keys): the bits where they differ
};

// The sort first assumes that the keys differ only below this bit (rows of
// tables up to 2^27: three 9-bit passes) and learns whether they did from the
// span computed on the way, so no host round trip sits between the key
// preparation and the sort; a batch whose keys differ higher up is sorted
// again on its exact bits.
constexpr int kSpecSortBits = 27;
inline bool dedup_spec_failed(const DedupHead& h) { return (h.span >> kSpecSortBits) != 0; }

// Sorted unique keys, counts, stable inverse map and exclusive offsets (all of
// the key type); returns the number of unique keys (synchronizes the stream).
// pos_key (optional, n entries): the unique index of each position of the
// dedup order.  head_dev (optional): instead of reading the head back (a
// stream synchronization), return -1 and point *head_dev at the head in the
// workspace (valid once the stream reaches it, until the workspace is
// reused); the caller reads it and, if dedup_spec_failed, runs again with
// exact = true.  exact: read the key span back first and sort on exactly its
// bits (never needs a second run).
// pg (optional): also each dedup position's gradient row and weight (the
// backprop's per-position step, done on the way).
int64_t dedup_run(int key_bytes, int64_t n, const void* keys, void* unique, void* counts,
                  void* inverse, void* offsets, void* ws, size_t ws_bytes, hipStream_t s,
                  uint32_t* pos_key = nullptr, const DedupHead** head_dev = nullptr, bool exact = false,
                  const PositionGrad* pg = nullptr);

// out[i] = table row keys[i] for keys in [0, num_rows), each distinct row read
// from the table once (asynchronous).
void dedup_gather_run(int key_bytes, int64_t n, const void* keys, const uint8_t* table,
                      int64_t num_rows, int64_t row_bytes, void* out, int64_t out_stride, void* ws,
                      size_t ws_bytes, hipStream_t s);

}  // namespace nve_amd
