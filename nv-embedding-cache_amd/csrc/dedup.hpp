// dedup.hpp -- key dedup and dedup-ordered gather (device buffers, caller workspace).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstddef>

namespace nve_amd {

size_t dedup_workspace_bytes(int64_t n);

// Sorted unique keys, counts, stable inverse map and exclusive offsets (all of
// the key type); returns the number of unique keys (synchronizes the stream).
// pos_key (optional, n entries): the unique index of each position of the
// dedup order.  count_dev (optional): instead of reading the count back (a
// stream synchronization), return -1 and point *count_dev at the count in the
// workspace (valid once the stream reaches it, until the workspace is reused).
int64_t dedup_run(int key_bytes, int64_t n, const void* keys, void* unique, void* counts,
                  void* inverse, void* offsets, void* ws, size_t ws_bytes, hipStream_t s,
                  uint32_t* pos_key = nullptr, const uint32_t** count_dev = nullptr);

// out[i] = table row keys[i] for keys in [0, num_rows), each distinct row read
// from the table once (asynchronous).
void dedup_gather_run(int key_bytes, int64_t n, const void* keys, const uint8_t* table,
                      int64_t num_rows, int64_t row_bytes, void* out, int64_t out_stride, void* ws,
                      size_t ws_bytes, hipStream_t s);

}  // namespace nve_amd
