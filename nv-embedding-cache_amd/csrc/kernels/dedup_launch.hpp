// dedup_launch.hpp -- host launchers of the dedup kernels (dedup.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "backprop_launch.hpp"

namespace nve_amd {

// Words of the key-span parts the radix sort's first pass writes for n keys
// (one per tile, radix_tiles(n)).
int64_t dedup_span_parts(int64_t n);
// k64[i] = key i as an unsigned sort key (sign bit flipped when flip != 0), v[i] = i.
hipError_t launch_dedup_prep(const void* keys, int key_bytes, int64_t n, int flip, uint64_t* k64,
                             uint32_t* v, hipStream_t stream);
// Outputs from the sorted keys and the run-head scan; with span_part
// (dedup_span_parts(n) words), also *span_out = OR of the span parts.
hipError_t launch_dedup_outputs(const uint64_t* ks, const uint32_t* vs, const uint32_t* scan,
                                int64_t n, int key_bytes, void* unique, void* inverse,
                                void* offsets, uint32_t* start, uint32_t* pos_key,
                                const uint64_t* span_part, unsigned long long* span_out,
                                hipStream_t stream);
// The runs of sorted keys ks (values vs) in two launches: unique keys, counts,
// inverse and offsets of the key type, pos_key (optional) the unique index of
// every position, *total the unique count; with span_part, also *span_out as
// launch_dedup_outputs; with pg, each dedup position's gradient row and
// weight (as launch_backprop_prep).  Scratch: blk_count / blk_last,
// run_blocks(n) words each.  At most kRunMaxBlocks blocks
// (hipErrorInvalidValue beyond).
constexpr int64_t kRunMaxBlocks = 4096;
int64_t run_blocks(int64_t n);
hipError_t launch_dedup_runs(const uint64_t* ks, const uint32_t* vs, int64_t n, int key_bytes, void* unique,
                             void* counts, void* inverse, void* offsets, uint32_t* pos_key, uint32_t* total,
                             uint32_t* blk_count, int64_t* blk_last, const uint64_t* span_part,
                             unsigned long long* span_out, const PositionGrad* pg, hipStream_t stream);
// counts[u] for u < u_n, or for u < *u_dev when u_dev is given (u_n an upper bound).
hipError_t launch_dedup_counts(const uint32_t* start, uint32_t u_n, const uint32_t* u_dev,
                               int key_bytes, void* counts, hipStream_t stream);

// Hash slots for a batch of n keys: a power of two, at least 2n (and 1024).
size_t hash_dedup_slots(int64_t n);
// Bytes per hash-table key: 4 when every row index fits 32 bits, else 8.
size_t hash_dedup_key_bytes(int64_t num_rows);
// out row i = table row keys[i] for keys in [0, num_rows) (others untouched),
// deduplicated by hashing.  Scratch: tab (hash_dedup_slots(n) 8-byte slots:
// key and owner position when hash_dedup_key_bytes(num_rows) is 4, else the
// key), owner (one word per slot, 8-byte keys only) and slot_of (n words:
// each position's owner, or with 8-byte keys its slot).  Three launches,
// asynchronous.
hipError_t launch_hash_dedup_gather(const void* keys, int key_bytes, int64_t n, const uint8_t* table,
                                    int64_t num_rows, int64_t row_bytes, void* out, int64_t out_stride,
                                    void* tab, uint32_t* owner, uint32_t* slot_of, hipStream_t stream);

}  // namespace nve_amd
