// update_launch.hpp -- host launchers of the row-update kernels (update.hip):
// overwrite or accumulate rows of the cache (resident keys only) and of a
// linear table (keys inside the table only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nve_amd {

// Record i for key i of keys[0..n): the slot set*8+way of its first
// matching way (rebuilt key equal to it, empty ways included, as the
// reference compares them), the tag to commit (own_tag: the key's own tag,
// key / num_sets, as the device policy records it; else the way's current
// tag, as the host policy does) and the address of the key's update row
// (values + i*stride); kNoRecord as the slot when no way matches.  A key
// matching several ways sets *multi (a pinned host word the caller zeroes):
// then launch_update_more_records records the further ways.
hipError_t launch_update_records(const void* keys, int64_t n, int key_bytes, const void* tags,
                                 uint64_t num_sets, const uint8_t* values, int64_t value_stride,
                                 uint64_t* rec_slot, int64_t* rec_tag, uint64_t* rec_src,
                                 uint32_t* multi, bool own_tag, hipStream_t stream);
// The second and later matching ways of every key of keys[0..n) (device
// policy: each with the key's own tag): records [0, *count) (*count zeroed
// by the caller), at most cap of them.
hipError_t launch_update_more_records(const void* keys, int64_t n, int key_bytes, const void* tags,
                                      uint64_t num_sets, const uint8_t* values, int64_t value_stride,
                                      uint64_t* rec_slot, int64_t* rec_tag, uint64_t* rec_src,
                                      uint32_t* count, uint32_t cap, hipStream_t stream);

// Adds the update row of each record (as launch_copy_rows takes them) to its
// cache slot, element by element in
// the table's float type (kF32 or kF16; f16 sums rounded to nearest even once
// per addition), atomically so that repeated keys all land.
hipError_t launch_accumulate_rows(const uint32_t* num, uint32_t max_records, const uint64_t* slot,
                                  const uint64_t* src, uint8_t* data, uint64_t row_bytes, int dtype,
                                  hipStream_t stream);

// Linear table: row key of `table` = update row i, for every key inside
// [0, num_rows) (others are ignored).  Repeated keys: one of their rows wins.
hipError_t launch_table_update(const void* keys, int64_t n, int key_bytes, const uint8_t* values,
                               int64_t value_stride, uint8_t* table, uint64_t row_bytes,
                               uint64_t num_rows, hipStream_t stream);

// Linear table in device memory: row key += update row i (kF32 or kF16,
// atomic per element) for every key inside [0, num_rows).
hipError_t launch_table_accumulate(const void* keys, int64_t n, int key_bytes,
                                   const uint8_t* values, int64_t value_stride, uint8_t* table,
                                   uint64_t row_bytes, uint64_t num_rows, int dtype,
                                   hipStream_t stream);

}  // namespace nve_amd
