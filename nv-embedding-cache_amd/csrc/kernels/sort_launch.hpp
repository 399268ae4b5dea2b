// sort_launch.hpp -- stable radix sort, exclusive scan and key-span helpers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

namespace nve_amd {

// Bytes of temporary storage radix_sort_pairs needs for n pairs; it also
// covers exclusive_scan_u32 of up to n elements.
size_t radix_sort_temp_bytes(int64_t n);
// Bytes of temporary storage exclusive_scan_u32 needs for m elements.
size_t scan_temp_bytes(int64_t m);

// The caller's keys as the first pass's input: keys of key_bytes bytes at
// `keys` (sign bit flipped when flip != 0), values = positions; span_part
// (optional, radix_tiles(n) words) receives each tile's OR of key ^ key[0].
struct RadixSource {
  const void* keys;
  int key_bytes;
  int flip;
  uint64_t* span_part;
};
// Tiles (workgroups) of one radix pass over n keys.
int64_t radix_tiles(int64_t n);

// Stable ascending sort of (keys[i], vals[i]) on bits [begin_bit, end_bit) of
// the keys (digits of 8 or 9 bits from begin_bit).  Ping-pongs between (keys, vals) and
// (keys_alt, vals_alt); *result_in_alt says which pair holds the result.
// With src, the first pass reads src instead of keys / vals (which it never
// reads); at least one pass must then run (n >= 2, end_bit > begin_bit), else
// hipErrorInvalidValue.
hipError_t radix_sort_pairs(uint64_t* keys, uint32_t* vals, uint64_t* keys_alt, uint32_t* vals_alt,
                            int64_t n, int begin_bit, int end_bit, void* temp, int* result_in_alt,
                            hipStream_t stream, const RadixSource* src = nullptr);

// In-place exclusive scan of m uint32 (total, if non-null, gets the sum);
// temp holds scan_temp_bytes(m) bytes.
hipError_t exclusive_scan_u32(uint32_t* data, int64_t m, uint32_t* total, void* temp,
                              hipStream_t stream);

// *out |= OR over i of (keys[i] ^ keys[0]); *out must start at 0.
hipError_t key_span(const uint64_t* keys, int64_t n, unsigned long long* out, hipStream_t stream);

}  // namespace nve_amd
