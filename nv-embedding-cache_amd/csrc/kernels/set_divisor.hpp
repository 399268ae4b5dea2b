// set_divisor.hpp -- the cache's set / tag arithmetic without a division.
//
// The set-associative cache places key k in set (unsigned)k % num_sets with
// tag (unsigned)k / num_sets, and a way holds k when its rebuilt key
// tag * num_sets + set equals k in the key's width (ec_hash.h:36-60,
// ec_set_associative.cuh:46-80).  On the GPU a 64-bit division by a runtime
// value is a long software sequence, run once per key of every lookup, so the
// host prepares, once per table, the constants of division by the invariant
// num_sets (Granlund & Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994, section 4, unsigned N-bit division):
//     l = ceil(log2 d),  m = floor(2^N (2^l - d) / d) + 1,
//     q = (t + ((n - t) >> min(l, 1))) >> max(l - 1, 0),  t = mulhi_N(m, n)
// which is exact for every N-bit n and 1 <= d < 2^N.
//
// The way test needs no multiplication either: with d = odd * 2^v, the
// rebuilt key tag * d + set equals k = q * d + set exactly when
// (tag - q) * d == 0 modulo 2^N, i.e. when ((tag - q) << v) == 0 (the odd
// factor is invertible).  For v > 0 this accepts tags that differ from q in
// their top v bits, as the reference's rebuilt-key compare does (an empty
// way's sentinel tag can rebuild to a real key when d divides 2^N).
//
// Host code (g++) and device code (hipcc) share this header.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nve_amd {

struct SetDivisor {
  uint64_t m64;  // multiplier, 64-bit keys
  uint32_t m32;  // multiplier, 32-bit keys
  uint32_t d;    // num_sets, 1 <= d < 2^32
  uint32_t sh1;  // min(l, 1)
  uint32_t sh2;  // max(l - 1, 0)
  uint32_t v;    // trailing zero bits of d
  uint32_t pad_;
};

// Constants of division by d (1 <= d <= 2^32 - 1); host only.
inline SetDivisor make_set_divisor(uint64_t d) {
  SetDivisor s{};
  uint32_t l = 0;
  while (l < 64 && (uint64_t(1) << l) < d) ++l;
  const unsigned __int128 span = (unsigned __int128)((uint64_t(1) << l) - d);
  s.m64 = (uint64_t)((span << 64) / d) + 1;
  s.m32 = (uint32_t)(((uint64_t)span << 32) / d) + 1;
  s.d = (uint32_t)d;
  s.sh1 = l < 1 ? l : 1;
  s.sh2 = l > 1 ? l - 1 : 0;
  uint32_t v = 0;
  while (v < 32 && ((d >> v) & 1u) == 0) ++v;
  s.v = v;
  return s;
}

__host__ __device__ inline uint64_t mulhi64(uint64_t a, uint64_t b) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __umul64hi(a, b);
#else
  return (uint64_t)(((unsigned __int128)a * b) >> 64);
#endif
}

__host__ __device__ inline uint32_t mulhi32(uint32_t a, uint32_t b) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __umulhi(a, b);
#else
  return (uint32_t)(((uint64_t)a * b) >> 32);
#endif
}

// n / d and n % d for 64-bit n.
__host__ __device__ inline uint64_t set_div64(const SetDivisor& s, uint64_t n) {
  const uint64_t t = mulhi64(s.m64, n);
  return (t + ((n - t) >> s.sh1)) >> s.sh2;
}

// n / d for 32-bit n.
__host__ __device__ inline uint32_t set_div32(const SetDivisor& s, uint32_t n) {
  const uint32_t t = mulhi32(s.m32, n);
  return (t + ((n - t) >> s.sh1)) >> s.sh2;
}

// Does a way with tag `tag` hold the key whose quotient is q (the rebuilt key
// compare of the reference, in 64 or 32 bits)?
__host__ __device__ inline bool tag_matches64(const SetDivisor& s, uint64_t tag, uint64_t q) {
  return ((tag - q) << s.v) == 0;
}
__host__ __device__ inline bool tag_matches32(const SetDivisor& s, uint32_t tag, uint32_t q) {
  return (uint32_t)((tag - q) << s.v) == 0;
}

}  // namespace nve_amd
