// Brute-force check of set_divisor.hpp on the host: the multiply-high
// quotient equals n / d and the shift test equals the reference's rebuilt-key
// compare (tag * d + n % d == n, in the key's width), over edge and random
// divisors, dividends and tags.  Prints "ok <cases>" or the first mismatch.
#include <stdint.h>
#include <stdio.h>

#include <random>
#include <vector>

#include "kernels/set_divisor.hpp"

using nve_amd::SetDivisor;

static int fail(const char* what, uint64_t d, uint64_t n, uint64_t got, uint64_t want) {
  printf("FAIL %s d=%llu n=%llu got=%llu want=%llu\n", what, (unsigned long long)d, (unsigned long long)n,
         (unsigned long long)got, (unsigned long long)want);
  return 1;
}

int main() {
  std::mt19937_64 rng(0x5e7d1u);
  std::vector<uint64_t> divs = {1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 12, 64, 100, 127, 128, 129, 255, 256, 1000,
                                1u << 16, (1u << 16) + 1, 65535, 14925373, 16025997, 16026016, 0x7fffffffu,
                                0x80000000u, 0x80000001u, 0xfffffffeu, 0xffffffffu, 3u << 30, 5u << 28};
  for (int i = 0; i < 200; ++i) {
    const uint64_t odd = (rng() | 1) & 0xffffffffu;
    const int v = (int)(rng() % 32);
    const uint64_t d = (odd << v) & 0xffffffffu;
    divs.push_back(d ? d : 1);
    divs.push_back((rng() % 0xffffffffu) + 1);
  }
  long cases = 0;
  for (uint64_t d : divs) {
    const SetDivisor s = nve_amd::make_set_divisor(d);
    std::vector<uint64_t> ns = {0, 1, d - 1, d, d + 1, 2 * d - 1, 2 * d, ~0ull, ~0ull - 1, 1ull << 63,
                                (1ull << 63) - 1, 0xffffffffull, 0x100000000ull, (~0ull / d) * d,
                                (~0ull / d) * d - 1, ~0ull - (~0ull % d)};
    for (int i = 0; i < 400; ++i) ns.push_back(rng());
    for (int i = 0; i < 100; ++i) ns.push_back(rng() >> (rng() % 64));
    for (uint64_t n : ns) {
      const uint64_t q = nve_amd::set_div64(s, n);
      if (q != n / d) return fail("div64", d, n, q, n / d);
      const uint64_t set = n - q * d;
      // tags: the key's own, the empty-way sentinel, neighbours, tags equal
      // to q in the low 64 - v bits only, random ones
      std::vector<uint64_t> tags = {q, ~0ull, q + 1, q - 1, 0, q ^ (1ull << 63), rng(), rng() >> 20};
      if (s.v) tags.push_back(q + (1ull << (64 - s.v))), tags.push_back(q - (1ull << (64 - s.v)));
      for (uint64_t t : tags) {
        const bool want = t * d + set == n;
        if (nve_amd::tag_matches64(s, t, q) != want) return fail("match64", d, n, t, want);
        ++cases;
      }
      const uint32_t n32 = (uint32_t)n;
      const uint32_t q32 = nve_amd::set_div32(s, n32);
      if (q32 != n32 / (uint32_t)d) return fail("div32", d, n32, q32, n32 / (uint32_t)d);
      const uint32_t set32 = n32 - q32 * (uint32_t)d;
      std::vector<uint32_t> tags32 = {q32, 0xffffffffu, q32 + 1, q32 - 1, 0, (uint32_t)rng()};
      if (s.v) tags32.push_back(q32 + (uint32_t)(1ull << (32 - s.v)));
      for (uint32_t t : tags32) {
        const bool want = (uint32_t)(t * (uint32_t)d + set32) == n32;
        if (nve_amd::tag_matches32(s, t, q32) != want) return fail("match32", d, n32, t, want);
        ++cases;
      }
    }
  }
  printf("ok %ld\n", cases);
  return 0;
}
