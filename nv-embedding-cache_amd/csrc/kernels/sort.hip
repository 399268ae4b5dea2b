// sort.hip -- stable LSD radix sort of (uint64 key, uint32 value) pairs, an
// exclusive scan and a key-span reduction: the sorting primitives behind the
// cache insert (histogram and set grouping) and dedup.
//
// The reference uses CUB (cub::DeviceRadixSort::SortPairs[Descending],
// DeviceRunLengthEncode::Encode, DeviceScan::ExclusiveSum; deduper.cuh:157-200,
// gather_keys_data_ptrs.cuh:154-183, ec_set_associative_modify.cuh:472-497).
// Only the mathematical results matter (a stable sort; descending sorts are
// expressed by the caller as ascending sorts of a complemented key).
//
// One pass per digit of 8 bits, or of 9 when that takes fewer passes (the
// last digit keeps only the bits below end_bit), three kernels per pass:
//   hist     each 256-thread workgroup counts the digits of its 1024-key tile
//            into LDS and writes the counts digit-major;
//   rowscan  one workgroup per digit turns its row of per-tile counts into
//            exclusive prefixes (a separate array) and writes the digit's total;
//   scatter  each workgroup scans the digit totals (digit d starts after
//            every smaller digit) and adds its tile's row prefix (digit d of
//            tile t lands after digit d of tiles < t: this is what makes the
//            pass stable).  It ranks its keys stably inside the tile -- a wave
//            finds the lanes sharing its digit with one ballot per digit bit, ranks by
//            popcount of the lower lanes, and adds the counts of earlier waves
//            and rounds -- stages the tile in LDS in digit order, and writes
//            it out so that consecutive threads store consecutive positions of
//            a digit's run.
//
// The exclusive scan of an array (run heads in dedup and insert) is
// reduce-then-scan over 4096-element blocks: block sums, a scan of the sums
// (recursively, in the caller's temporary storage), then each block rescans
// its elements from its offset.
#include "device_common.cuh"
#include "sort_launch.hpp"

namespace nve_amd {

constexpr int kSortThreads = 256;
constexpr int kSortItems = 4;
constexpr int kSortTile = kSortThreads * kSortItems;
constexpr int kMaxBins = 512;  // digits of at most 9 bits

// The sort key of position i: keys[i], or with a raw source the caller's key
// converted on the fly (sign bit flipped when src.flip).
template <bool RAW>
__device__ __forceinline__ uint64_t sort_key(const uint64_t* keys, const RadixSource& src, int64_t i) {
  if constexpr (RAW) {
    const int64_t k = load_key(src.keys, src.key_bytes, i);
    return src.flip ? flip_key(k, src.key_bytes) : (uint64_t)k;
  } else {
    return keys[i];
  }
}

// RAW: the first pass over the caller's keys; with src.span_part, also the
// tile's OR of key ^ key[0] (the bits where its keys differ from the first).
template <int RB, bool RAW>
__global__ __launch_bounds__(256) void radix_hist_kernel(const uint64_t* keys, RadixSource src, int64_t n,
                                                         int shift, uint32_t mask, uint32_t* counts,
                                                         int nblocks) {
  constexpr int kBins = 1 << RB;
  __shared__ uint32_t h[kBins];
  const int tid = threadIdx.x;
#pragma unroll
  for (int d = tid; d < kBins; d += kSortThreads) h[d] = 0;
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * kSortTile;
  uint64_t diff = 0;
  const uint64_t k0 = RAW && src.span_part != nullptr ? sort_key<RAW>(keys, src, 0) : 0;
#pragma unroll
  for (int r = 0; r < kSortItems; ++r) {
    const int64_t i = base + r * kSortThreads + tid;
    if (i < n) {
      const uint64_t k = sort_key<RAW>(keys, src, i);
      atomicAdd(&h[(uint32_t)(k >> shift) & mask], 1u);
      diff |= k ^ k0;
    }
  }
  if constexpr (RAW) {
    if (src.span_part != nullptr) {  // uniform
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) diff |= __shfl_xor(diff, o);
      __shared__ uint64_t red[kSortThreads / 64];
      if ((tid & 63) == 0) red[tid >> 6] = diff;
      __syncthreads();
      if (tid == 0) {
        uint64_t x = 0;
#pragma unroll
        for (int w = 0; w < kSortThreads / 64; ++w) x |= red[w];
        src.span_part[blockIdx.x] = x;
      }
    }
  }
  __syncthreads();
#pragma unroll
  for (int d = tid; d < kBins; d += kSortThreads) counts[(int64_t)d * nblocks + blockIdx.x] = h[d];
}

// Inclusive scan across the 64 lanes of a wave.
__device__ __forceinline__ uint32_t wave_inclusive_scan(uint32_t v) {
  const int lane = lane_id();
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t t = shfl32(v, lane >= o ? lane - o : lane);
    if (lane >= o) v += t;
  }
  return v;
}

// Exclusive scan of one value per thread over a workgroup of NT threads
// (NT a multiple of 64, at most 4096); `total` receives the sum.  `lds` holds
// NT / 64 + 1 words; every thread of the workgroup must call it.
template <int NT>
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* lds,
                                                         uint32_t* total) {
  constexpr int kWaves = NT / 64;
  const int lane = lane_id();
  const int wave = (int)threadIdx.x >> 6;
  const uint32_t inc = wave_inclusive_scan(v);
  if (lane == 63) lds[wave] = inc;
  __syncthreads();
  if (threadIdx.x < 64) {
    const uint32_t w = (int)threadIdx.x < kWaves ? lds[threadIdx.x] : 0u;
    const uint32_t wi = wave_inclusive_scan(w);
    if ((int)threadIdx.x < kWaves) lds[threadIdx.x] = wi - w;
    if ((int)threadIdx.x == kWaves - 1) lds[kWaves] = wi;
  }
  __syncthreads();
  const uint32_t res = inc - v + lds[wave];
  *total = lds[kWaves];
  __syncthreads();
  return res;
}

constexpr int kScanThreads = 256;
constexpr int kScanItems = 16;
constexpr int kScanBlock = kScanThreads * kScanItems;

// Sum of each 4096-element block.
__global__ __launch_bounds__(256) void scan_reduce_kernel(const uint32_t* data, int64_t m,
                                                          uint32_t* sums) {
  __shared__ uint32_t lds[kScanThreads / 64 + 1];
  const int64_t base = (int64_t)blockIdx.x * kScanBlock + (int64_t)threadIdx.x * kScanItems;
  uint32_t s = 0;
#pragma unroll
  for (int j = 0; j < kScanItems; ++j)
    if (base + j < m) s += data[base + j];
  uint32_t total;
  (void)block_exclusive_scan<kScanThreads>(s, lds, &total);
  if (threadIdx.x == 0) sums[blockIdx.x] = total;
}

// Exclusive scan of each block from its offset (sums[block], or 0 with a
// single block); the last block writes the grand total.
__global__ __launch_bounds__(256) void scan_down_kernel(uint32_t* data, int64_t m,
                                                        const uint32_t* offsets, uint32_t* total) {
  __shared__ uint32_t lds[kScanThreads / 64 + 1];
  const int64_t base = (int64_t)blockIdx.x * kScanBlock + (int64_t)threadIdx.x * kScanItems;
  uint32_t v[kScanItems];
  uint32_t s = 0;
#pragma unroll
  for (int j = 0; j < kScanItems; ++j) {
    v[j] = base + j < m ? data[base + j] : 0u;
    s += v[j];
  }
  uint32_t block_total;
  uint32_t run = block_exclusive_scan<kScanThreads>(s, lds, &block_total);
  const uint32_t off = offsets ? offsets[blockIdx.x] : 0u;
  run += off;
#pragma unroll
  for (int j = 0; j < kScanItems; ++j) {
    if (base + j < m) data[base + j] = run;
    run += v[j];
  }
  if (total != nullptr && blockIdx.x == gridDim.x - 1 && threadIdx.x == 0)
    *total = off + block_total;
}

// Exclusive scan of the D consecutive values v[0..D) of each of the
// workgroup's NT threads (thread t holds items t*D .. t*D+D-1), in place.
template <int NT, int D>
__device__ __forceinline__ void block_exclusive_scan_items(uint32_t* v, uint32_t* lds,
                                                           uint32_t* total) {
  uint32_t s = 0;
#pragma unroll
  for (int j = 0; j < D; ++j) s += v[j];
  uint32_t run = block_exclusive_scan<NT>(s, lds, total);
#pragma unroll
  for (int j = 0; j < D; ++j) {
    const uint32_t x = v[j];
    v[j] = run;
    run += x;
  }
}

// Row d of the digit-major per-tile counts -> exclusive prefixes in offs;
// totals[d] = the row's sum.  One workgroup per digit.
__global__ __launch_bounds__(256) void radix_rowscan_kernel(const uint32_t* counts, uint32_t* offs,
                                                            int nblocks, uint32_t* totals) {
  __shared__ uint32_t lds[256 / 64 + 1];
  const uint32_t* row = counts + (int64_t)blockIdx.x * nblocks;
  uint32_t* orow = offs + (int64_t)blockIdx.x * nblocks;
  uint32_t carry = 0;
  for (int c = 0; c < nblocks; c += 256 * 4) {
    const int b = c + (int)threadIdx.x * 4;
    uint32_t v[4];
    uint32_t s = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[j] = b + j < nblocks ? row[b + j] : 0u;
      s += v[j];
    }
    uint32_t chunk_total;
    uint32_t run = carry + block_exclusive_scan<256>(s, lds, &chunk_total);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (b + j < nblocks) orow[b + j] = run;
      run += v[j];
    }
    carry += chunk_total;
  }
  if (threadIdx.x == 0) totals[blockIdx.x] = carry;
}

// RAW: the first pass reads the caller's keys (src) and takes each key's
// position as its value.
template <int RB, bool RAW>
__global__ __launch_bounds__(256) void radix_scatter_kernel(const uint64_t* keys, const uint32_t* vals,
                                                            RadixSource src, uint64_t* ko, uint32_t* vo,
                                                            int64_t n, int shift, uint32_t mask,
                                                            const uint32_t* counts,
                                                            const uint32_t* offs,
                                                            const uint32_t* totals, int nblocks) {
  constexpr int kBins = 1 << RB;
  constexpr int D = kBins / kSortThreads;                    // digits per thread
  constexpr int kSlots = kSortItems * (kSortThreads / 64);  // (round, wave) pairs in key order
  __shared__ uint64_t sk[kSortTile];
  __shared__ uint32_t sv[kSortTile];
  __shared__ uint32_t lstart[kBins];          // first local position of digit d in the tile
  __shared__ uint32_t gbase[kBins];           // output position of that key
  __shared__ uint32_t slot[kSlots][kBins];    // keys of digit d per (round, wave), then their prefix
  __shared__ uint32_t lds[256 / 64 + 1];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t base = (int64_t)blockIdx.x * kSortTile;
  const int tile_n = (int)(n - base < kSortTile ? n - base : kSortTile);
  // all of the tile's loads in flight at once
  uint64_t k[kSortItems];
  uint32_t v[kSortItems];
#pragma unroll
  for (int r = 0; r < kSortItems; ++r) {
    const int li = r * kSortThreads + tid;
    k[r] = li < tile_n ? sort_key<RAW>(keys, src, base + li) : 0ull;
    if constexpr (RAW)
      v[r] = (uint32_t)(base + li);
    else
      v[r] = li < tile_n ? vals[base + li] : 0u;
  }
  // thread t owns digits t*D .. t*D+D-1
  uint32_t dbase[D], loc[D];
#pragma unroll
  for (int j = 0; j < D; ++j) {
    const int d = tid * D + j;
    dbase[j] = totals[d];
    loc[j] = counts[(int64_t)d * nblocks + blockIdx.x];
  }
  uint32_t all;
  block_exclusive_scan_items<kSortThreads, D>(dbase, lds, &all);
  block_exclusive_scan_items<kSortThreads, D>(loc, lds, &all);
#pragma unroll
  for (int j = 0; j < D; ++j) {
    const int d = tid * D + j;
    lstart[d] = loc[j];
    gbase[d] = dbase[j] + offs[(int64_t)d * nblocks + blockIdx.x];
#pragma unroll
    for (int q = 0; q < kSlots; ++q) slot[q][d] = 0;
  }
  __syncthreads();
  // per (round, wave): lanes sharing the digit, rank among them, count by the leader
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  uint32_t rank[kSortItems];
#pragma unroll
  for (int r = 0; r < kSortItems; ++r) {
    const bool valid = r * kSortThreads + tid < tile_n;
    const uint32_t d = (uint32_t)(k[r] >> shift) & mask;
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < RB; ++b) {
      const uint64_t m = __ballot((d >> b) & 1u);
      peers &= ((d >> b) & 1u) ? m : ~m;
    }
    rank[r] = (uint32_t)__popcll(peers & lt_mask);
    if (valid && rank[r] == 0) slot[r * (kSortThreads / 64) + wave][d] = (uint32_t)__popcll(peers);
  }
  __syncthreads();
  // digit d: exclusive prefix over the slots, from its local start
#pragma unroll
  for (int j = 0; j < D; ++j) {
    const int d = tid * D + j;
    uint32_t acc = lstart[d];
#pragma unroll
    for (int q = 0; q < kSlots; ++q) {
      const uint32_t c = slot[q][d];
      slot[q][d] = acc;
      acc += c;
    }
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < kSortItems; ++r) {
    if (r * kSortThreads + tid < tile_n) {
      const uint32_t d = (uint32_t)(k[r] >> shift) & mask;
      const uint32_t pos = slot[r * (kSortThreads / 64) + wave][d] + rank[r];
      sk[pos] = k[r];
      sv[pos] = v[r];
    }
  }
  __syncthreads();
  // the tile in digit order: runs of one digit go to consecutive positions
  for (int j = tid; j < tile_n; j += kSortThreads) {
    const uint64_t kk = sk[j];
    const uint32_t d = (uint32_t)(kk >> shift) & mask;
    const uint32_t pos = gbase[d] + (uint32_t)j - lstart[d];
    ko[pos] = kk;
    vo[pos] = sv[j];
  }
}

// OR over i of keys[i] ^ keys[0]: the bits where keys differ.  One atomic per
// workgroup at most, and none when the workgroup adds no new bit: thousands
// of atomics on one address serialize in one L2 channel.
__global__ __launch_bounds__(256) void key_span_kernel(const uint64_t* keys, int64_t n,
                                                       unsigned long long* out) {
  __shared__ uint64_t red[4];
  const uint64_t k0 = keys[0];
  uint64_t acc = 0;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    acc |= keys[i] ^ k0;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) acc |= __shfl_xor(acc, o);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint64_t a = red[0] | red[1] | red[2] | red[3];
    const uint64_t seen = __hip_atomic_load(out, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (a & ~seen) atomicOr(out, (unsigned long long)a);
  }
}

// ---------------------------------------------------------------------------
size_t scan_temp_bytes(int64_t m) {
  // block sums of every level of the recursion, each level 256-byte aligned
  size_t bytes = 0;
  for (int64_t nb = (m + kScanBlock - 1) / kScanBlock; nb > 1; nb = (nb + kScanBlock - 1) / kScanBlock)
    bytes += ((size_t)nb * sizeof(uint32_t) + 255) / 256 * 256;
  return bytes;
}

size_t radix_sort_temp_bytes(int64_t n) {
  const int64_t nblocks = (n + kSortTile - 1) / kSortTile;
  const size_t sort = (size_t)(nblocks > 0 ? nblocks : 1) * kMaxBins * sizeof(uint32_t) * 2 +
                      kMaxBins * sizeof(uint32_t) + 1024;
  const size_t scan = scan_temp_bytes(n);
  return sort > scan ? sort : scan;
}

hipError_t radix_sort_pairs(uint64_t* keys, uint32_t* vals, uint64_t* keys_alt, uint32_t* vals_alt,
                            int64_t n, int begin_bit, int end_bit, void* temp, int* result_in_alt,
                            hipStream_t stream, const RadixSource* src) {
  *result_in_alt = 0;
  if (n <= 1 || end_bit <= begin_bit) return src != nullptr ? hipErrorInvalidValue : hipSuccess;
  const int64_t nblocks = (n + kSortTile - 1) / kSortTile;
  if (nblocks > 0x7fffffff) return hipErrorInvalidValue;
  uint32_t* counts = static_cast<uint32_t*>(temp);
  uint32_t* offs = counts + nblocks * kMaxBins;
  uint32_t* totals = offs + nblocks * kMaxBins;
  uint64_t* ki = keys;
  uint32_t* vi = vals;
  uint64_t* ka = keys_alt;
  uint32_t* va = vals_alt;
  const RadixSource none{};
  // 9-bit digits when they take fewer passes than 8-bit ones (26-bit keys: 3
  // passes instead of 4); the last digit keeps only the bits below end_bit.
  // (10-bit digits measured no better: three 10-bit passes over 262,144 keys
  // took as long as four 8-bit ones, 17.4 against 13.1 us a pass.)
  const int width = end_bit - begin_bit;
  const int rb = (width + 8) / 9 < (width + 7) / 8 ? 9 : 8;
  for (int shift = begin_bit; shift < end_bit; shift += rb) {
    const int bits = end_bit - shift < rb ? end_bit - shift : rb;
    const uint32_t mask = (1u << bits) - 1u;
    const bool raw = src != nullptr && shift == begin_bit;
    const RadixSource& s = raw ? *src : none;
#define NVE_RADIX_PASS(RB, RAW)                                                                           \
  hipLaunchKernelGGL((radix_hist_kernel<RB, RAW>), dim3(nblocks), dim3(kSortThreads), 0, stream, ki, s, n, \
                     shift, mask, counts, (int)nblocks);                                                  \
  hipLaunchKernelGGL(radix_rowscan_kernel, dim3(1u << RB), dim3(256), 0, stream, counts, offs,            \
                     (int)nblocks, totals);                                                               \
  hipLaunchKernelGGL((radix_scatter_kernel<RB, RAW>), dim3(nblocks), dim3(kSortThreads), 0, stream, ki,   \
                     vi, s, ka, va, n, shift, mask, counts, offs, totals, (int)nblocks)
    if (rb == 9) {
      if (raw) {
        NVE_RADIX_PASS(9, true);
      } else {
        NVE_RADIX_PASS(9, false);
      }
    } else {
      if (raw) {
        NVE_RADIX_PASS(8, true);
      } else {
        NVE_RADIX_PASS(8, false);
      }
    }
#undef NVE_RADIX_PASS
    std::swap(ki, ka);
    std::swap(vi, va);
    *result_in_alt ^= 1;
  }
  return hipGetLastError();
}

int64_t radix_tiles(int64_t n) { return n > 0 ? (n + kSortTile - 1) / kSortTile : 0; }

hipError_t exclusive_scan_u32(uint32_t* data, int64_t m, uint32_t* total, void* temp,
                              hipStream_t stream) {
  if (m <= 0) return hipSuccess;
  const int64_t nb = (m + kScanBlock - 1) / kScanBlock;
  if (nb > 0x7fffffff) return hipErrorInvalidValue;
  if (nb == 1) {
    hipLaunchKernelGGL(scan_down_kernel, dim3(1), dim3(kScanThreads), 0, stream, data, m,
                       (const uint32_t*)nullptr, total);
    return hipGetLastError();
  }
  uint32_t* sums = static_cast<uint32_t*>(temp);
  void* rest = static_cast<uint8_t*>(temp) + ((size_t)nb * sizeof(uint32_t) + 255) / 256 * 256;
  hipLaunchKernelGGL(scan_reduce_kernel, dim3(nb), dim3(kScanThreads), 0, stream, data, m, sums);
  hipError_t e = exclusive_scan_u32(sums, nb, nullptr, rest, stream);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(scan_down_kernel, dim3(nb), dim3(kScanThreads), 0, stream, data, m, sums,
                     total);
  return hipGetLastError();
}

hipError_t key_span(const uint64_t* keys, int64_t n, unsigned long long* out, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  int64_t grid = (n + 1023) / 1024;  // four keys per thread
  if (grid > 512) grid = 512;
  hipLaunchKernelGGL(key_span_kernel, dim3(grid), dim3(256), 0, stream, keys, n, out);
  return hipGetLastError();
}

}  // namespace nve_amd
