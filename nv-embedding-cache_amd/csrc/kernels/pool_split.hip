// pool_split.hip -- find-and-pool over linear tables without the general
// pool_kernel's generality (cache, backing table, passes, 64-bit address
// shuffles, a 1 KB argument block):
//  * pool_split_kernel: long bags (the GPULayer benchmark: a few hundred bags
//    of ~1K keys), one workgroup per bag;
//  * pool_short_kernel: short bags (DLRM-style jagged batches, one or many
//    tables), one lane group per bag.
//
// Reference behaviour restated: find_and_combine (cuda_ops/find_and_combine_kernel.cuh:40-154)
// over a linear table (GPULayer, gpu_embedding_layer.cu:153-189).
//
// Same decomposition and summation order as pool_kernel's split-bag path, so
// the two produce the same bits: one workgroup per bag, the bag cut into gpb
// contiguous key chunks, one chunk per G-lane group, each group accumulating
// its chunk in key order; an xor butterfly inside each wave; the waves'
// partial rows added in wave order through LDS.  What is leaner:
//  * row indices travel between lanes as 32 bits and by VALU lane moves, not
//    LDS permutes: DPP row_newbcast inside a 16-lane row, v_permlane16_swap /
//    v_permlane32_swap across rows (gfx950), v_readlane for a whole-wave
//    group; the address is formed by the consuming lane;
//  * the butterfly uses the same lane moves: a + (a of lane l ^ m), formed as
//    the sum of the two swapped halves, which is the same float addition;
//  * no cache / backing-table / multi-table / hit-mask branches, one pass per
//    row (G * 16 bytes cover the row), G and the weighting fixed at compile
//    time;
//  * the cross-wave sum is unrolled so its LDS reads are all in flight.
#include <type_traits>

#include "device_common.cuh"
#include "lane_moves.cuh"
#include "pool_launch.hpp"

namespace nve_amd {

namespace {

constexpr uint32_t kNoRow = 0xffffffffu;

// a + (a of lane l ^ M), the same float addition as a + __shfl_xor(a, M)
// (addition commutes exactly, so both partners get the same bits).
template <int M>
__device__ __forceinline__ float xor_add(float a) {
  if constexpr (M == 32) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(a), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  } else if constexpr (M == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(a), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  } else {
    static_assert(M == 8, "lane groups of 8 to 64 lanes");
    return a + __uint_as_float(dpp_mov<kDppRowRor8>(__float_as_uint(a)));
  }
}

// ri[u] / wu[u] = lane J0 + u of the group, u < U (J0 + U <= G)
template <int G, int U, bool W, int J0, int u = 0>
__device__ __forceinline__ void group_bcast_batch(uint32_t ridx, float w, int lane, uint32_t* ri,
                                                  float* wu) {
  if constexpr (u < U) {
    static_assert(J0 + u < G, "broadcast source outside the group");
    ri[u] = group_bcast<G, J0 + u>(ridx, lane);
    wu[u] = W ? __uint_as_float(group_bcast<G, J0 + u>(__float_as_uint(w), lane)) : 1.0f;
    group_bcast_batch<G, U, W, J0, u + 1>(ridx, w, lane, ri, wu);
  }
}

template <int G, int M = G>
__device__ __forceinline__ void butterfly(float* acc, int e, float& wsum, bool weighted) {
  if constexpr (M < 64) {
    for (int c = 0; c < e; ++c) acc[c] = xor_add<M>(acc[c]);
    if (weighted) wsum = xor_add<M>(wsum);
    butterfly<G, 2 * M>(acc, e, wsum, weighted);
  }
}

// acc += row, or acc = fma(row, wt, acc) when weighted, for one 16-byte slice
// of a stored f16 / f32 row.  f16 slices accumulate with one v_fma_mix_f32 per
// element (same bits as widening then adding).  A lane with nothing to add
// has loaded the zero row: adding +0 leaves acc unchanged (acc starts at +0
// and a round-to-nearest sum is -0 only when both terms are), so the
// unweighted sum needs no select; weighted callers pass wt = 0 for such a
// lane (0 * 0 + acc), which also keeps a non-finite weight of a key outside
// the table out of the sum.
template <int SDT, int E, bool W>
__device__ __forceinline__ void add_slice(float (&acc)[E], const Vec<16>& v, float wt) {
  if constexpr (SDT == kF16) {
#pragma unroll
    for (int c = 0; c < E / 2; ++c) {
      if constexpr (W) {
        acc[2 * c] = fma_half_lo(v.w[c], wt, acc[2 * c]);
        acc[2 * c + 1] = fma_half_hi(v.w[c], wt, acc[2 * c + 1]);
      } else {
        acc[2 * c] = acc_half_lo(acc[2 * c], v.w[c]);
        acc[2 * c + 1] = acc_half_hi(acc[2 * c + 1], v.w[c]);
      }
    }
  } else {
    static_assert(SDT == kF32, "f16 or f32 rows");
#pragma unroll
    for (int c = 0; c < E; ++c) {
      const float x = __uint_as_float(v.w[c]);
      acc[c] = W ? __builtin_fmaf(x, wt, acc[c]) : acc[c] + x;
    }
  }
}

// The kernel's arguments: only what this shape reads (PoolLaunch carries a
// table array for multi-table launches; a smaller kernarg segment is quicker
// to set up per launch).
struct SplitArgs {
  const void* keys;
  const void* offsets;  // null: fixed hotness
  const void* weights;
  const uint8_t* table;
  void* out;
  int64_t num_keys;
  int64_t hotness;
  uint64_t row_bytes;
  uint64_t num_rows;
  int64_t count;
  int64_t out_stride;
  int key_bytes;
  int weight_dtype;
  int mean;
  int out_dtype;
  int gpb_shift;
};

// Long bags over a set-associative cache (with or without a backing table):
// the split kernel's arguments plus the cache.
struct SplitCacheArgs : SplitArgs {
  const uint8_t* cache_data;
  const void* cache_tags;
  uint64_t num_sets;
  unsigned long long* miss_counter;  // optional, kMissStripes * kMissStripeWords words
};

constexpr uint32_t kBackingRow = 0x80000000u;  // code bit: a backing-table row, not a cache slot

// The 32-bit code of a key's row in a cache-backed table: the cache slot
// set * 8 + way on a hit (the lowest way whose rebuilt key tag * num_sets + set
// equals the key, as resolve_row), else kBackingRow | key when the backing
// table holds the key, else kNoRow.  *miss reports a cache miss.
template <typename A>
__device__ __forceinline__ uint32_t cache_code(const A& a, int64_t key, bool* miss) {
  uint32_t set, mask = 0;
  if (a.key_bytes == 4) {
    const uint32_t uk = (uint32_t)(int32_t)key;
    const uint32_t ns = (uint32_t)a.num_sets;
    set = uk % ns;
    const uint4* tp = reinterpret_cast<const uint4*>(reinterpret_cast<const int32_t*>(a.cache_tags) +
                                                     (uint64_t)set * 8);
    const uint4 t0 = tp[0];
    const uint4 t1 = tp[1];
    const uint32_t t[8] = {t0.x, t0.y, t0.z, t0.w, t1.x, t1.y, t1.z, t1.w};
#pragma unroll
    for (int w = 0; w < 8; ++w) mask |= (uint32_t)(t[w] * ns + set == uk) << w;
  } else {
    const uint64_t uk = (uint64_t)key;
    set = (uint32_t)(uk % a.num_sets);
    const uint4* tp = reinterpret_cast<const uint4*>(reinterpret_cast<const int64_t*>(a.cache_tags) +
                                                     (uint64_t)set * 8);
    uint64_t t[8];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint4 q = tp[c];
      t[2 * c] = (uint64_t)q.x | ((uint64_t)q.y << 32);
      t[2 * c + 1] = (uint64_t)q.z | ((uint64_t)q.w << 32);
    }
#pragma unroll
    for (int w = 0; w < 8; ++w) mask |= (uint32_t)(t[w] * a.num_sets + set == uk) << w;
  }
  *miss = mask == 0;
  if (mask) return set * 8u + (uint32_t)__builtin_ctz(mask);
  if (a.table != nullptr && (uint64_t)key < a.num_rows) return kBackingRow | (uint32_t)key;
  return kNoRow;
}

// Adds the workgroup's per-lane miss counts to its word of the striped miss
// counter with one atomic (every thread of the workgroup calls it).
__device__ __forceinline__ void add_group_misses(unsigned long long* counter, uint32_t misses) {
  __shared__ uint32_t wave_misses[16];
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) misses += __shfl_xor(misses, o);
  if ((threadIdx.x & 63) == 0) wave_misses[threadIdx.x >> 6] = misses;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t m = 0;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) m += wave_misses[w];
    if (m) atomicAdd(counter + (blockIdx.x & (kMissStripes - 1)) * kMissStripeWords, (unsigned long long)m);
  }
}

template <int SDT, int G, bool W, bool CACHE = false>
__global__ __launch_bounds__(1024) void pool_split_kernel(
    std::conditional_t<CACHE, SplitCacheArgs, SplitArgs> a) {
  constexpr int VB = 16;
  constexpr int ES = Fmt<SDT>::esize;
  constexpr int E = VB / ES;
  constexpr int U = G < 16 ? G : 16;  // row loads in flight per lane; a group's keys in G / U batches
  extern __shared__ float lds[];

  const int tid = threadIdx.x;
  const int gl = tid & (G - 1);
  const int chunk = tid / G;
  const int gpb_shift = a.gpb_shift;
  const int gpb = 1 << gpb_shift;
  const int64_t bag = blockIdx.x;

  int64_t s, e;
  if (a.offsets != nullptr) {
    s = load_key(a.offsets, a.key_bytes, bag);
    e = load_key(a.offsets, a.key_bytes, bag + 1);
    s = s < 0 ? 0 : (s > a.num_keys ? a.num_keys : s);
    e = e < s ? s : (e > a.num_keys ? a.num_keys : e);
  } else {
    s = bag * a.hotness;
    e = s + a.hotness;
  }
  int64_t cs = s, ce = e;
  if (e > s) {
    const int64_t per = (e - s + gpb - 1) >> gpb_shift;
    cs = s + chunk * per;
    if (cs > e) cs = e;
    ce = cs + per < e ? cs + per : e;
  }

  const uint64_t table = (uint64_t)a.table;
  const uint64_t row_bytes = a.row_bytes;
  const uint64_t num_rows = a.num_rows;
  const uint64_t zero_row = (uint64_t)g_zero_row;
  const uint32_t rb32 = (uint32_t)row_bytes;  // launcher: row_bytes < 2^32, off < the zero row's size
  const int64_t value_bytes = a.count * ES;
  const int off = gl * VB;
  const bool in_row = off < value_bytes;

  float acc[E];
#pragma unroll
  for (int c = 0; c < E; ++c) acc[c] = 0.0f;
  float wsum = 0.0f;

  const int lane = tid & 63;
  uint32_t misses = 0;
  for (int64_t k0 = cs; k0 < ce; k0 += G) {
    const int64_t kk = k0 + gl;
    uint32_t ridx = kNoRow;
    float w = 0.0f;
    if (kk < ce) {
      const int64_t key = load_key(a.keys, a.key_bytes, kk);
      if constexpr (CACHE) {
        bool miss;
        ridx = cache_code(a, key, &miss);
        misses += miss ? 1u : 0u;
      } else {
        if ((uint64_t)key < num_rows) ridx = (uint32_t)key;  // keys outside the table read nothing
      }
      if (W) w = load_weight(a.weights, a.weight_dtype, kk);
    }
    const int n = (int)((ce - k0) < G ? (ce - k0) : G);
    // batch starting at key j0 of the group (compile time, so every lane move
    // has an immediate source lane); lanes past the group's keys hold kNoRow:
    // they load the zero row and are not added
    auto batch = [&](auto jc) {
      constexpr int j0 = decltype(jc)::value;
      if (j0 >= n) return;
      uint32_t ri[U];
      float wu[U];
      group_bcast_batch<G, U, W, j0>(ridx, w, lane, ri, wu);
      Vec<VB> v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        // base and row index picked by selects (no divergent branch), then one
        // 32 x 32 -> 64-bit multiply-add: row_bytes < 2^32
        // one 32 x 32 -> 64-bit multiply-add per address (row_bytes < 2^32);
        // select-based addressing (base and index picked per lane) measured
        // slower than this form on both bag shapes
        const bool real = ri[u] != kNoRow && in_row;
        uint64_t base;
        if constexpr (CACHE) {
          base = (ri[u] & kBackingRow) ? table + (uint64_t)(ri[u] & ~kBackingRow) * rb32
                                       : (uint64_t)a.cache_data + (uint64_t)ri[u] * rb32;
        } else {
          base = table + (uint64_t)ri[u] * rb32;
        }
        v[u] = load_vec<VB>(real ? base + (uint64_t)off : zero_row + (uint64_t)off);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool use = j0 + u < n;  // uniform over the group
        if (W && use) wsum += wu[u];
        add_slice<SDT, E, W>(acc, v[u], (use && in_row && ri[u] != kNoRow) ? wu[u] : 0.0f);
      }
    };
    for_batches<U, 0, G / U>(batch);
  }

  // butterfly over the wave's groups (the same pairing and additions as pool_kernel)
  butterfly<G>(acc, E, wsum, W);
  if constexpr (CACHE) {
    // one miss-counter atomic per workgroup: thousands on one address serialize
    if (a.miss_counter != nullptr) add_group_misses(a.miss_counter, misses);
  }

  // waves' partial rows, added in wave order
  constexpr int row_elems = G * E;
  const int wave = tid >> 6;
  const int waves = (gpb * G) >> 6;
  float* red = lds;
  float* wred = lds + (blockDim.x >> 6) * row_elems;
  if ((tid & 63) < G) {
#pragma unroll
    for (int c = 0; c < E; ++c) red[wave * row_elems + gl * E + c] = acc[c];
    if (gl == 0) wred[wave] = wsum;
  }
  __syncthreads();
  if (tid < row_elems && ((tid / E) * VB) < value_bytes) {
    float part[16];
    float wp[16];
#pragma unroll
    for (int w = 0; w < 16; ++w) {
      part[w] = w < waves ? red[w * row_elems + tid] : 0.0f;
      wp[w] = (W && w < waves) ? wred[w] : 0.0f;
    }
    float v = part[0];
    float ws = wp[0];
#pragma unroll
    for (int w = 1; w < 16; ++w) {
      if (w < waves) {
        v += part[w];
        ws += wp[w];
      }
    }
    if (a.mean) {
      const float d = W ? ws : (float)(e - s);
      v = (d == 0.0f) ? 0.0f : v / d;
    }
    uint8_t* o = reinterpret_cast<uint8_t*>(a.out) + bag * a.out_stride;
    if (a.out_dtype == kF16)
      *reinterpret_cast<gptr_w<uint16_t>>((uint64_t)o + (uint64_t)tid * 2) = f2h(v);
    else
      *reinterpret_cast<gptr_w<float>>((uint64_t)o + (uint64_t)tid * 4) = v;
  }
}

template <int SDT, int G>
hipError_t launch_split_g(const PoolLaunch& a, const PoolGeometry& g, hipStream_t stream) {
  SplitArgs s{};
  s.keys = a.keys;
  s.offsets = a.offsets;
  s.weights = a.weights;
  s.table = a.src.table;
  s.out = a.out;
  s.num_keys = a.num_keys;
  s.hotness = a.hotness;
  s.row_bytes = a.src.row_bytes;
  s.num_rows = a.src.num_rows;
  s.count = a.count;
  s.out_stride = a.out_stride;
  s.key_bytes = a.key_bytes;
  s.weight_dtype = a.weight_dtype;
  s.mean = a.mean;
  s.out_dtype = a.out_dtype;
  s.gpb_shift = 0;
  while ((1 << s.gpb_shift) < g.gpb) ++s.gpb_shift;
  const dim3 grid((unsigned)g.grid), block((unsigned)g.threads);
  if (a.src.cache_data != nullptr) {
    SplitCacheArgs c{};
    static_cast<SplitArgs&>(c) = s;
    c.cache_data = a.src.cache_data;
    c.cache_tags = a.src.cache_tags;
    c.num_sets = a.src.num_sets;
    c.miss_counter = a.miss_counter;
    if (a.weighted)
      hipLaunchKernelGGL((pool_split_kernel<SDT, G, true, true>), grid, block, g.lds_bytes, stream, c);
    else
      hipLaunchKernelGGL((pool_split_kernel<SDT, G, false, true>), grid, block, g.lds_bytes, stream, c);
    return hipGetLastError();
  }
  if (a.weighted)
    hipLaunchKernelGGL((pool_split_kernel<SDT, G, true>), grid, block, g.lds_bytes, stream, s);
  else
    hipLaunchKernelGGL((pool_split_kernel<SDT, G, false>), grid, block, g.lds_bytes, stream, s);
  return hipGetLastError();
}

template <int SDT>
hipError_t launch_split_sdt(const PoolLaunch& a, const PoolGeometry& g, hipStream_t stream) {
  switch (g.g) {
    case 8: return launch_split_g<SDT, 8>(a, g, stream);
    case 16: return launch_split_g<SDT, 16>(a, g, stream);
    case 32: return launch_split_g<SDT, 32>(a, g, stream);
    case 64: return launch_split_g<SDT, 64>(a, g, stream);
    default: return hipErrorInvalidValue;
  }
}

// ---------------------------------------------------------------------------
// short bags: one G-lane group per bag, 256 / G bags per workgroup, the bag's
// keys in key order (the same additions as pool_kernel's one-group-per-bag
// path, so the same bits).  MT: several tables in one launch (bag b belongs to
// table b / bags_per_table and writes row (b % bags_per_table) * out_stride +
// table * out_table_stride).
// ---------------------------------------------------------------------------
struct ShortArgs {
  const void* keys;
  const void* offsets;  // null: fixed hotness
  const void* weights;
  void* out;
  const uint8_t* table;  // one table (MT = false)
  int64_t num_keys;
  int64_t num_bags;
  int64_t hotness;
  uint64_t row_bytes;
  uint64_t num_rows;
  int64_t count;
  int64_t out_stride;
  int64_t bags_per_table;
  int64_t out_table_stride;
  int key_bytes;
  int weight_dtype;
  int mean;
  int out_dtype;
};
struct ShortArgsMT : ShortArgs {
  const uint8_t* tables[kMaxPoolTables];
  uint32_t table_rows[kMaxPoolTables];
};

template <int SDT, int G, bool W, bool MT, int UMAX>
__global__ __launch_bounds__(256) void pool_short_kernel(std::conditional_t<MT, ShortArgsMT, ShortArgs> a) {
  constexpr int VB = 16;
  constexpr int ES = Fmt<SDT>::esize;
  constexpr int E = VB / ES;
  constexpr int U = G < UMAX ? G : UMAX;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int gl = tid & (G - 1);
  const int64_t bag = (int64_t)blockIdx.x * (256 / G) + tid / G;
  const bool live = bag < a.num_bags;  // uniform over the group

  int64_t s = 0, e = 0;
  if (live) {
    if (a.offsets != nullptr) {
      s = load_key(a.offsets, a.key_bytes, bag);
      e = load_key(a.offsets, a.key_bytes, bag + 1);
      s = s < 0 ? 0 : (s > a.num_keys ? a.num_keys : s);
      e = e < s ? s : (e > a.num_keys ? a.num_keys : e);
    } else {
      s = bag * a.hotness;
      e = s + a.hotness;
    }
  }
  uint64_t table = (uint64_t)a.table;
  uint64_t num_rows = a.num_rows;
  uint8_t* out_row = reinterpret_cast<uint8_t*>(a.out);
  if constexpr (MT) {
    const int64_t t = live ? bag / a.bags_per_table : 0;
    table = (uint64_t)a.tables[t];
    num_rows = a.table_rows[t];
    out_row += (bag - t * a.bags_per_table) * a.out_stride + t * a.out_table_stride;
  } else {
    out_row += bag * a.out_stride;
  }
  const uint32_t rb32 = (uint32_t)a.row_bytes;  // launcher: row_bytes < 2^32
  const uint64_t zero_row = (uint64_t)g_zero_row;
  const int off = gl * VB;  // < the zero row's size: one pass covers the row
  const bool in_row = off < a.count * ES;

  float acc[E];
#pragma unroll
  for (int c = 0; c < E; ++c) acc[c] = 0.0f;
  float wsum = 0.0f;

  for (int64_t k0 = s; k0 < e; k0 += G) {
    const int64_t kk = k0 + gl;
    uint32_t ridx = kNoRow;
    float w = 0.0f;
    if (kk < e) {
      const int64_t key = load_key(a.keys, a.key_bytes, kk);
      if ((uint64_t)key < num_rows) ridx = (uint32_t)key;  // keys outside the table read nothing
      if (W) w = load_weight(a.weights, a.weight_dtype, kk);
    }
    const int n = (int)((e - k0) < G ? (e - k0) : G);
    auto batch = [&](auto jc) {
      constexpr int j0 = decltype(jc)::value;
      if (j0 >= n) return;
      uint32_t ri[U];
      float wu[U];
      group_bcast_batch<G, U, W, j0>(ridx, w, lane, ri, wu);
      Vec<VB> v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool real = ri[u] != kNoRow && in_row;
        v[u] = load_vec<VB>(real ? table + (uint64_t)ri[u] * rb32 + (uint64_t)off : zero_row + (uint64_t)off);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool use = j0 + u < n;
        if (W && use) wsum += wu[u];
        add_slice<SDT, E, W>(acc, v[u], (use && in_row && ri[u] != kNoRow) ? wu[u] : 0.0f);
      }
    };
    for_batches<U, 0, G / U>(batch);
  }

  if (live && in_row) {
    if (a.mean) {
      const float d = W ? wsum : (float)(e - s);
#pragma unroll
      for (int c = 0; c < E; ++c) acc[c] = (d == 0.0f) ? 0.0f : acc[c] / d;
    }
    const bool out_f16 = a.out_dtype == kF16;
    store_out<E>(out_row + (int64_t)gl * E * (out_f16 ? 2 : 4), acc, out_f16);
  }
}

template <int SDT, int G, bool MT>
hipError_t launch_short_g(const PoolLaunch& a, hipStream_t stream) {
  std::conditional_t<MT, ShortArgsMT, ShortArgs> s{};
  s.keys = a.keys;
  s.offsets = a.offsets;
  s.weights = a.weights;
  s.out = a.out;
  s.table = a.src.table;
  s.num_keys = a.num_keys;
  s.num_bags = a.num_bags;
  s.hotness = a.hotness;
  s.row_bytes = a.src.row_bytes;
  s.num_rows = a.src.num_rows;
  s.count = a.count;
  s.out_stride = a.out_stride;
  s.bags_per_table = a.bags_per_table;
  s.out_table_stride = a.out_table_stride;
  s.key_bytes = a.key_bytes;
  s.weight_dtype = a.weight_dtype;
  s.mean = a.mean;
  s.out_dtype = a.out_dtype;
  if constexpr (MT) {
    for (int t = 0; t < a.num_tables; ++t) {
      s.tables[t] = a.tables[t];
      s.table_rows[t] = (uint32_t)a.table_rows[t];
    }
  }
  const int64_t per_wg = 256 / G;
  const dim3 grid((unsigned)((a.num_bags + per_wg - 1) / per_wg)), block(256);
  // bags of a few dozen keys: 4 loads in flight per lane keep more waves
  // resident, which hides the latency chain of each bag (offsets -> keys ->
  // rows) better than wider batches (measured on 26-table, Poisson(20) bags:
  // 4 -> 124 us, 8 -> 130 us, 16 -> 147 us, 2 -> 128 us); longer bags keep 16
  const int64_t avg = a.keys_per_bag > 0 ? a.keys_per_bag
                                         : a.num_keys / (a.num_bags > 0 ? a.num_bags : 1);
  const bool narrow = avg <= 48;
  if (a.weighted) {
    if (narrow)
      hipLaunchKernelGGL((pool_short_kernel<SDT, G, true, MT, 4>), grid, block, 0, stream, s);
    else
      hipLaunchKernelGGL((pool_short_kernel<SDT, G, true, MT, 16>), grid, block, 0, stream, s);
  } else {
    if (narrow)
      hipLaunchKernelGGL((pool_short_kernel<SDT, G, false, MT, 4>), grid, block, 0, stream, s);
    else
      hipLaunchKernelGGL((pool_short_kernel<SDT, G, false, MT, 16>), grid, block, 0, stream, s);
  }
  return hipGetLastError();
}

template <int SDT, bool MT>
hipError_t launch_short_sdt(const PoolLaunch& a, const PoolGeometry& g, hipStream_t stream) {
  switch (g.g) {
    case 8: return launch_short_g<SDT, 8, MT>(a, stream);
    case 16: return launch_short_g<SDT, 16, MT>(a, stream);
    case 32: return launch_short_g<SDT, 32, MT>(a, stream);
    case 64: return launch_short_g<SDT, 64, MT>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

bool pool_short_eligible(const PoolLaunch& a, const PoolGeometry& g) {
  // short bags over a cache stay on pool_kernel: measured as fast (12.8 us for
  // 8192 bags of 32 keys, all hits) as a cache variant of this kernel
  if (a.src.cache_data != nullptr || !a.src.load_indices) return false;
  if (a.stored_dtype != kF16 && a.stored_dtype != kF32) return false;
  if (a.out_dtype != kF16 && a.out_dtype != kF32) return false;
  if (a.src.row_bytes == 0 || a.src.row_bytes > 0xffffffffull) return false;  // 32-bit row stride
  if (g.vb != 16 || g.passes != 1 || g.gpb != 1 || g.g < 8 || g.g > 64) return false;
  if (a.num_tables > 0) {
    for (int t = 0; t < a.num_tables; ++t)
      if (a.tables[t] == nullptr || a.table_rows[t] == 0 || a.table_rows[t] >= kNoRow) return false;
  } else if (a.src.table == nullptr || a.src.num_rows == 0 || a.src.num_rows >= kNoRow) {
    return false;
  }
  return a.num_bags <= 0x7fffffffLL * (256 / g.g);
}

hipError_t launch_pool_short(const PoolLaunch& a, const PoolGeometry& g, hipStream_t stream) {
  const bool mt = a.num_tables > 0;
  if (a.stored_dtype == kF16)
    return mt ? launch_short_sdt<kF16, true>(a, g, stream) : launch_short_sdt<kF16, false>(a, g, stream);
  if (a.stored_dtype == kF32)
    return mt ? launch_short_sdt<kF32, true>(a, g, stream) : launch_short_sdt<kF32, false>(a, g, stream);
  return hipErrorInvalidValue;
}

bool pool_split_eligible(const PoolLaunch& a, const PoolGeometry& g) {
  if (a.num_tables > 0 || !a.src.load_indices) return false;
  if (a.src.cache_data != nullptr) {
    // 32-bit row codes: cache slots and backing rows below 2^31
    if (a.src.num_sets == 0 || a.src.num_sets * 8 >= kBackingRow) return false;
    if (a.src.table != nullptr && (a.src.num_rows == 0 || a.src.num_rows >= kBackingRow)) return false;
    if (a.key_bytes == 4 && a.src.num_sets > 0xffffffffull) return false;
  } else if (a.src.table == nullptr || a.src.num_rows == 0 || a.src.num_rows >= kNoRow) {
    return false;
  }
  if (a.stored_dtype != kF16 && a.stored_dtype != kF32) return false;
  if (a.out_dtype != kF16 && a.out_dtype != kF32) return false;
  if (a.src.row_bytes == 0 || a.src.row_bytes > 0xffffffffull) return false;  // 32-bit row stride
  if (g.vb != 16 || g.passes != 1 || g.bags_per_wg != 1) return false;
  if (g.g < 8 || g.g > 64 || g.gpb * g.g <= 64 || g.gpb * g.g > 1024) return false;
  if (g.threads != g.gpb * g.g) return false;
  // the cross-wave sum reads at most 16 waves' partials, one element per thread
  const int row_elems = g.g * (16 / (a.stored_dtype == kF16 ? 2 : 4));
  return row_elems <= g.threads;
}

hipError_t launch_pool_split(const PoolLaunch& a, const PoolGeometry& g, hipStream_t stream) {
  if (a.stored_dtype == kF16) return launch_split_sdt<kF16>(a, g, stream);
  if (a.stored_dtype == kF32) return launch_split_sdt<kF32>(a, g, stream);
  return hipErrorInvalidValue;
}

}  // namespace nve_amd
