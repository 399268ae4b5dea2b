// lookup.hip -- gather / dequant / find-and-pool kernels for gfx950 (wave64).
//
// Reference behaviour restated here:
//   find_and_combine  cuda_ops/find_and_combine_kernel.cuh:40-154  (fused find + pool)
//   find_and_dequant  cuda_ops/find_and_dequant.cuh:41-123         (per-key gather + dequant)
//   query / query_uvm include/ecache/ec_set_associative.cuh:263-466, embed_cache.cuh:52-118
//   sanitize          cuda_ops/sanitize_keys.cuh:30-45
//
// Design (MI355X-first, not the reference's warp32 shape):
//  * A "group" of G lanes (G a power of two <= 64) owns one row at a time; lane
//    l of the group moves bytes [l*VB, l*VB+VB) of the row with one VB-byte
//    load (VB = 16 for 16-byte aligned rows), so a 256-byte fp16 row is one
//    dwordx4 load per lane over 16 lanes and a wave carries four rows per
//    instruction.
//  * Keys are resolved one per lane (the cache's 8-tag compare included), then
//    row addresses are broadcast inside the group with ds_bpermute; U = 8 row
//    loads are issued before any is consumed to keep HBM requests in flight.
//  * Pooling keeps one fp32 accumulator per element in registers.  Short bags
//    (the common CSR case) are reduced by one group in key order -- the
//    reference's per-element order.  Few long bags are split over up to 64
//    groups of one workgroup in contiguous key chunks, combined by a fixed
//    binary tree in LDS (deterministic, within fp32 tolerance of key order).
#include "device_common.cuh"

namespace nve_amd {

constexpr int kUnroll = 8;

__device__ __forceinline__ float load_weight(const void* w, int wdt, int64_t k) {
  return wdt == kF16 ? h2f(reinterpret_cast<const uint16_t*>(w)[k])
                     : reinterpret_cast<const float*>(w)[k];
}

__device__ __forceinline__ void add_misses(unsigned long long* counter, uint32_t n) {
  // every lane of the wave is active here; fold the per-lane counts
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) n += __shfl_xor(n, o);
  if (__lane_id() == 0 && n) atomicAdd(counter, (unsigned long long)n);
}

// ---------------------------------------------------------------------------
// gather: one output row per key (raw bytes or dequantized values)
// ---------------------------------------------------------------------------
template <int SDT, int VB, bool RAW>
__global__ __launch_bounds__(256) void gather_kernel(GatherLaunch a, int g_shift, int passes) {
  constexpr int ES = RAW ? 1 : Fmt<SDT>::esize;
  constexpr int E = VB / ES;
  const int lane = threadIdx.x & 63;
  const int64_t tile = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int64_t i = tile * 64 + lane;
  const bool valid = i < a.n;

  // ---- resolve: one key per lane ----
  uint64_t in_word = 0;
  bool skip = false;
  if (a.hitmask != nullptr && tile * 64 < a.n) {
    in_word = a.hitmask[tile];
    skip = (in_word >> lane) & 1u;
  }
  uint64_t addr = 0;
  bool miss = false;
  uint32_t orow = (uint32_t)i;  // output row of this key
  if (valid && !skip) {
    const int64_t key = a.src.load_indices ? load_key(a.keys, a.key_bytes, i) : i;
    addr = resolve_row(a.src, a.key_bytes, key, i, &miss);
    if (a.out_index != nullptr) orow = a.out_index[i];
  }
  if (a.hitmask != nullptr) {
    const uint64_t hits = __ballot(addr != 0);
    if (lane == 0 && tile * 64 < a.n) a.hitmask[tile] = in_word | hits;
  }
  if (a.miss_counter != nullptr) add_misses(a.miss_counter, miss ? 1u : 0u);

  // ---- copy: group grp moves keys grp, grp+groups, ... of the tile ----
  const int G = 1 << g_shift;
  const int gl = lane & (G - 1);
  const int grp = lane >> g_shift;
  const int groups = 64 >> g_shift;
  const int64_t area = RAW ? (int64_t)a.src.row_bytes : a.count * ES;
  const int out_es = (a.out_dtype == kF16) ? 2 : 4;
  uint8_t* out = reinterpret_cast<uint8_t*>(a.out);
  for (int p = 0; p < passes; ++p) {
    const int64_t off = ((int64_t)p * G + gl) * VB;
    const bool in_row = off < area;
    for (int q0 = 0; q0 < G; q0 += kUnroll) {
      Vec<VB> v[kUnroll];
      Meta m[kUnroll];
      uint64_t ra[kUnroll];
      uint32_t orw[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int q = q0 + u;
        const int j = grp + (q < G ? q : 0) * groups;
        ra[u] = shfl64(addr, j);
        orw[u] = a.out_index != nullptr ? shfl32(orow, j) : 0u;
        if (q >= G) ra[u] = 0;
        if (ra[u] != 0 && in_row) v[u] = load_vec<VB>(reinterpret_cast<const uint8_t*>(ra[u]) + off);
        if constexpr (!RAW && Fmt<SDT>::meta != 0) {
          if (ra[u] != 0) m[u] = load_meta<SDT>(reinterpret_cast<const uint8_t*>(ra[u]), area);
        }
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        if (ra[u] == 0 || !in_row) continue;
        const int64_t row = a.out_index != nullptr ? (int64_t)orw[u]
                                                   : tile * 64 + grp + (int64_t)(q0 + u) * groups;
        uint8_t* o = out + row * a.out_stride;
        if constexpr (RAW) {
          store_vec<VB>(o + off, v[u]);
        } else {
          float x[E];
          decode<SDT, VB>(v[u], m[u], x);
          store_out<E>(o + ((int64_t)p * G + gl) * E * out_es, x, a.out_dtype == kF16);
        }
      }
    }
  }
}

// Readable zeros for keys that resolve to no row: their loads are pointed
// here (offsets folded into the buffer) so that every load of a batch can be
// issued unconditionally.
constexpr int kZeroRowBytes = 4096;
constexpr int64_t kZeroRowMask = kZeroRowBytes - 1;
__device__ __align__(16) uint8_t g_zero_row[kZeroRowBytes + 64] = {};

// ---------------------------------------------------------------------------
// find-and-pool: one output row per bag
// ---------------------------------------------------------------------------
// Output row of bag g (one table, or bag g of several tables in one launch).
__device__ __forceinline__ uint8_t* bag_out_row(const PoolLaunch& a, int64_t g) {
  uint8_t* out = reinterpret_cast<uint8_t*>(a.out);
  if (a.num_tables > 0)
    return out + (g % a.bags_per_table) * a.out_stride + (g / a.bags_per_table) * a.out_table_stride;
  return out + g * a.out_stride;
}

template <int SDT, int VB, int U>
__global__ __launch_bounds__(1024) void pool_kernel(PoolLaunch a, int g_shift, int gpb_shift,
                                                   int passes) {
  constexpr int ES = Fmt<SDT>::esize;
  constexpr int E = VB / ES;
  extern __shared__ float lds[];

  const int G = 1 << g_shift;
  const int tid = threadIdx.x;
  const int gl = tid & (G - 1);
  const int grp = tid >> g_shift;
  const int gbase = (tid & 63) - gl;  // first lane of this group inside the wave
  const int gpb = 1 << gpb_shift;
  const int chunk = grp & (gpb - 1);
  const int bags_per_wg = (int)(blockDim.x >> g_shift) >> gpb_shift;
  const int64_t bag = (int64_t)blockIdx.x * bags_per_wg + (grp >> gpb_shift);
  const bool live = bag < a.num_bags;

  int64_t s = 0, e = 0;
  if (live) {
    if (a.offsets != nullptr) {
      s = load_key(a.offsets, a.key_bytes, bag);
      e = load_key(a.offsets, a.key_bytes, bag + 1);
      // offsets are caller data: keep every key / weight access inside [0, num_keys)
      s = s < 0 ? 0 : (s > a.num_keys ? a.num_keys : s);
      e = e < s ? s : (e > a.num_keys ? a.num_keys : e);
    } else {
      s = bag * a.hotness;
      e = s + a.hotness;
    }
  }
  // the bag's table (several tables in one launch) and output row
  RowSource src = a.src;
  if (a.num_tables > 0 && live) src.table = a.tables[bag / a.bags_per_table];
  int64_t cs = s, ce = e;
  if (gpb > 1 && e > s) {
    const int64_t per = (e - s + gpb - 1) >> gpb_shift;
    cs = s + chunk * per;
    if (cs > e) cs = e;
    ce = cs + per < e ? cs + per : e;
  }

  const bool weighted = a.weighted != 0;
  const int64_t value_bytes = a.count * ES;
  const uint64_t zero_row = (uint64_t)g_zero_row;
  const bool out_f16 = a.out_dtype == kF16;
  const int out_es = out_f16 ? 2 : 4;
  uint32_t misses = 0;

  for (int p = 0; p < passes; ++p) {
    const int64_t off = ((int64_t)p * G + gl) * VB;
    const bool in_row = off < value_bytes;
    float acc[E];
#pragma unroll
    for (int x = 0; x < E; ++x) acc[x] = 0.0f;
    float wsum = 0.0f;

    for (int64_t k0 = cs; k0 < ce; k0 += G) {
      // resolve G keys, one per lane
      const int64_t kk = k0 + gl;
      uint64_t addr = 0;
      float w = 0.0f;
      if (kk < ce) {
        const int64_t key = a.src.load_indices ? load_key(a.keys, a.key_bytes, kk) : kk;
        bool miss;
        addr = resolve_row(src, a.key_bytes, key, kk, &miss);
        if (p == 0 && miss) misses++;
        if (weighted) w = load_weight(a.weights, a.weight_dtype, kk);
      }
      const int n = (int)((ce - k0) < G ? (ce - k0) : G);
      for (int j0 = 0; j0 < n; j0 += U) {
        // (1) the batch's row addresses (and weights) from the lanes that
        // resolved them; slots past the group's keys repeat its last key
        uint64_t ra[U];
        float wu[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int j = (j0 + u < n) ? j0 + u : n - 1;
          ra[u] = shfl64(addr, gbase + j);
          wu[u] = weighted ? shflf(w, gbase + j) : 1.0f;
        }
        // (2) every row load of the batch in flight at once; a key that did
        // not resolve (outside the table) reads the zero row instead
        Vec<VB> v[U];
        Meta m[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const bool real = ra[u] != 0;
          const uint64_t row = real ? ra[u] : zero_row;
          v[u] = load_vec<VB>(row + ((real && in_row) ? off : (off & kZeroRowMask)));
          if constexpr (Fmt<SDT>::meta != 0)
            m[u] = load_meta<SDT>(reinterpret_cast<const uint8_t*>(row),
                                  real ? value_bytes : (value_bytes & kZeroRowMask));
        }
        // (3) accumulate in key order; an unresolved key adds a zero row
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const bool use = j0 + u < n;  // uniform over the group
          if (weighted && use) wsum += wu[u];
          const bool add = use && in_row && ra[u] != 0;
          float x[E];
          decode<SDT, VB>(v[u], m[u], x);
#pragma unroll
          for (int c = 0; c < E; ++c) {
            const float t = weighted ? __builtin_fmaf(x[c], wu[u], acc[c]) : acc[c] + x[c];
            acc[c] = add ? t : acc[c];
          }
        }
      }
    }

    if (gpb == 1) {
      // one group per bag: the bag was reduced in key order
      if (live && in_row) {
        if (a.mean) {
          const float d = weighted ? wsum : (float)(e - s);
#pragma unroll
          for (int c = 0; c < E; ++c) acc[c] = (d == 0.0f) ? 0.0f : acc[c] / d;
        }
        uint8_t* o = bag_out_row(a, bag) + ((int64_t)p * G + gl) * E * out_es;
        store_out<E>(o, acc, out_f16);
      }
      continue;
    }

    // Split bag.  (1) Butterfly over the bag's groups inside the wave: step m
    // pairs lane l with lane l ^ m, so after log2(span / G) steps every lane of
    // the bag holds ((g0 + g1) + (g2 + g3)) ... (float addition is commutative,
    // both partners compute the same bits).
    const int span = gpb * G < 64 ? gpb * G : 64;
    for (int mk = G; mk < span; mk <<= 1) {
#pragma unroll
      for (int c = 0; c < E; ++c) acc[c] += __shfl_xor(acc[c], mk);
      wsum += __shfl_xor(wsum, mk);
    }
    if (gpb * G <= 64) {
      if (chunk == 0 && live && in_row) {
        if (a.mean) {
          const float d = weighted ? wsum : (float)(e - s);
#pragma unroll
          for (int c = 0; c < E; ++c) acc[c] = (d == 0.0f) ? 0.0f : acc[c] / d;
        }
        uint8_t* o = bag_out_row(a, bag) + ((int64_t)p * G + gl) * E * out_es;
        store_out<E>(o, acc, out_f16);
      }
      continue;
    }

    // (2) The bag spans several waves: each wave's first group parks its
    // partial row in LDS, then one thread per output element adds the waves'
    // partials in wave order and writes the element.
    const int row_elems = G * E;
    const int wave = tid >> 6;
    const int waves_per_bag = (gpb * G) >> 6;
    float* red = lds;
    float* wred = lds + (blockDim.x >> 6) * row_elems;
    if ((tid & 63) < G) {
#pragma unroll
      for (int c = 0; c < E; ++c) red[wave * row_elems + gl * E + c] = acc[c];
      if (gl == 0) wred[wave] = wsum;
    }
    __syncthreads();
    for (int idx = tid; idx < bags_per_wg * row_elems; idx += blockDim.x) {
      const int b = idx / row_elems;
      const int x = idx - b * row_elems;
      const int64_t bg = (int64_t)blockIdx.x * bags_per_wg + b;
      const bool elem_in_row = ((int64_t)p * G + x / E) * VB < value_bytes;
      if (bg < a.num_bags && elem_in_row) {
        const int w0 = b * waves_per_bag;
        float v = red[w0 * row_elems + x];
        float ws = wred[w0];
        for (int w = 1; w < waves_per_bag; ++w) {
          v += red[(w0 + w) * row_elems + x];
          ws += wred[w0 + w];
        }
        if (a.mean) {
          float d;
          if (weighted) {
            d = ws;
          } else {
            int64_t bs, be;
            if (a.offsets != nullptr) {
              bs = load_key(a.offsets, a.key_bytes, bg);
              be = load_key(a.offsets, a.key_bytes, bg + 1);
              bs = bs < 0 ? 0 : (bs > a.num_keys ? a.num_keys : bs);
              be = be < bs ? bs : (be > a.num_keys ? a.num_keys : be);
            } else {
              bs = 0;
              be = a.hotness;
            }
            d = (float)(be - bs);
          }
          v = (d == 0.0f) ? 0.0f : v / d;
        }
        uint8_t* o = bag_out_row(a, bg) + ((int64_t)p * row_elems + x) * out_es;
        if (out_f16)
          *reinterpret_cast<uint16_t*>(o) = f2h(v);
        else
          *reinterpret_cast<float*>(o) = v;
      }
    }
    __syncthreads();
  }
  if (a.miss_counter != nullptr) add_misses(a.miss_counter, misses);
}

// ---------------------------------------------------------------------------
// sanitize (sanitize_keys.cuh:30-45): keys outside [0, rows) -> default row
// ---------------------------------------------------------------------------
template <typename K>
__global__ __launch_bounds__(256) void sanitize_kernel(const K* in, K* out, int64_t n,
                                                       uint64_t rows, K def) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    const K k = in[i];
    out[i] = (k >= 0 && (uint64_t)k < rows) ? k : def;
  }
}

// ---------------------------------------------------------------------------
// random-row read ceiling: 16 lanes x 16 bytes per 256-byte row, 8 rows in
// flight per lane group, nothing written but one word per workgroup.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void read_ceiling_kernel(const uint8_t* table, uint64_t row_bytes,
                                                           const int64_t* idx, int64_t n,
                                                           uint32_t* sink) {
  const int lane = threadIdx.x & 63;
  const int vecs = (int)(row_bytes / 16);
  const int gl = lane & 15;
  const int grp = lane >> 4;
  const int64_t tile = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  uint32_t fold = 0;
  const int64_t base = tile * 32;  // 32 rows per wave: 4 groups x 8 rows
  int64_t r[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int64_t i = base + grp + 4 * u;
    r[u] = i < n ? idx[i] : -1;
  }
  for (int c = gl; c < vecs; c += 16) {
    Vec<16> v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u)
      v[u] = load_vec<16>((uint64_t)table + (uint64_t)(r[u] >= 0 ? r[u] : 0) * row_bytes + 16 * c);
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (r[u] >= 0) fold ^= v[u].w[0] ^ v[u].w[1] ^ v[u].w[2] ^ v[u].w[3];
  }
  __shared__ uint32_t red[256];
  red[threadIdx.x] = fold;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t f = 0;
    for (int t = 0; t < (int)blockDim.x; ++t) f ^= red[t];
    sink[blockIdx.x] = f;
  }
}

// ---------------------------------------------------------------------------
// host launchers
// ---------------------------------------------------------------------------
namespace {

int pow2_ceil(int64_t x) {
  int p = 1;
  while (p < x) p <<= 1;
  return p;
}
int log2i(int x) {
  int l = 0;
  while ((1 << l) < x) ++l;
  return l;
}
bool aligned(const void* p, int a) { return ((uintptr_t)p % (uintptr_t)a) == 0; }

// Largest vector width (bytes) every row slice, output slice and base pointer
// is aligned to.
int pick_vb(int max_vb, int esize, int out_es, int64_t area, const RowSource& src,
            const void* out, int64_t out_stride) {
  for (int vb = max_vb; vb >= esize; vb >>= 1) {
    if (area % vb) continue;
    if (src.row_bytes % (uint64_t)vb) continue;
    if (src.table && !aligned(src.table, vb)) continue;
    if (src.cache_data && !aligned(src.cache_data, vb)) continue;
    const int ob = (vb / esize) * out_es;  // output bytes per lane slice
    if (out_es > 0) {
      if (!aligned(out, ob) || (out_stride % ob)) continue;
    }
    return vb;
  }
  return 0;
}

int max_vb_of(int sdt) { return value_elem_bytes(sdt) == 1 ? 8 : 16; }

#define NVE_DISPATCH_VB(VBV, CALL) \
  switch (VBV) {                   \
    case 16: CALL(16); break;      \
    case 8: CALL(8); break;        \
    case 4: CALL(4); break;        \
    case 2: CALL(2); break;        \
    case 1: CALL(1); break;        \
    default: return hipErrorInvalidValue; \
  }

}  // namespace

hipError_t launch_gather(const GatherLaunch& a, hipStream_t stream) {
  if (a.n <= 0) return hipSuccess;
  const int esize = a.raw ? 1 : value_elem_bytes(a.stored_dtype);
  const int64_t area = a.raw ? (int64_t)a.src.row_bytes : a.count * esize;
  const int out_es = a.raw ? 0 : (a.out_dtype == kF16 ? 2 : 4);
  int vb;
  if (a.raw) {
    vb = 0;
    for (int c = 16; c >= 1; c >>= 1) {
      if (area % c || (a.src.table && !aligned(a.src.table, c)) ||
          (a.src.cache_data && !aligned(a.src.cache_data, c)) || !aligned(a.out, c) ||
          a.out_stride % c)
        continue;
      vb = c;
      break;
    }
  } else {
    vb = pick_vb(max_vb_of(a.stored_dtype), esize, out_es, area, a.src, a.out, a.out_stride);
  }
  if (vb == 0) return hipErrorInvalidValue;
  const int64_t nv = area / vb;
  const int g = nv >= 64 ? 64 : pow2_ceil(nv);
  const int passes = (int)((nv + g - 1) / g);
  const int64_t waves = (a.n + 63) / 64;
  const int threads = 256;
  const int64_t grid = (waves * 64 + threads - 1) / threads;
  const int gs = log2i(g);
#define L_RAW(V) hipLaunchKernelGGL((gather_kernel<kF16, V, true>), dim3(grid), dim3(threads), 0, stream, a, gs, passes)
#define L_DQ(S, V) hipLaunchKernelGGL((gather_kernel<S, V, false>), dim3(grid), dim3(threads), 0, stream, a, gs, passes)
  if (a.raw) {
    NVE_DISPATCH_VB(vb, L_RAW);
  } else {
    switch (a.stored_dtype) {
#define C_F32(V) L_DQ(kF32, V)
#define C_F16(V) L_DQ(kF16, V)
#define C_QI8F32(V) L_DQ(kQI8F32, V)
#define C_QI8F16(V) L_DQ(kQI8F16, V)
#define C_QU8F32(V) L_DQ(kQU8F32, V)
#define C_QU8F16(V) L_DQ(kQU8F16, V)
#define C_XI8A(V) L_DQ(kXI8AF32, V)
#define C_XE4M3(V) L_DQ(kXE4M3F32, V)
      case kF32:
        switch (vb) { case 16: C_F32(16); break; case 8: C_F32(8); break; case 4: C_F32(4); break; default: return hipErrorInvalidValue; }
        break;
      case kF16:
        switch (vb) { case 16: C_F16(16); break; case 8: C_F16(8); break; case 4: C_F16(4); break; case 2: C_F16(2); break; default: return hipErrorInvalidValue; }
        break;
      case kQI8F32: NVE_DISPATCH_VB(vb, C_QI8F32); break;
      case kQI8F16: NVE_DISPATCH_VB(vb, C_QI8F16); break;
      case kQU8F32: NVE_DISPATCH_VB(vb, C_QU8F32); break;
      case kQU8F16: NVE_DISPATCH_VB(vb, C_QU8F16); break;
      case kXI8AF32: NVE_DISPATCH_VB(vb, C_XI8A); break;
      case kXE4M3F32: NVE_DISPATCH_VB(vb, C_XE4M3); break;
      default: return hipErrorInvalidValue;
    }
  }
  return hipGetLastError();
}

bool pool_geometry(const PoolLaunch& a, PoolGeometry* g) {
  const int esize = value_elem_bytes(a.stored_dtype);
  const int64_t area = a.count * esize;
  const int out_es = a.out_dtype == kF16 ? 2 : 4;
  int vb = pick_vb(max_vb_of(a.stored_dtype), esize, out_es, area, a.src, a.out, a.out_stride);
  // several tables: every table and every table's output column must allow it
  for (int t = 0; t < a.num_tables && vb > 0; ++t) {
    RowSource st = a.src;
    st.table = a.tables[t];
    vb = pick_vb(vb, esize, out_es, area, st, a.out, a.out_stride);
  }
  if (a.num_tables > 0) {
    while (vb >= esize && a.out_table_stride % ((vb / esize) * out_es) != 0) vb >>= 1;
    if (vb < esize) vb = 0;
  }
  if (vb == 0) return false;
  const int64_t nv = area / vb;
  const int G = nv >= 64 ? 64 : pow2_ceil(nv);
  const int passes = (int)((nv + G - 1) / G);
  const int64_t bags = a.num_bags;
  const int64_t avg = a.keys_per_bag > 0 ? a.keys_per_bag : (bags > 0 ? a.num_keys / bags : 0);
  int gpb = 1;
  if (a.force_split > 0) {
    gpb = pow2_ceil(a.force_split);
  } else if (a.force_split == 0) {
    // split long bags when there are too few bags to keep the chip's 256 CUs
    // streaming: aim at ~16 keys per group
    if (avg > 32 && bags * (int64_t)G < 256LL * 1024) {
      int64_t want = avg / 16;
      gpb = 1;
      while ((int64_t)gpb * 2 <= want) gpb <<= 1;
    }
  }
  if (gpb * G > 1024) gpb = 1024 / G;
  if (gpb < 1) gpb = 1;
  int threads;
  if (gpb == 1) {
    threads = 256;
  } else {
    threads = gpb * G;
    if (threads < 256) threads = 256;
  }
  const int bags_per_wg = threads / (gpb * G);
  g->vb = vb;
  g->g = G;
  g->passes = passes;
  g->gpb = gpb;
  g->threads = threads;
  g->bags_per_wg = bags_per_wg;
  g->grid = (bags + bags_per_wg - 1) / bags_per_wg;
  // LDS only when a bag spans several waves: one partial row + weight sum per wave
  g->lds_bytes = gpb * G > 64 ? (int)((threads / 64) * (G * (vb / esize) * 4 + 4)) : 0;
  // 16 row loads in flight per group only pay off when a group walks long
  // key runs; 16-key chunks (the 1024-key bags of the benchmark over 64
  // groups) measured slightly faster with 8
  g->unroll = (avg / gpb) >= 32 ? 16 : 8;
  if (a.force_unroll == 8 || a.force_unroll == 16) g->unroll = a.force_unroll;
  return true;
}

hipError_t launch_pool(const PoolLaunch& a, hipStream_t stream) {
  if (a.num_bags <= 0) return hipSuccess;
  PoolGeometry g;
  if (!pool_geometry(a, &g)) return hipErrorInvalidValue;
  if (g.grid > 0x7fffffffLL) return hipErrorInvalidValue;
  const int gs = log2i(g.g);
  const int ps = log2i(g.gpb);
#define L_POOL(S, V)                                                                        \
  do {                                                                                      \
    if (g.unroll == 16)                                                                     \
      hipLaunchKernelGGL((pool_kernel<S, V, 16>), dim3(g.grid), dim3(g.threads), g.lds_bytes, \
                         stream, a, gs, ps, g.passes);                                      \
    else                                                                                    \
      hipLaunchKernelGGL((pool_kernel<S, V, 8>), dim3(g.grid), dim3(g.threads), g.lds_bytes,  \
                         stream, a, gs, ps, g.passes);                                      \
  } while (0)
#define P_F32(V) L_POOL(kF32, V)
#define P_F16(V) L_POOL(kF16, V)
#define P_QI8F32(V) L_POOL(kQI8F32, V)
#define P_QI8F16(V) L_POOL(kQI8F16, V)
#define P_QU8F32(V) L_POOL(kQU8F32, V)
#define P_QU8F16(V) L_POOL(kQU8F16, V)
#define P_XI8A(V) L_POOL(kXI8AF32, V)
#define P_XE4M3(V) L_POOL(kXE4M3F32, V)
  switch (a.stored_dtype) {
    case kF32:
      switch (g.vb) { case 16: P_F32(16); break; case 8: P_F32(8); break; case 4: P_F32(4); break; default: return hipErrorInvalidValue; }
      break;
    case kF16:
      switch (g.vb) { case 16: P_F16(16); break; case 8: P_F16(8); break; case 4: P_F16(4); break; case 2: P_F16(2); break; default: return hipErrorInvalidValue; }
      break;
    case kQI8F32: NVE_DISPATCH_VB(g.vb, P_QI8F32); break;
    case kQI8F16: NVE_DISPATCH_VB(g.vb, P_QI8F16); break;
    case kQU8F32: NVE_DISPATCH_VB(g.vb, P_QU8F32); break;
    case kQU8F16: NVE_DISPATCH_VB(g.vb, P_QU8F16); break;
    case kXI8AF32: NVE_DISPATCH_VB(g.vb, P_XI8A); break;
    case kXE4M3F32: NVE_DISPATCH_VB(g.vb, P_XE4M3); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_sanitize(const void* keys, void* out, int64_t n, int key_bytes, uint64_t num_rows,
                           int64_t default_row, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  const int64_t grid = (n + 255) / 256;
  if (key_bytes == 4) {
    hipLaunchKernelGGL(sanitize_kernel<int32_t>, dim3(grid), dim3(256), 0, stream,
                       (const int32_t*)keys, (int32_t*)out, n, num_rows, (int32_t)default_row);
  } else {
    hipLaunchKernelGGL(sanitize_kernel<int64_t>, dim3(grid), dim3(256), 0, stream,
                       (const int64_t*)keys, (int64_t*)out, n, num_rows, (int64_t)default_row);
  }
  return hipGetLastError();
}

hipError_t launch_read_ceiling(const uint8_t* table, uint64_t row_bytes, const int64_t* idx,
                               int64_t n, uint32_t* sink, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  if (row_bytes % 16 || !aligned(table, 16)) return hipErrorInvalidValue;
  const int64_t waves = (n + 31) / 32;
  const int64_t grid = (waves * 64 + 255) / 256;
  hipLaunchKernelGGL(read_ceiling_kernel, dim3(grid), dim3(256), 0, stream, table, row_bytes, idx,
                     n, sink);
  return hipGetLastError();
}

}  // namespace nve_amd
