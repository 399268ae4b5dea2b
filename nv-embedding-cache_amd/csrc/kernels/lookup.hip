// lookup.hip -- gather / dequant / find-and-pool kernels for gfx950 (wave64).
//
// Reference behaviour restated here:
//   find_and_combine  cuda_ops/find_and_combine_kernel.cuh:40-154  (fused find + pool)
//   find_and_dequant  cuda_ops/find_and_dequant.cuh:41-123         (per-key gather + dequant)
//   query / query_uvm include/ecache/ec_set_associative.cuh:263-466, embed_cache.cuh:52-118
//   sanitize          cuda_ops/sanitize_keys.cuh:30-45
//
// Design (MI355X-first, not the reference's warp32 shape): a "group" of G
// lanes owns one row at a time, lane l moving bytes [l*VB, l*VB+VB) with one
// VB-byte load; keys are resolved one per lane (the cache's 8-tag compare
// included) and their row addresses broadcast inside the group with
// ds_bpermute; a batch's row loads are all issued before any is consumed.
// The find-and-pool kernel lives in pool_kernel.cuh.
#include "device_common.cuh"
#include "pool_launch.hpp"

namespace nve_amd {

// ---------------------------------------------------------------------------
// gather: one output row per key (raw bytes or dequantized values)
//
// U row loads per lane group are issued before any is used; a key that
// resolves to no row (hit-mask skip, cache miss without a backing table, past
// the end of the keys) reads the zero row, so no load sits behind a branch and
// nothing is stored for it.  MW: the row's quantization metadata is aligned to
// its own size, so scale (and offset) come with one load.
// ---------------------------------------------------------------------------
template <int SDT, int VB, bool RAW, int U, bool MW>
__global__ __launch_bounds__(256) void gather_kernel(GatherLaunch a, int g_shift, int t_shift,
                                                     int passes) {
  constexpr int ES = RAW ? 1 : Fmt<SDT>::esize;
  constexpr int E = VB / ES;
  // a wave resolves T = 2^t_shift keys (T <= 64): enough for each lane group
  // to move its share in one batch of U loads, so narrow launches still have
  // many waves and every wave one round trip
  const int T = 1 << t_shift;
  const int lane = threadIdx.x & 63;
  const int64_t tile = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int64_t base = tile << t_shift;
  const int64_t i = base + lane;
  const bool valid = lane < T && i < a.n;

  // ---- resolve: one key per lane ----
  // hit-mask words cover 64 keys; a wave owns bits [sub, sub + T) of its word
  const int64_t word = base >> 6;
  const int sub = (int)(base & 63);
  uint64_t in_word = 0;
  bool skip = false;
  if (a.hitmask != nullptr && base < a.n) {
    in_word = a.hitmask[word];
    skip = lane < T && ((in_word >> (sub + lane)) & 1u);
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
    const uint64_t hits = __ballot(addr != 0);  // lanes >= T never resolve
    if (lane == 0 && base < a.n) {
      if (T == 64)
        a.hitmask[word] = in_word | hits;
      else if (hits)  // other waves own the word's other bits
        atomicOr(reinterpret_cast<unsigned long long*>(a.hitmask + word),
                 (unsigned long long)(hits << sub));
    }
  }
  if (a.miss_counter != nullptr) add_misses(a.miss_counter, miss ? 1u : 0u);

  // ---- copy: group grp moves keys grp, grp+groups, ... of the tile ----
  const int G = 1 << g_shift;
  const int gl = lane & (G - 1);
  const int grp = lane >> g_shift;
  const int groups = 64 >> g_shift;
  const int per_group = T >> (6 - g_shift) > 0 ? T >> (6 - g_shift) : 1;  // keys per group
  const int64_t area = RAW ? (int64_t)a.src.row_bytes : a.count * ES;
  const bool out_f16 = a.out_dtype == kF16;
  const int out_es = out_f16 ? 2 : 4;
  const uint64_t zero_row = (uint64_t)g_zero_row;
  uint8_t* out = reinterpret_cast<uint8_t*>(a.out);
  for (int p = 0; p < passes; ++p) {
    const int64_t off = ((int64_t)p * G + gl) * VB;
    const bool in_row = off < area;
    for (int q0 = 0; q0 < per_group; q0 += U) {
      uint64_t ra[U];
      uint32_t orw[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int q = q0 + u;
        const int j = grp + (q < per_group ? q : 0) * groups;
        ra[u] = shfl64(addr, j);
        orw[u] = a.out_index != nullptr ? shfl32(orow, j) : 0u;
        if (q >= per_group) ra[u] = 0;
      }
      Vec<VB> v[U];
      Meta m[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool real = ra[u] != 0;
        const uint64_t row = real ? ra[u] : zero_row;
        v[u] = load_vec<VB>(row + ((real && in_row) ? off : (off & kZeroRowMask)));
        if constexpr (!RAW && Fmt<SDT>::meta != 0)
          m[u] = load_meta<SDT, MW>(row, real ? area : (area & kZeroRowMask));
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (ra[u] == 0 || !in_row) continue;
        const int64_t row = a.out_index != nullptr ? (int64_t)orw[u]
                                                   : base + grp + (int64_t)(q0 + u) * groups;
        uint8_t* o = out + row * a.out_stride;
        if constexpr (RAW) {
          store_vec<VB>(o + off, v[u]);
        } else {
          float x[E];
          decode<SDT, VB>(v[u], m[u], x);
          store_out<E>(o + ((int64_t)p * G + gl) * E * out_es, x, out_f16);
        }
      }
    }
  }
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
  const int gs = log2i(g);
  // 16 loads in flight per lane group for rows of 16+ lane slices; a wave
  // resolves groups * unroll keys (at most 64), one batch per group
  const int unroll = g >= 16 ? 16 : 8;
  const int tkeys = (64 / g) * unroll < 64 ? (64 / g) * unroll : 64;
  const int ts = log2i(tkeys);
  const int64_t waves = (a.n + tkeys - 1) / tkeys;
  const int threads = 256;
  const int64_t grid = (waves * 64 + threads - 1) / threads;
  // metadata aligned to its own size in every row (cache rows included)
  bool mw = false;
  if (!a.raw) {
    const int mb = meta_bytes(a.stored_dtype);
    const int ma = (mb == 8) ? 8 : 4;
    mw = mb >= 4 && area % ma == 0 && a.src.row_bytes % (uint64_t)ma == 0 &&
         (!a.src.table || aligned(a.src.table, ma)) && (!a.src.cache_data || aligned(a.src.cache_data, ma));
  }
#define L_RAW(V)                                                                                  \
  do {                                                                                            \
    if (unroll == 16)                                                                             \
      hipLaunchKernelGGL((gather_kernel<kF16, V, true, 16, false>), dim3(grid), dim3(threads), 0, \
                         stream, a, gs, ts, passes);                                                  \
    else                                                                                          \
      hipLaunchKernelGGL((gather_kernel<kF16, V, true, 8, false>), dim3(grid), dim3(threads), 0,  \
                         stream, a, gs, ts, passes);                                                  \
  } while (0)
#define L_DQ_U(S, V, M)                                                                           \
  do {                                                                                            \
    if (unroll == 16)                                                                             \
      hipLaunchKernelGGL((gather_kernel<S, V, false, 16, M>), dim3(grid), dim3(threads), 0,       \
                         stream, a, gs, ts, passes);                                                  \
    else                                                                                          \
      hipLaunchKernelGGL((gather_kernel<S, V, false, 8, M>), dim3(grid), dim3(threads), 0,        \
                         stream, a, gs, ts, passes);                                                  \
  } while (0)
#define L_DQ(S, V)             \
  do {                         \
    if (mw)                    \
      L_DQ_U(S, V, true);      \
    else                       \
      L_DQ_U(S, V, false);     \
  } while (0)
#define L_DQN(S, V) L_DQ_U(S, V, false)
  if (a.raw) {
    NVE_DISPATCH_VB(vb, L_RAW);
  } else {
    switch (a.stored_dtype) {
#define C_F32(V) L_DQN(kF32, V)
#define C_F16(V) L_DQN(kF16, V)
#define C_QI8F32(V) L_DQ(kQI8F32, V)
#define C_QI8F16(V) L_DQN(kQI8F16, V)
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
  if (a.force_unroll == 0 && pool_split_eligible(a, g)) return launch_pool_split(a, g, stream);
  if (a.force_unroll == 0 && pool_short_eligible(a, g)) return launch_pool_short(a, g, stream);
  switch (a.stored_dtype) {
    case kF32:
    case kF16:
      return launch_pool_float(a, g, stream);
    case kQI8F32:
    case kQI8F16:
    case kQU8F32:
    case kQU8F16:
      return launch_pool_quant(a, g, stream);
    case kXI8AF32:
    case kXE4M3F32:
      return launch_pool_ext(a, g, stream);
    default:
      return hipErrorInvalidValue;
  }
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
