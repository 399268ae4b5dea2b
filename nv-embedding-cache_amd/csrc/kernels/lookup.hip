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
#include "lane_moves.cuh"
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
// Keys base .. base + T - 1 of the launch, one per lane (T <= 64): returns
// the lane's row address (0: no row) and sets its output row.  Updates the
// hit mask and the miss counter.
__device__ __forceinline__ uint64_t resolve_tile(const GatherLaunch& a, int64_t base, int T,
                                                 int lane, uint32_t* out_row) {
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
  *out_row = orow;
  return addr;
}

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
  uint32_t orow;
  const uint64_t addr = resolve_tile(a, base, T, lane, &orow);

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
// gather_realign: dequantizing gather of one-byte formats whose rows are not
// 16-byte aligned (the quantized layouts: count values + 2..8 bytes of scale
// and offset, so a 256-value row is 258..264 bytes and starts at any 2-, 4- or
// 8-byte boundary).
//
// A row at address R = B + s (B 16-byte aligned, s = R % 16) is owned by
// G = count / 16 lanes.  Lane gl loads the aligned chunk B + 16*gl, and the
// group's last lane also loads the chunk B + count, which holds the metadata
// at byte s (the metadata is never wider than the row alignment, so it does
// not cross into the next chunk).  Every global load is an aligned 16-byte
// load: loads straddling 16-byte boundaries are split by the memory pipeline,
// and at 4- or 8-byte widths a 264-byte row needs twice the load instructions
// plus a metadata load per lane.
//
// The lane's 16 values, row bytes [16*gl, 16*gl + 16), are bytes [s, 16) of
// its own chunk followed by bytes [0, s) of the next lane's, moved with one
// DPP row shift per word (the last lane takes the metadata chunk instead).
// The realigned rows then go through LDS so that every store instruction
// writes one contiguous run: lane gl takes values V*(G*j + gl) .. + V - 1 for
// its store j (V = 4 for fp32 output, 8 for fp16), G*16 contiguous output
// bytes per group and instruction.  (Writing the raw chunks to LDS and reading
// them back from byte s, without the DPP shift, measured slower: C4a 17.3 ->
// 18.9 us; its row images are 16 bytes longer, which costs LDS conflicts.)
//
// The chunks read up to 15 bytes before the row and after its metadata; they
// lie in the same 16-byte-aligned blocks as bytes of the row, hence in the
// same memory page.
// ---------------------------------------------------------------------------

// Word k of x shifted down by (s & 12) bytes: two rounds of bitwise selects on
// the bits of s / 4.  Masks rather than `c ? x[k + 2] : x[k]`, which the
// compiler turns into a dynamically indexed array (kept in LDS), and no branch
// depends on s (it differs between the rows of a wave).
__device__ __forceinline__ uint32_t pick(uint32_t a, uint32_t b, uint32_t take_b) {
  return a ^ ((a ^ b) & take_b);
}
template <int N>
__device__ __forceinline__ void shift_words(const uint32_t (&x)[N], uint32_t s,
                                            uint32_t (&y)[N - 3]) {
  const uint32_t m8 = 0u - ((s >> 3) & 1u);
  const uint32_t m4 = 0u - ((s >> 2) & 1u);
  uint32_t t[N - 2];
#pragma unroll
  for (int k = 0; k < N - 2; ++k) t[k] = pick(x[k], x[k + 2], m8);
#pragma unroll
  for (int k = 0; k < N - 3; ++k) y[k] = pick(t[k], t[k + 1], m4);
}

// bytes [s, s + 16) of the 32-byte concatenation lo ++ hi, s in [0, 16)
__device__ __forceinline__ Vec<16> realign16(const u32x4& lo, const u32x4& hi, uint32_t s) {
  const uint32_t x[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
  uint32_t y[5];
  shift_words<8>(x, s, y);
  Vec<16> v;
#pragma unroll
  for (int j = 0; j < 4; ++j) v.w[j] = __builtin_amdgcn_alignbyte(y[j + 1], y[j], s & 3u);
  return v;
}

// The row's scale (and offset) from its metadata chunk, which holds them at
// byte s (s + metadata bytes <= 16).
template <int SDT>
__device__ __forceinline__ Meta meta_at(const u32x4& c, uint32_t s) {
  const uint32_t x[6] = {c.x, c.y, c.z, c.w, 0u, 0u};
  uint32_t y[3];
  shift_words<6>(x, s, y);
  const uint32_t m0 = __builtin_amdgcn_alignbyte(y[1], y[0], s & 3u);
  Meta m{1.0f, 0.0f};
  if constexpr (SDT == kQU8F32 || SDT == kXI8AF32) {
    m.s = __uint_as_float(m0);
    m.o = __uint_as_float(__builtin_amdgcn_alignbyte(y[2], y[1], s & 3u));
  } else if constexpr (SDT == kQI8F32 || SDT == kXE4M3F32) {
    m.s = __uint_as_float(m0);
  } else if constexpr (SDT == kQU8F16) {
    m.s = h2f((uint16_t)(m0 & 0xffffu));
    m.o = h2f((uint16_t)(m0 >> 16));
  } else {
    static_assert(SDT == kQI8F16, "one-byte quantized formats only");
    m.s = h2f((uint16_t)(m0 & 0xffffu));
  }
  return m;
}

// U rows per lane group: G = 16 for U = 16, G = 8 for U = 8, G <= 4 for U = 4.
template <int SDT, int U, bool OUT_F16>
__global__ __launch_bounds__(256) void gather_realign_kernel(GatherLaunch a, int g_shift,
                                                             int t_shift) {
  const int T = 1 << t_shift;
  const int lane = threadIdx.x & 63;
  const int64_t tile = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int64_t base = tile << t_shift;
  uint32_t orow;
  const uint64_t addr = resolve_tile(a, base, T, lane, &orow);

  const int G = 1 << g_shift;  // count / 16, at most 16: a group never spans two DPP rows
  const int gl = lane & (G - 1);
  const int grp = lane >> g_shift;
  const int groups = 64 >> g_shift;
  const int per_group = T >> (6 - g_shift);  // keys per group, <= U
  const uint64_t area = (uint64_t)a.count;
  constexpr int out_es = OUT_F16 ? 2 : 4;
  const uint64_t zero_row = (uint64_t)g_zero_row;
  const bool last = gl == G - 1;
  uint8_t* out = reinterpret_cast<uint8_t*>(a.out);

  uint64_t ra[U];
  uint32_t orw[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int j = grp + (u < per_group ? u : 0) * groups;
    ra[u] = shfl64(addr, j);
    orw[u] = a.out_index != nullptr ? shfl32(orow, j) : 0u;
    if (u >= per_group) ra[u] = 0;
  }
  u32x4 c[U];
  u32x4 mc[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint64_t b = (ra[u] != 0 ? ra[u] : zero_row) & ~(uint64_t)15;
    c[u] = gload<u32x4>(b + 16u * (uint32_t)gl);
    mc[u] = u32x4{0u, 0u, 0u, 0u};
    if (last) mc[u] = gload<u32x4>(b + area);
  }

  // One 1 KiB LDS slot per wave and row (64 lanes x 16 bytes), and the scale
  // and offset of the wave's T <= 64 rows (row u of group grp is key
  // u * groups + grp of the wave), written by each group's last lane.
  __shared__ u32x4 stage[4][U][64];
  __shared__ Meta stage_meta[4][64];
  u32x4(&slots)[U][64] = stage[threadIdx.x >> 6];
  Meta(&metas)[64] = stage_meta[threadIdx.x >> 6];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    // The next lane's chunk; the last lane of a 16-lane group has no next
    // lane in its DPP row and takes the metadata chunk from the move itself,
    // that of a narrower group takes it by a select.
    uint32_t w[4] = {c[u].x, c[u].y, c[u].z, c[u].w};
    const uint32_t mw[4] = {mc[u].x, mc[u].y, mc[u].z, mc[u].w};
    row_next_pin(w, mw);
    u32x4 nx;
    nx.x = last ? mw[0] : w[0];
    nx.y = last ? mw[1] : w[1];
    nx.z = last ? mw[2] : w[2];
    nx.w = last ? mw[3] : w[3];
    const uint32_t s = (uint32_t)ra[u] & 15u;
    const Vec<16> v = realign16(c[u], nx, s);
    u32x4 q;
    q.x = v.w[0];
    q.y = v.w[1];
    q.z = v.w[2];
    q.w = v.w[3];
    slots[u][lane] = q;
    if (last && u < per_group) metas[u * groups + grp] = meta_at<SDT>(mc[u], s);
  }
  // lanes read what other lanes of the wave wrote: LDS keeps a wave's
  // accesses in order; the fences keep the compiler from moving them
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  constexpr int V = OUT_F16 ? 8 : 4;  // values per 16-byte store
  constexpr int NS = 16 / V;          // stores per lane and row
#pragma unroll
  for (int u = 0; u < U; ++u) {
    // decoded for every row (absent ones read zeros), stored for real ones
    const uint8_t* row_bytes = reinterpret_cast<const uint8_t*>(&slots[u][grp * G]);
    const int64_t row = a.out_index != nullptr ? (int64_t)orw[u] : base + grp + (int64_t)u * groups;
    uint8_t* o = out + row * a.out_stride;
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      const int off = V * (G * j + gl);  // value index = byte offset in the row
      Vec<V> v;
      if constexpr (V == 8) {
        const u32x2 t = *reinterpret_cast<const u32x2*>(row_bytes + off);
        v.w[0] = t.x;
        v.w[1] = t.y;
      } else {
        v.w[0] = *reinterpret_cast<const uint32_t*>(row_bytes + off);
      }
      float x[V];
      decode<SDT, V>(v, metas[(u * groups + grp) & 63], x);
      if (ra[u] != 0) store_out<V, OUT_F16>(o + off * out_es, x, OUT_F16);
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

// Largest power of two <= 16 that every row address is a multiple of.
int row_alignment(const RowSource& src) {
  int al = 16;
  while (al > 1 && (src.row_bytes % (uint64_t)al || (src.table && !aligned(src.table, al)) ||
                    (src.cache_data && !aligned(src.cache_data, al))))
    al >>= 1;
  return al;
}

// gather_realign_kernel takes one-byte formats with 16..256 values (a power of
// two times 16, so a row is at most 16 lanes: one DPP row), metadata no wider
// than the row alignment, and 16-byte aligned output rows.
bool realign_eligible(const GatherLaunch& a) {
  if (a.raw || value_elem_bytes(a.stored_dtype) != 1) return false;
  const int64_t g = a.count / 16;
  if (a.count % 16 || g < 1 || g > 16 || (g & (g - 1))) return false;
  if (meta_bytes(a.stored_dtype) > row_alignment(a.src)) return false;
  return aligned(a.out, 16) && a.out_stride % 16 == 0;
}

hipError_t launch_gather_realign(const GatherLaunch& a, hipStream_t stream) {
  const int g = (int)(a.count / 16);
  const int gs = log2i(g);
  const int groups = 64 / g;
  // one batch of U rows per group; a wave resolves groups * U keys (<= 64)
  const int unroll = g >= 16 ? 16 : g >= 8 ? 8 : 4;
  const int tkeys = groups * unroll < 64 ? groups * unroll : 64;
  const int ts = log2i(tkeys);
  const int64_t waves = (a.n + tkeys - 1) / tkeys;
  const int threads = 256;
  const int64_t grid = (waves * 64 + threads - 1) / threads;
  if (grid > 0x7fffffffLL) return hipErrorInvalidValue;
#define L_RA_U(S, U, O) \
  hipLaunchKernelGGL((gather_realign_kernel<S, U, O>), dim3(grid), dim3(threads), 0, stream, a, gs, ts)
#define L_RA_O(S, O)           \
  do {                         \
    if (unroll == 16)          \
      L_RA_U(S, 16, O);        \
    else if (unroll == 8)      \
      L_RA_U(S, 8, O);         \
    else                       \
      L_RA_U(S, 4, O);         \
  } while (0)
#define L_RA(S)                                                                                \
  do {                                                                                         \
    if (a.out_dtype == kF16)                                                                   \
      L_RA_O(S, true);                                                                         \
    else                                                                                       \
      L_RA_O(S, false);                                                                        \
  } while (0)
  switch (a.stored_dtype) {
    case kQI8F32: L_RA(kQI8F32); break;
    case kQI8F16: L_RA(kQI8F16); break;
    case kQU8F32: L_RA(kQU8F32); break;
    case kQU8F16: L_RA(kQU8F16); break;
    case kXI8AF32: L_RA(kXI8AF32); break;
    case kXE4M3F32: L_RA(kXE4M3F32); break;
    default: return hipErrorInvalidValue;
  }
#undef L_RA
#undef L_RA_O
#undef L_RA_U
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gather(const GatherLaunch& a, hipStream_t stream) {
  if (a.n <= 0) return hipSuccess;
  if (realign_eligible(a)) return launch_gather_realign(a, stream);
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
