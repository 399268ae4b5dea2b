// device_common.cuh -- device helpers shared by the lookup kernels (gfx950, wave64).
//
// Row formats follow the reference's stored layouts (nve_types.hpp:143-189,
// kernels_common.cuh:67-172): a row is `count` values followed by the per-row
// quantization metadata (scale, then offset when the type has one).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../dtypes.hpp"
#include "launch.hpp"

namespace nve_amd {

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// wave primitives
// ---------------------------------------------------------------------------
__device__ __forceinline__ int lane_id() { return __lane_id(); }

// Read `v` from lane `src` of the wave (ds_bpermute; every lane of the source
// group must be active, which the callers guarantee by keeping the branches
// around a shuffle uniform over a lane group).
__device__ __forceinline__ uint32_t shfl32(uint32_t v, int src) {
  return (uint32_t)__builtin_amdgcn_ds_bpermute(src << 2, (int)v);
}
__device__ __forceinline__ uint64_t shfl64(uint64_t v, int src) {
  const uint32_t lo = shfl32((uint32_t)v, src);
  const uint32_t hi = shfl32((uint32_t)(v >> 32), src);
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ float shflf(float v, int src) {
  return __uint_as_float(shfl32(__float_as_uint(v), src));
}

// ---------------------------------------------------------------------------
// scalar conversions
// ---------------------------------------------------------------------------
__device__ __forceinline__ float h2f(uint16_t h) {
  _Float16 x;
  __builtin_memcpy(&x, &h, 2);
  return (float)x;
}
// binary32 -> binary16, round to nearest even (v_cvt_f16_f32 in the default mode).
// The empty asm keeps the binary32 value as it is: without it the compiler may
// fold a conversion of an fma or product into one v_fma_mixlo_f16, which
// rounds once to binary16 where the formulas round to binary32 first.
__device__ __forceinline__ uint16_t f2h(float f) {
  asm("" : "+v"(f));
  _Float16 x = (_Float16)f;
  uint16_t h;
  __builtin_memcpy(&h, &x, 2);
  return h;
}
// acc + float(h) (lo: the low half of w, hi: the high half) and
// fma(float(h), wt, acc) as one v_fma_mix_f32 each: the half is widened inside
// the instruction (exactly) and the result rounded once to binary32, so the
// bits are those of the widen-then-add / widen-then-fma pair it replaces
// (h * 1.0 is exact).  One VALU instruction per element instead of two.
__device__ __forceinline__ float acc_half_lo(float acc, uint32_t w) {
  float r;
  asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(w), "v"(acc));
  return r;
}
__device__ __forceinline__ float acc_half_hi(float acc, uint32_t w) {
  float r;
  asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(w), "v"(acc));
  return r;
}
__device__ __forceinline__ float fma_half_lo(uint32_t w, float wt, float acc) {
  float r;
  asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(w), "v"(wt), "v"(acc));
  return r;
}
__device__ __forceinline__ float fma_half_hi(uint32_t w, float wt, float acc) {
  float r;
  asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(w), "v"(wt), "v"(acc));
  return r;
}

// OCP FP8 E4M3FN (bias 7, no infinities, NaN = S.1111.111), decoded exactly
// and without branches: a normal code E.M becomes exponent E + 120, mantissa
// M << 20, i.e. (code << 20) + (120 << 23); a subnormal code (E = 0) is
// M * 2^-9, exact in binary32; S.1111.111 is the quiet NaN with the code's sign.
__device__ __forceinline__ float e4m3_to_f32(uint32_t v) {
  const uint32_t a = v & 0x7fu;
  const uint32_t sub = __float_as_uint((float)a * 0.001953125f);
  uint32_t bits = a < 8u ? sub : (a << 20) + (120u << 23);
  bits = a == 0x7fu ? 0x7fc00000u : bits;
  return __uint_as_float(((v & 0x80u) << 24) | bits);
}

// The four E4M3 codes of w (byte k = value k) through gfx950's packed
// conversion, two codes per instruction.  It gives e4m3_to_f32's bits for
// every code except 0.1111.111, the positive NaN, which it returns with the
// sign bit set; putting each code's own sign bit back (one bitfield insert per
// value) makes all 256 codes agree.
__device__ __forceinline__ void e4m3x4_to_f32(uint32_t w, float (&x)[4]) {
  const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);  // bytes 0 and 1
  const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);   // bytes 2 and 3
  const uint32_t r[4] = {__float_as_uint(lo[0]), __float_as_uint(lo[1]), __float_as_uint(hi[0]),
                         __float_as_uint(hi[1])};
  const uint32_t sign[4] = {w << 24, w << 16, w << 8, w};  // byte k's top bit at bit 31
#pragma unroll
  for (int k = 0; k < 4; ++k) x[k] = __uint_as_float((r[k] & 0x7fffffffu) | (sign[k] & 0x80000000u));
}

// ---------------------------------------------------------------------------
// vector loads / stores of VB bytes (VB in {1,2,4,8,16}, address VB-aligned)
//
// Row addresses are computed integers, so the accesses go through pointers in
// the global address space: they become global_load / global_store, which
// count only against vmcnt.  (Generic pointers would give flat accesses that
// also count against lgkmcnt, so every wait for a lane shuffle would drain the
// row loads in flight as well.)
// ---------------------------------------------------------------------------
template <typename T>
using gptr = const __attribute__((address_space(1))) T*;
template <typename T>
using gptr_w = __attribute__((address_space(1))) T*;

template <typename T>
__device__ __forceinline__ T gload(uint64_t addr) {
  return *reinterpret_cast<gptr<T>>(addr);
}
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// VB bytes as 32-bit words (the low bytes of w[0] for VB < 4); element e of
// an ES-byte type is bits [8*ES*(e % (4/ES)), ...) of word e / (4/ES).
template <int VB>
struct Vec {
  uint32_t w[VB >= 4 ? VB / 4 : 1];
};

template <int VB>
__device__ __forceinline__ Vec<VB> load_vec(uint64_t addr) {
  Vec<VB> v;
  if constexpr (VB == 16) {
    const u32x4 x = gload<u32x4>(addr);
    v.w[0] = x.x;
    v.w[1] = x.y;
    v.w[2] = x.z;
    v.w[3] = x.w;
  } else if constexpr (VB == 8) {
    const u32x2 x = gload<u32x2>(addr);
    v.w[0] = x.x;
    v.w[1] = x.y;
  } else if constexpr (VB == 4) {
    v.w[0] = gload<uint32_t>(addr);
  } else if constexpr (VB == 2) {
    v.w[0] = gload<uint16_t>(addr);
  } else {
    v.w[0] = gload<uint8_t>(addr);
  }
  return v;
}
template <int VB>
__device__ __forceinline__ Vec<VB> load_vec(const uint8_t* p) {
  return load_vec<VB>((uint64_t)p);
}

__device__ __forceinline__ uint32_t vbyte(const uint32_t* w, int e) {
  return (w[e >> 2] >> ((e & 3) * 8)) & 0xffu;
}
__device__ __forceinline__ uint16_t vhalf(const uint32_t* w, int e) {
  return (uint16_t)(w[e >> 1] >> ((e & 1) * 16));
}

// NT: streaming (nontemporal) store, the output being written once and not
// re-read by the lookup; otherwise an ordinary store.  Measured per kernel:
// the dequantizing gather's 1 KiB fp32 rows write faster as ordinary stores
// (C4b 32.2 -> 28.7 us), the pooled and plain gathers slightly faster as
// streaming stores.
template <int VB, bool NT = true>
__device__ __forceinline__ void store_vec(uint8_t* p, const Vec<VB>& v) {
  const uint64_t a = (uint64_t)p;
  if constexpr (VB >= 4) {
#pragma unroll
    for (int i = 0; i < VB / 4; ++i) {
      if constexpr (NT)
        __builtin_nontemporal_store(v.w[i], reinterpret_cast<gptr_w<uint32_t>>(a) + i);
      else
        reinterpret_cast<gptr_w<uint32_t>>(a)[i] = v.w[i];
    }
  } else if constexpr (VB == 2) {
    *reinterpret_cast<gptr_w<uint16_t>>(a) = (uint16_t)v.w[0];
  } else {
    *reinterpret_cast<gptr_w<uint8_t>>(a) = (uint8_t)v.w[0];
  }
}

// Store E floats (as f32 or RNE f16) at p, which is aligned to E*element bytes.
template <int E, bool NT = true>
__device__ __forceinline__ void store_out(uint8_t* p, const float* v, bool out_f16) {
  if (out_f16) {
    Vec<2 * E> o;
    if constexpr (E == 1) {
      o.w[0] = f2h(v[0]);
    } else {
#pragma unroll
      for (int i = 0; i < E / 2; ++i)
        o.w[i] = (uint32_t)f2h(v[2 * i]) | ((uint32_t)f2h(v[2 * i + 1]) << 16);
    }
    store_vec<2 * E, NT>(p, o);
  } else {
    if constexpr (E <= 4) {
      Vec<4 * E> o;
#pragma unroll
      for (int i = 0; i < E; ++i) o.w[i] = __float_as_uint(v[i]);
      store_vec<4 * E, NT>(p, o);
    } else {
      // Several 16-byte pieces per lane: each store instruction covers only
      // part of every line it touches.  Streaming stores send those partial
      // lines to HBM one by one (the multi-table pool wrote 131,693 KiB for
      // 106,496 KiB of fp32 output), ordinary stores merge them in L2 first
      // (exactly 106,496 KiB, same time), so these always go through L2.
#pragma unroll
      for (int c = 0; c < E / 4; ++c) {
        Vec<16> o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o.w[i] = __float_as_uint(v[4 * c + i]);
        store_vec<16, false>(p + 16 * c, o);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// per-row dequantization: decode the E values of a VB-byte slice of the row's
// value area into fp32.  Metadata (scale, offset) is read per row.
// ---------------------------------------------------------------------------
template <int SDT>
struct Fmt;

template <>
struct Fmt<kF32> {
  static constexpr int esize = 4;
  static constexpr int meta = 0;
};
template <>
struct Fmt<kF16> {
  static constexpr int esize = 2;
  static constexpr int meta = 0;
};
template <>
struct Fmt<kQI8F32> {
  static constexpr int esize = 1;
  static constexpr int meta = 4;
};
template <>
struct Fmt<kQI8F16> {
  static constexpr int esize = 1;
  static constexpr int meta = 2;
};
template <>
struct Fmt<kQU8F32> {
  static constexpr int esize = 1;
  static constexpr int meta = 8;
};
template <>
struct Fmt<kQU8F16> {
  static constexpr int esize = 1;
  static constexpr int meta = 4;
};
template <>
struct Fmt<kXI8AF32> {
  static constexpr int esize = 1;
  static constexpr int meta = 8;
};
template <>
struct Fmt<kXE4M3F32> {
  static constexpr int esize = 1;
  static constexpr int meta = 4;
};

struct Meta {
  float s;
  float o;
};

// Metadata sits right after the value area; its address is only 2-byte
// aligned in general, so it is assembled from 16-bit loads.
__device__ __forceinline__ float ld_f32_unaligned(const uint8_t* p) {
  const uint64_t a = (uint64_t)p;
  const uint32_t v = (uint32_t)gload<uint16_t>(a) | ((uint32_t)gload<uint16_t>(a + 2) << 16);
  return __uint_as_float(v);
}

// MW: the metadata is aligned to its own size (4 or 8 bytes) in every row, so
// it comes with one load; otherwise it is assembled from 16-bit loads.
template <int SDT, bool MW = false>
__device__ __forceinline__ Meta load_meta(uint64_t row, int64_t value_bytes) {
  Meta m{1.0f, 0.0f};
  const uint64_t p = row + (uint64_t)value_bytes;
  if constexpr (MW && (SDT == kQU8F32 || SDT == kXI8AF32)) {
    const u32x2 x = gload<u32x2>(p);
    m.s = __uint_as_float(x.x);
    m.o = __uint_as_float(x.y);
  } else if constexpr (MW && (SDT == kQI8F32 || SDT == kXE4M3F32)) {
    m.s = __uint_as_float(gload<uint32_t>(p));
  } else if constexpr (MW && SDT == kQU8F16) {
    const uint32_t x = gload<uint32_t>(p);
    m.s = h2f((uint16_t)(x & 0xffffu));
    m.o = h2f((uint16_t)(x >> 16));
  } else if constexpr (SDT == kQI8F32 || SDT == kXE4M3F32) {
    m.s = ld_f32_unaligned(reinterpret_cast<const uint8_t*>(p));
  } else if constexpr (SDT == kQU8F32 || SDT == kXI8AF32) {
    m.s = ld_f32_unaligned(reinterpret_cast<const uint8_t*>(p));
    m.o = ld_f32_unaligned(reinterpret_cast<const uint8_t*>(p + 4));
  } else if constexpr (SDT == kQI8F16) {
    m.s = h2f(gload<uint16_t>(p));
  } else if constexpr (SDT == kQU8F16) {
    m.s = h2f(gload<uint16_t>(p));
    m.o = h2f(gload<uint16_t>(p + 2));
  }
  return m;
}
template <int SDT>
__device__ __forceinline__ Meta load_meta(const uint8_t* row, int64_t value_bytes) {
  return load_meta<SDT, false>((uint64_t)row, value_bytes);
}

// Decoded element formulas (kernels_common.cuh:174-297):
//   F32/F16    the stored value
//   QI8 F32    fma(q, s, 0)               (float(q)*scale + 0, contracted)
//   QU8 F32    fma(q, s, o)
//   QI8 F16    half(float(q) * s)          rounded to half once, then widened
//   QU8 F16    half(fma(q, s, o))
//   XI8A F32   fma(q, s, o)                (extension: int8 affine)
//   XE4M3 F32  e4m3(q) * s                 (extension: OCP fp8 with scale)
template <int SDT, int VB>
__device__ __forceinline__ void decode(const Vec<VB>& v, const Meta& m,
                                       float (&x)[VB / Fmt<SDT>::esize]) {
  constexpr int E = VB / Fmt<SDT>::esize;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    if constexpr (SDT == kF32) {
      x[e] = __uint_as_float(v.w[e]);
    } else if constexpr (SDT == kF16) {
      x[e] = h2f(vhalf(v.w, e));
    } else if constexpr (SDT == kQI8F32) {
      x[e] = __builtin_fmaf((float)(int8_t)vbyte(v.w, e), m.s, 0.0f);
    } else if constexpr (SDT == kQU8F32 || SDT == kXI8AF32) {
      const float q = (SDT == kQU8F32) ? (float)vbyte(v.w, e) : (float)(int8_t)vbyte(v.w, e);
      x[e] = __builtin_fmaf(q, m.s, m.o);
    } else if constexpr (SDT == kQI8F16) {
      x[e] = h2f(f2h((float)(int8_t)vbyte(v.w, e) * m.s));
    } else if constexpr (SDT == kQU8F16) {
      x[e] = h2f(f2h(__builtin_fmaf((float)vbyte(v.w, e), m.s, m.o)));
    } else if constexpr (SDT == kXE4M3F32) {
      if constexpr (VB >= 4) {
        if (e % 4 == 0) {
          float q[4];
          e4m3x4_to_f32(v.w[e / 4], q);
#pragma unroll
          for (int k = 0; k < 4; ++k) x[e + k] = q[k] * m.s;
        }
      } else {
        x[e] = e4m3_to_f32((uint8_t)vbyte(v.w, e)) * m.s;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// shared pieces of the lookup kernels
// ---------------------------------------------------------------------------
// Readable zeros for keys that resolve to no row: their loads are pointed
// here (offsets folded into the buffer) so that every load of a batch can be
// issued unconditionally.  One copy per translation unit.
constexpr int kZeroRowBytes = 4096;
constexpr int64_t kZeroRowMask = kZeroRowBytes - 1;
static __device__ __align__(16) uint8_t g_zero_row[kZeroRowBytes + 64] = {};

// Miss counters are kMissStripes words, each at the start of its own 128-byte
// line (kMissStripeWords apart); a workgroup adds to stripe
// blockIdx.x % kMissStripes and readers add the words up: same-address (and
// same-line) atomics serialize at the memory side, thousands of them per
// launch when every wave adds its misses.
constexpr int kMissStripes = 8;
constexpr int kMissStripeWords = 16;

// Adds the wave's per-lane miss counts to the workgroup's counter word (every
// lane active).
__device__ __forceinline__ void add_misses(unsigned long long* counter, uint32_t n) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) n += __shfl_xor(n, o);
  if (__lane_id() == 0 && n)
    atomicAdd(counter + (blockIdx.x & (kMissStripes - 1)) * kMissStripeWords, (unsigned long long)n);
}

// ---------------------------------------------------------------------------
// key / row resolution
// ---------------------------------------------------------------------------
__device__ __forceinline__ int64_t load_key(const void* keys, int key_bytes, int64_t i) {
  return key_bytes == 4 ? (int64_t) reinterpret_cast<const int32_t*>(keys)[i]
                        : reinterpret_cast<const int64_t*>(keys)[i];
}

// per-key pooling weight (f32 or f16), indexed by the key's global position
__device__ __forceinline__ float load_weight(const void* w, int wdt, int64_t k) {
  return wdt == kF16 ? h2f(reinterpret_cast<const uint16_t*>(w)[k])
                     : reinterpret_cast<const float*>(w)[k];
}

__device__ __forceinline__ void store_key(void* keys, int key_bytes, int64_t i, int64_t v) {
  if (key_bytes == 4)
    reinterpret_cast<int32_t*>(keys)[i] = (int32_t)v;
  else
    reinterpret_cast<int64_t*>(keys)[i] = v;
}

// Order-preserving map of a signed key to an unsigned radix-sort key (the
// sign bit flipped), and back.
__device__ __forceinline__ uint64_t flip_key(int64_t k, int key_bytes) {
  if (key_bytes == 4) return (uint64_t)((uint32_t)(int32_t)k ^ 0x80000000u);
  return (uint64_t)k ^ 0x8000000000000000ull;
}
__device__ __forceinline__ int64_t unflip_key(uint64_t f, int key_bytes) {
  if (key_bytes == 4) return (int64_t)(int32_t)((uint32_t)f ^ 0x80000000u);
  return (int64_t)(f ^ 0x8000000000000000ull);
}

// Where rows come from (RowSource, launch.hpp).  Without a cache: row =
// table + index*row_bytes, index being the key (load_indices) or the key's
// position (a buffer gathered earlier).  With a cache (EmbedCacheSA layout,
// ec_set_associative.h:104-112, ec_set_associative.cuh:46-80): 8 tags per set
// at tags + set*8, rows at data + (set*8 + way)*row_bytes;
// set = (unsigned)key % num_sets; a hit is the lowest way whose rebuilt key
// tag*num_sets + set equals the key; a miss resolves to table + key*row_bytes,
// or to nothing when table is null.
// Returns the row address (0 when unresolved); *hit reports a cache hit or a
// linear-table row; *miss a cache miss (whether or not a backing row exists).
__device__ __forceinline__ uint64_t resolve_row(const RowSource& src, int key_bytes, int64_t key,
                                                int64_t pos, bool* miss) {
  *miss = false;
  if (src.cache_data == nullptr) {
    const uint64_t idx = src.load_indices ? (uint64_t)key : (uint64_t)pos;
    if (src.num_rows != 0 && idx >= src.num_rows) return 0;
    return (uint64_t)src.table + idx * src.row_bytes;
  }
  uint32_t set;
  uint32_t mask = 0;
  if (key_bytes == 4) {
    const uint32_t uk = (uint32_t)(int32_t)key;
    const uint32_t ns = (uint32_t)src.num_sets;
    set = uk % ns;
    const uint4* tp = reinterpret_cast<const uint4*>(
        reinterpret_cast<const int32_t*>(src.cache_tags) + (uint64_t)set * 8);
    const uint4 t0 = tp[0];
    const uint4 t1 = tp[1];
    const uint32_t t[8] = {t0.x, t0.y, t0.z, t0.w, t1.x, t1.y, t1.z, t1.w};
#pragma unroll
    for (int w = 0; w < 8; ++w) mask |= (uint32_t)(t[w] * ns + set == uk) << w;
  } else {
    const uint64_t uk = (uint64_t)key;
    set = (uint32_t)(uk % src.num_sets);
    const uint4* tp = reinterpret_cast<const uint4*>(
        reinterpret_cast<const int64_t*>(src.cache_tags) + (uint64_t)set * 8);
    uint64_t t[8];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint4 q = tp[c];
      t[2 * c] = (uint64_t)q.x | ((uint64_t)q.y << 32);
      t[2 * c + 1] = (uint64_t)q.z | ((uint64_t)q.w << 32);
    }
#pragma unroll
    for (int w = 0; w < 8; ++w) mask |= (uint32_t)(t[w] * src.num_sets + set == uk) << w;
  }
  if (mask) {
    const uint32_t way = (uint32_t)__builtin_ctz(mask);
    return (uint64_t)src.cache_data + ((uint64_t)set * 8 + way) * src.row_bytes;
  }
  *miss = true;
  // the backing row; none for a table without one, or a key outside it
  if (src.table == nullptr || (src.num_rows != 0 && (uint64_t)key >= src.num_rows)) return 0;
  return (uint64_t)src.table + (uint64_t)key * src.row_bytes;
}

}  // namespace nve_amd
