// pool_kernel.cuh -- the fused find-and-pool kernel template, instantiated
// per stored type in pool_float.hip, pool_quant.hip and pool_ext.hip (the
// instantiations are many; separate translation units build in parallel).
//
// Reference behaviour restated: find_and_combine (cuda_ops/find_and_combine_kernel.cuh:40-154).
//
// Design (MI355X-first, not the reference's warp32 shape):
//  * A "group" of G lanes (G a power of two <= 64) owns one row at a time; lane
//    l of the group moves bytes [l*VB, l*VB+VB) of the row with one VB-byte
//    load, so a 256-byte fp16 row is one dwordx4 load per lane over 16 lanes.
//  * Keys are resolved one per lane (the cache's 8-tag compare included), then
//    row addresses are broadcast inside the group with ds_bpermute; the U row
//    loads of a batch are all issued before any is consumed.
//  * One fp32 accumulator per element in registers.  Short bags are reduced by
//    one group in key order -- the reference's per-element order.  Few long
//    bags are split over up to 64 groups of one workgroup in contiguous key
//    chunks, combined by a fixed binary tree (deterministic, within fp32
//    tolerance of key order).
//  * Weighted pooling is a template parameter: a runtime flag kept both paths
//    live in the batch loop and cost about a fifth of the kernel's time.
#pragma once

#include "device_common.cuh"
#include "launch.hpp"

namespace nve_amd {

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

template <int SDT, int VB, int U, bool W>
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
  if (a.num_tables > 0 && live) {
    src.table = a.tables[bag / a.bags_per_table];
    src.num_rows = a.table_rows[bag / a.bags_per_table];
  }
  int64_t cs = s, ce = e;
  if (gpb > 1 && e > s) {
    const int64_t per = (e - s + gpb - 1) >> gpb_shift;
    cs = s + chunk * per;
    if (cs > e) cs = e;
    ce = cs + per < e ? cs + per : e;
  }

  constexpr bool weighted = W;  // a.weighted, fixed at compile time
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

}  // namespace nve_amd

namespace nve_amd {

inline int pool_log2(int x) {
  int r = 0;
  while ((1 << r) < x) ++r;
  return r;
}

// Launches pool_kernel<S, V, U, W> for the geometry's unroll and the launch's
// weighting.  Row formats with per-row metadata (scale / offset) keep fewer
// rows in flight (8, or 4 when a lane decodes 16 elements): the kernel is
// built for 1024-thread workgroups, 128 registers per lane, and with more
// rows their decode state would go to scratch memory.
template <int S, int V>
hipError_t launch_pool_sv(const PoolLaunch& a, const PoolGeometry& g, hipStream_t stream) {
  const int gs = pool_log2(g.g);
  const int ps = pool_log2(g.gpb);
  const dim3 grid((unsigned)g.grid), block((unsigned)g.threads);
  if constexpr (Fmt<S>::meta != 0) {
    constexpr int kU = V / Fmt<S>::esize >= 16 ? 4 : 8;
    if (a.weighted)
      hipLaunchKernelGGL((pool_kernel<S, V, kU, true>), grid, block, g.lds_bytes, stream, a, gs, ps, g.passes);
    else
      hipLaunchKernelGGL((pool_kernel<S, V, kU, false>), grid, block, g.lds_bytes, stream, a, gs, ps, g.passes);
  } else if (g.unroll == 16) {
    if (a.weighted)
      hipLaunchKernelGGL((pool_kernel<S, V, 16, true>), grid, block, g.lds_bytes, stream, a, gs, ps, g.passes);
    else
      hipLaunchKernelGGL((pool_kernel<S, V, 16, false>), grid, block, g.lds_bytes, stream, a, gs, ps, g.passes);
  } else {
    if (a.weighted)
      hipLaunchKernelGGL((pool_kernel<S, V, 8, true>), grid, block, g.lds_bytes, stream, a, gs, ps, g.passes);
    else
      hipLaunchKernelGGL((pool_kernel<S, V, 8, false>), grid, block, g.lds_bytes, stream, a, gs, ps, g.passes);
  }
  return hipGetLastError();
}

// row-slice widths a stored type of 1-byte elements can use
template <int S>
hipError_t launch_pool_bytes(const PoolLaunch& a, const PoolGeometry& g, hipStream_t stream) {
  switch (g.vb) {
    case 16: return launch_pool_sv<S, 16>(a, g, stream);
    case 8: return launch_pool_sv<S, 8>(a, g, stream);
    case 4: return launch_pool_sv<S, 4>(a, g, stream);
    case 2: return launch_pool_sv<S, 2>(a, g, stream);
    case 1: return launch_pool_sv<S, 1>(a, g, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace nve_amd
