// backprop.hip -- kernels of the training backprop (the sparse gradient of a
// lookup): bag denominators, the gradient row and weight of every key
// position in dedup order, and the two summation kernels.
//
// Summation order (fixed, and the CPU oracle's): the dedup order of the
// positions is cut into blocks of kPieceBlock; a piece is one key's positions
// inside one block, added in fp32 in position order from 0 (acc + g, or
// fmaf(g, w, acc) for the weighted modes).  piece_pool_kernel walks one block
// per lane group: a key whose positions all lie in the block is finished there
// (rounded once to the gradient type); a piece of a key that crosses a block
// edge goes to one of the block's two fp32 slots (slot 2b: the piece holding
// the block's first position, 2b + 1: the piece holding its last), and each
// crossing key is recorded as its first block's entry.  piece_combine_kernel
// then finishes those keys: a key's J pieces in kPieceFanIn consecutive sub-sequences of
// ceil(J / kPieceFanIn), each added in order from 0 (one wave each), the
// sub-sequence sums added in order from 0, rounded once.
//
// Reference behaviour restated: GradientCalculator::compute_gradients
// (cuda_ops/gradient_calculator.cuh:238-301): compute_normalized_weights
// (:29-63), compute_pooling_inverse_mapping (:65-82), compute_pooling_gradients
// (:84-135); GradientDedup (cuda_ops/dedup_grads_kernel.cuh:57-107).
#include "backprop_launch.hpp"
#include "device_common.cuh"
#include "lane_moves.cuh"
#include "position_grad.cuh"

namespace nve_amd {

namespace {

// [s, e) of bag b (Fixed: b*hotness; CSR: the caller's offsets)
__device__ __forceinline__ void bag_range(const void* offsets, int key_bytes, int64_t hotness,
                                          int64_t b, int64_t* s, int64_t* e) {
  if (offsets == nullptr) {
    *s = b * hotness;
    *e = *s + hotness;
  } else {
    *s = load_key(offsets, key_bytes, b);
    *e = load_key(offsets, key_bytes, b + 1);
  }
}

// Mean: the bag's key count; WeightedMean: its weights added in position order.
__global__ __launch_bounds__(256) void bag_denom_kernel(const void* offsets, int key_bytes,
                                                        int64_t num_bags, int64_t hotness,
                                                        const void* weights, int wdt, int wmean,
                                                        float* denom) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= num_bags) return;
  int64_t s, e;
  bag_range(offsets, key_bytes, hotness, b, &s, &e);
  if (!wmean) {
    denom[b] = (float)(e - s);
    return;
  }
  float acc = 0.0f;
  for (int64_t p = s; p < e; ++p) acc += load_weight(weights, wdt, p);
  denom[b] = acc;
}

// rows / nw of dedup position j (key position p = inverse[j])
__global__ __launch_bounds__(256) void backprop_prep_kernel(const void* inverse, int key_bytes, int64_t n,
                                                            PositionGrad g) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j < n) position_grad(g, j, load_key(inverse, key_bytes, j));
}

constexpr int kPieceThreads = 256;
constexpr uint32_t kNoKey = 0xffffffffu;

template <typename T>
__device__ __forceinline__ float grad_elem(const uint32_t* w, int e) {
  if constexpr (sizeof(T) == 2) return h2f(vhalf(w, e));
  else return __uint_as_float(w[e]);
}

// plain (cached) stores of fp32 partial rows: the combine kernel reads them next
template <int V>
__device__ __forceinline__ void store_partial(float* p, const float* v) {
  if constexpr (V % 4 == 0) {
#pragma unroll
    for (int c = 0; c < V / 4; ++c) {
      u32x4 x;
      x.x = __float_as_uint(v[4 * c]);
      x.y = __float_as_uint(v[4 * c + 1]);
      x.z = __float_as_uint(v[4 * c + 2]);
      x.w = __float_as_uint(v[4 * c + 3]);
      *reinterpret_cast<gptr_w<u32x4>>((uint64_t)(p + 4 * c)) = x;
    }
  } else {
#pragma unroll
    for (int i = 0; i < V; ++i) *reinterpret_cast<gptr_w<float>>((uint64_t)(p + i)) = v[i];
  }
}

// A finished piece: the key's row when the piece holds all of the key's
// positions, else slot 2b (the piece holds the block's first position) or
// 2b + 1 (its last).
template <typename T, int V>
__device__ __forceinline__ void emit_piece(const PieceArgs& a, int64_t b, uint32_t key,
                                           const float* acc, bool first, bool whole, int col) {
  if (whole) {
    store_out<V>(a.out + ((int64_t)key * a.dim + col) * (int64_t)sizeof(T), acc, sizeof(T) == 2);
  } else {
    store_partial<V>(a.slots + (2 * b + (first ? 0 : 1)) * a.dim + col, acc);
  }
}

// One lane group of G lanes per block of kPieceBlock dedup positions; lane l
// holds V consecutive columns of a chunk of G * V.  Lane l also loads the
// key, gradient row and weight of positions j * G + l (j < kPieceBlock / G);
// position i's values reach the whole group by a lane move from lane i % G
// (i is a compile-time constant: the block is unrolled in batches of U).  The
// row loads of batch t + 1 are issued before batch t is added, so the stores
// of finished keys never sit between a batch's loads and their use.
template <typename T, int V, int G, bool W, int BLK = kPieceBlock>
__global__ __launch_bounds__(kPieceThreads) void piece_pool_kernel(PieceArgs a) {
  constexpr int kGroups = kPieceThreads / G;
  constexpr int VB = V * (int)sizeof(T);
  constexpr int P = BLK / G > 0 ? BLK / G : 1;
  constexpr int U = BLK < 16 ? BLK : 16;
  constexpr int NB = BLK / U;
  const int lane = threadIdx.x & (G - 1);
  const int wlane = threadIdx.x & 63;  // lane in the wave (the lane moves select by it)
  const int64_t b = (int64_t)blockIdx.x * kGroups + threadIdx.x / G;
  const int64_t p0 = b * BLK;
  if (p0 >= a.n) return;
  const int cnt = a.n - p0 < BLK ? (int)(a.n - p0) : BLK;
  if (lane == 0) a.cross[b] = kNoKey;  // replaced below when a key crosses out
  uint32_t key[P], row[P];
  float wt[P];
#pragma unroll
  for (int j = 0; j < P; ++j) {
    const int i = j * G + lane;
    key[j] = i < cnt ? a.kidx[p0 + i] : kNoKey;
    row[j] = i < cnt ? a.rows[p0 + i] : kNoGradRow;
    if constexpr (W) wt[j] = i < cnt ? a.nw[p0 + i] : 0.0f;
  }
  const uint32_t prev_key = p0 > 0 ? a.kidx[p0 - 1] : kNoKey;
  const uint32_t next_key = p0 + BLK < a.n ? a.kidx[p0 + BLK] : kNoKey;
  const uint64_t row_bytes = (uint64_t)a.dim * sizeof(T);
  const uint64_t zero = (uint64_t)g_zero_row;
  // key / row / weight of position I of the block (I == BLK: the next block's first key)
  auto key_at = [&](auto I) -> uint32_t {
    constexpr int i = decltype(I)::value;
    if constexpr (i == BLK) return next_key;
    else return group_bcast<G, i % G>(key[i / G], wlane);
  };
  auto row_at = [&](auto I) -> uint32_t {
    constexpr int i = decltype(I)::value;
    return group_bcast<G, i % G>(row[i / G], wlane);
  };
  auto wt_at = [&](auto I) -> float {
    constexpr int i = decltype(I)::value;
    return __uint_as_float(group_bcast<G, i % G>(__float_as_uint(wt[i / G]), wlane));
  };
  for (int c0 = 0; c0 < a.dim; c0 += G * V) {
    const int col = c0 + lane * V;
    const bool active = col < a.dim;
    float acc[V];
#pragma unroll
    for (int v = 0; v < V; ++v) acc[v] = 0.0f;
    bool first = true, head = key_at(std::integral_constant<int, 0>{}) != prev_key;
    Vec<VB> buf[2][U];
    auto issue = [&](auto T0) {
      constexpr int t = decltype(T0)::value;
      auto one = [&](auto U0) {
        constexpr int u = decltype(U0)::value;
        const uint32_t r = row_at(std::integral_constant<int, t * U + u>{});
        const uint64_t addr = (r != kNoGradRow && active)
                                  ? (uint64_t)a.grads + (uint64_t)r * row_bytes + (uint64_t)col * sizeof(T)
                                  : zero;
        buf[t & 1][u] = load_vec<VB>(addr);
      };
      for_each_const<0, U>(one);
    };
    auto add = [&](auto T0) {
      constexpr int t = decltype(T0)::value;
      auto one = [&](auto U0) {
        constexpr int i = t * U + decltype(U0)::value;
        if (i < cnt) {
          if (row_at(std::integral_constant<int, i>{}) != kNoGradRow) {
            const Vec<VB>& g = buf[t & 1][decltype(U0)::value];
            if constexpr (W) {
              const float w = wt_at(std::integral_constant<int, i>{});
#pragma unroll
              for (int v = 0; v < V; ++v) acc[v] = __builtin_fmaf(grad_elem<T>(g.w, v), w, acc[v]);
            } else {
#pragma unroll
              for (int v = 0; v < V; ++v) acc[v] = acc[v] + grad_elem<T>(g.w, v);
            }
          }
          const uint32_t k = key_at(std::integral_constant<int, i>{});
          const bool key_ends = key_at(std::integral_constant<int, i + 1>{}) != k;
          if (key_ends || i + 1 == cnt) {  // the piece ends at i
            if (active) emit_piece<T, V>(a, b, k, acc, first, head && key_ends, col);
            // a key that starts in this block and continues past it is the
            // block's entry for the combine kernel
            if (head && !key_ends && c0 == 0 && lane == 0) a.cross[b] = k;
#pragma unroll
            for (int v = 0; v < V; ++v) acc[v] = 0.0f;
            first = false;
            head = true;
          }
        }
      };
      for_each_const<0, U>(one);
    };
    auto step = [&](auto T0) {
      constexpr int t = decltype(T0)::value;
      if (t * U < cnt) {
        if constexpr (t + 1 < NB) {
          if ((t + 1) * U < cnt) issue(std::integral_constant<int, t + 1>{});
        }
        add(T0);
      }
    };
    issue(std::integral_constant<int, 0>{});
    for_each_const<0, NB>(step);
  }
}

// Slot of piece j of a key whose first position is d (first block b = d / kPieceBlock).
__device__ __forceinline__ int64_t piece_slot(int64_t d, int64_t b, int64_t j) {
  return j == 0 ? 2 * b + (d == b * kPieceBlock ? 0 : 1) : 2 * (b + j);
}

// The keys that start in one block and continue past it (each block's entry
// of a.cross, kNoKey for none), kCombineBlocks blocks per workgroup.  The row
// of such a key: its J pieces in kPieceFanIn sub-sequences of
// ceil(J / kPieceFanIn), each added in order from 0, the sub-sequence sums
// added in order from 0, rounded once.  A key of at most kLightPieces pieces
// is done by one wave (wave w: the workgroup's w-th block); the longer ones
// afterwards by the whole workgroup, wave q adding sub-sequence q.
template <typename T, int V>
__global__ __launch_bounds__(64 * kPieceFanIn) void piece_combine_kernel(PieceArgs a) {
  constexpr int U = 8;
  static_assert(kCombineBlocks == kPieceFanIn, "one wave per block entry");
  __shared__ float s_q[kPieceFanIn][64 * V];
  __shared__ uint32_t s_heavy[kCombineBlocks];
  const int64_t blocks = (a.n + kPieceBlock - 1) / kPieceBlock;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint64_t zero = (uint64_t)g_zero_row;
  const int64_t bw = (int64_t)blockIdx.x * kCombineBlocks + w;

  // (1) one wave per block entry: keys of at most kLightPieces pieces
  uint32_t key = bw < blocks ? a.cross[bw] : kNoKey;
  int64_t d = 0, pieces = 0;
  if (key != kNoKey) {
    d = load_key(a.doff, a.key_bytes, key);
    const int64_t end = d + load_key(a.counts, a.key_bytes, key);
    pieces = (end - 1) / kPieceBlock - d / kPieceBlock + 1;
  }
  const bool heavy = key != kNoKey && pieces > kLightPieces;
  if (lane == 0) s_heavy[w] = heavy ? key : kNoKey;
  if (key != kNoKey && !heavy) {
    const int64_t b = d / kPieceBlock;
    const int64_t per_part = (pieces + kPieceFanIn - 1) / kPieceFanIn;
    for (int c0 = 0; c0 < a.dim; c0 += 64 * V) {
      const int col = c0 + lane * V;
      const bool active = col < a.dim;
      float tot[V], part[V];
#pragma unroll
      for (int v = 0; v < V; ++v) tot[v] = part[v] = 0.0f;
      for (int64_t j0 = 0; j0 < pieces; j0 += U) {
        Vec<4 * V> pv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int64_t j = j0 + u;
          const uint64_t addr =
              (j < pieces && active) ? (uint64_t)(a.slots + piece_slot(d, b, j) * a.dim + col) : zero;
          pv[u] = load_vec<4 * V>(addr);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int64_t j = j0 + u;
          if (j < pieces) {
#pragma unroll
            for (int v = 0; v < V; ++v) part[v] = part[v] + __uint_as_float(pv[u].w[v]);
            if ((j + 1) % per_part == 0 || j + 1 == pieces) {  // a sub-sequence ends
#pragma unroll
              for (int v = 0; v < V; ++v) {
                tot[v] = tot[v] + part[v];
                part[v] = 0.0f;
              }
            }
          }
        }
      }
      if (active) store_out<V>(a.out + ((int64_t)key * a.dim + col) * (int64_t)sizeof(T), tot, sizeof(T) == 2);
    }
  }
  __syncthreads();

  // (2) the long keys, one at a time with every wave
  constexpr int UH = 16;
  for (int e = 0; e < kCombineBlocks; ++e) {
    const uint32_t hkey = s_heavy[e];
    if (hkey == kNoKey) continue;  // uniform over the workgroup
    const int64_t hd = load_key(a.doff, a.key_bytes, hkey);
    const int64_t hend = hd + load_key(a.counts, a.key_bytes, hkey);
    const int64_t b = hd / kPieceBlock;
    const int64_t hpieces = (hend - 1) / kPieceBlock - b + 1;
    const int64_t per_part = (hpieces + kPieceFanIn - 1) / kPieceFanIn;
    const int64_t j_lo = w * per_part;
    const int64_t j_hi = j_lo + per_part < hpieces ? j_lo + per_part : hpieces;
    for (int c0 = 0; c0 < a.dim; c0 += 64 * V) {
      const int col = c0 + lane * V;
      const bool active = col < a.dim;
      float part[V];
#pragma unroll
      for (int v = 0; v < V; ++v) part[v] = 0.0f;
      for (int64_t j0 = j_lo; j0 < j_hi; j0 += UH) {
        Vec<4 * V> pv[UH];
#pragma unroll
        for (int u = 0; u < UH; ++u) {
          const int64_t j = j0 + u;
          const uint64_t addr =
              (j < j_hi && active) ? (uint64_t)(a.slots + piece_slot(hd, b, j) * a.dim + col) : zero;
          pv[u] = load_vec<4 * V>(addr);
        }
#pragma unroll
        for (int u = 0; u < UH; ++u) {
          if (j0 + u < j_hi) {
#pragma unroll
            for (int v = 0; v < V; ++v) part[v] = part[v] + __uint_as_float(pv[u].w[v]);
          }
        }
      }
#pragma unroll
      for (int v = 0; v < V; ++v) s_q[w][lane * V + v] = part[v];
      __syncthreads();
      if (w == 0 && active) {
        float t[V];
#pragma unroll
        for (int v = 0; v < V; ++v) {
          t[v] = 0.0f;
#pragma unroll
          for (int qq = 0; qq < kPieceFanIn; ++qq) t[v] = t[v] + s_q[qq][lane * V + v];
        }
        store_out<V>(a.out + ((int64_t)hkey * a.dim + col) * (int64_t)sizeof(T), t, sizeof(T) == 2);
      }
      __syncthreads();
    }
  }
}
}  // namespace

hipError_t launch_bag_denom(const void* offsets, int key_bytes, int64_t num_bags, int64_t hotness,
                            const void* weights, int wdt, int wmean, float* denom,
                            hipStream_t stream) {
  if (num_bags <= 0) return hipSuccess;
  hipLaunchKernelGGL(bag_denom_kernel, dim3((unsigned)((num_bags + 255) / 256)), dim3(256), 0, stream,
                     offsets, key_bytes, num_bags, hotness, weights, wdt, wmean, denom);
  return hipGetLastError();
}

hipError_t launch_backprop_prep(const void* inverse, int key_bytes, int64_t n, const PositionGrad& g,
                                hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(backprop_prep_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                     inverse, key_bytes, n, g);
  return hipGetLastError();
}

namespace {

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int lanes_for(int64_t needed) {
  int g = 8;
  while (g < 64 && g < needed) g *= 2;
  return g;
}

template <typename T, int V, bool W>
hipError_t piece_pool_g(const PieceArgs& a, int g, hipStream_t s) {
  const int64_t blocks = (a.n + kPieceBlock - 1) / kPieceBlock;
#define NVE_PIECE_POOL(GG)                                                                         \
  hipLaunchKernelGGL((piece_pool_kernel<T, V, GG, W>),                                            \
                     dim3((unsigned)((blocks + kPieceThreads / GG - 1) / (kPieceThreads / GG))),   \
                     dim3(kPieceThreads), 0, s, a)
  if (g == 8) NVE_PIECE_POOL(8);
  else if (g == 16) NVE_PIECE_POOL(16);
  else if (g == 32) NVE_PIECE_POOL(32);
  else NVE_PIECE_POOL(64);
#undef NVE_PIECE_POOL
  return hipGetLastError();
}

template <typename T, bool W>
hipError_t piece_pool_t(const PieceArgs& a, hipStream_t s) {
  constexpr int kVec = 16 / (int)sizeof(T);
  if ((a.dim * (int64_t)sizeof(T)) % 16 == 0 && aligned16(a.grads) && aligned16(a.out))
    return piece_pool_g<T, kVec, W>(a, lanes_for(a.dim / kVec), s);
  return piece_pool_g<T, 1, W>(a, lanes_for(a.dim), s);
}

}  // namespace

hipError_t launch_piece_pool(const PieceArgs& a, int f16, int weighted, hipStream_t stream) {
  if (a.n <= 0) return hipSuccess;
  if (f16) return weighted ? piece_pool_t<uint16_t, true>(a, stream) : piece_pool_t<uint16_t, false>(a, stream);
  return weighted ? piece_pool_t<float, true>(a, stream) : piece_pool_t<float, false>(a, stream);
}

hipError_t launch_piece_combine(const PieceArgs& a, int f16, hipStream_t stream) {
  const int64_t blocks = (a.n + kPieceBlock - 1) / kPieceBlock;
  if (blocks <= 1) return hipSuccess;  // no key crosses out of the last block
  const bool vec = a.dim % 4 == 0 && aligned16(a.out);
  const dim3 grid((unsigned)((blocks + kCombineBlocks - 1) / kCombineBlocks)), block(64 * kPieceFanIn);
  if (f16) {
    if (vec) hipLaunchKernelGGL((piece_combine_kernel<uint16_t, 4>), grid, block, 0, stream, a);
    else hipLaunchKernelGGL((piece_combine_kernel<uint16_t, 1>), grid, block, 0, stream, a);
  } else {
    if (vec) hipLaunchKernelGGL((piece_combine_kernel<float, 4>), grid, block, 0, stream, a);
    else hipLaunchKernelGGL((piece_combine_kernel<float, 1>), grid, block, 0, stream, a);
  }
  return hipGetLastError();
}

}  // namespace nve_amd
