// host_kernels.cpp -- see host_kernels.hpp.  Built with -ffp-contract=off:
// the only fused multiply-adds are the explicit ones of the dequantization.
#include "host_kernels.hpp"

#include <immintrin.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <exception>
#include <future>
#include <numeric>
#include <vector>

#include "dtypes.hpp"

namespace nve_amd {
namespace hostk {

namespace {

int64_t load_key(const void* keys, int key_bytes, int64_t i) {
  return key_bytes == 4 ? (int64_t) static_cast<const int32_t*>(keys)[i]
                        : static_cast<const int64_t*>(keys)[i];
}

// key_utils.hpp:33-42: a negative key or one past the table addresses no row
bool in_range(int64_t key, uint64_t num_rows) { return key >= 0 && (uint64_t)key < num_rows; }

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

float ld_f32(const uint8_t* p) {
  float v;
  std::memcpy(&v, p, 4);
  return v;
}
uint16_t ld_u16(const uint8_t* p) {
  uint16_t v;
  std::memcpy(&v, p, 2);
  return v;
}

// OCP FP8 E4M3FN from its definition: 1 sign, 4 exponent (bias 7), 3 mantissa
// bits; exponent 0 is subnormal (m/8 * 2^-6); S.1111.111 is NaN; no infinity.
struct E4M3Table {
  float v[256];
  E4M3Table() {
    for (int c = 0; c < 256; ++c) {
      const int e = (c >> 3) & 15, m = c & 7;
      float mag;
      if ((c & 0x7F) == 0x7F)
        mag = std::nanf("");
      else if (e == 0)
        mag = std::ldexp((float)m, -9);
      else
        mag = std::ldexp((float)(8 + m), e - 10);
      v[c] = (c & 0x80) ? -mag : mag;
    }
  }
};
const E4M3Table kE4M3;

// Decodes the `count` values of one stored row to floats (the per-element
// arithmetic of the header comment).
void decode_row(int dtype, int64_t count, const uint8_t* row, float* out) {
  switch (dtype) {
    case kF32:
      std::memcpy(out, row, (size_t)count * 4);
      return;
    case kF16:
      for (int64_t i = 0; i < count; ++i) out[i] = half_bits_to_float(ld_u16(row + 2 * i));
      return;
    case kQI8F32:
    case kQI8F16: {
      const float s = dtype == kQI8F32 ? ld_f32(row + count) : half_bits_to_float(ld_u16(row + count));
      for (int64_t i = 0; i < count; ++i) out[i] = std::fma((float)(int8_t)row[i], s, 0.0f);
      return;
    }
    case kQU8F32:
    case kQU8F16: {
      const bool f32 = dtype == kQU8F32;
      const float s = f32 ? ld_f32(row + count) : half_bits_to_float(ld_u16(row + count));
      const float o = f32 ? ld_f32(row + count + 4) : half_bits_to_float(ld_u16(row + count + 2));
      for (int64_t i = 0; i < count; ++i) out[i] = std::fma((float)row[i], s, o);
      return;
    }
    case kXI8AF32: {
      const float s = ld_f32(row + count), o = ld_f32(row + count + 4);
      for (int64_t i = 0; i < count; ++i) out[i] = std::fma((float)(int8_t)row[i], s, o);
      return;
    }
    case kXE4M3F32: {
      const float s = ld_f32(row + count);
      for (int64_t i = 0; i < count; ++i) out[i] = kE4M3.v[row[i]] * s;
      return;
    }
    default:
      NVE_CHECK(false, "Unsupported row format ", dtype);
  }
}

// ---- row loops: portable versions ----
void add_f32_s(float* acc, const float* x, int64_t n) {
  for (int64_t i = 0; i < n; ++i) acc[i] += x[i];
}
void add_f32_w_s(float* acc, const float* x, float w, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    const float v = x[i] * w;
    acc[i] += v;
  }
}
void add_f16_s(float* acc, const uint16_t* x, int64_t n) {
  for (int64_t i = 0; i < n; ++i) acc[i] += half_bits_to_float(x[i]);
}
void add_f16_w_s(float* acc, const uint16_t* x, float w, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    const float v = half_bits_to_float(x[i]) * w;
    acc[i] += v;
  }
}
void store_f16_s(uint16_t* out, const float* acc, float inv, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = float_to_half_bits(acc[i] * inv);
}
void widen_f16_s(float* out, const uint16_t* x, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = half_bits_to_float(x[i]);
}

// ---- row loops: AVX2 + F16C (8 values per instruction) ----
__attribute__((target("avx2,f16c,fma"))) void add_f32_v(float* acc, const float* x, int64_t n) {
  int64_t i = 0;
  for (; i + 8 <= n; i += 8)
    _mm256_storeu_ps(acc + i, _mm256_add_ps(_mm256_loadu_ps(acc + i), _mm256_loadu_ps(x + i)));
  for (; i < n; ++i) acc[i] += x[i];
}
__attribute__((target("avx2,f16c,fma"))) void add_f32_w_v(float* acc, const float* x, float w,
                                                           int64_t n) {
  const __m256 vw = _mm256_set1_ps(w);
  int64_t i = 0;
  for (; i + 8 <= n; i += 8) {
    const __m256 v = _mm256_mul_ps(_mm256_loadu_ps(x + i), vw);
    _mm256_storeu_ps(acc + i, _mm256_add_ps(_mm256_loadu_ps(acc + i), v));
  }
  for (; i < n; ++i) {
    const float v = x[i] * w;
    acc[i] += v;
  }
}
__attribute__((target("avx2,f16c,fma"))) void add_f16_v(float* acc, const uint16_t* x, int64_t n) {
  int64_t i = 0;
  for (; i + 8 <= n; i += 8) {
    const __m256 v = _mm256_cvtph_ps(_mm_loadu_si128(reinterpret_cast<const __m128i*>(x + i)));
    _mm256_storeu_ps(acc + i, _mm256_add_ps(_mm256_loadu_ps(acc + i), v));
  }
  for (; i < n; ++i) acc[i] += _cvtsh_ss(x[i]);
}
__attribute__((target("avx2,f16c,fma"))) void add_f16_w_v(float* acc, const uint16_t* x, float w,
                                                           int64_t n) {
  const __m256 vw = _mm256_set1_ps(w);
  int64_t i = 0;
  for (; i + 8 <= n; i += 8) {
    const __m256 v =
        _mm256_mul_ps(_mm256_cvtph_ps(_mm_loadu_si128(reinterpret_cast<const __m128i*>(x + i))), vw);
    _mm256_storeu_ps(acc + i, _mm256_add_ps(_mm256_loadu_ps(acc + i), v));
  }
  for (; i < n; ++i) {
    const float v = _cvtsh_ss(x[i]) * w;
    acc[i] += v;
  }
}
__attribute__((target("avx2,f16c,fma"))) void store_f16_v(uint16_t* out, const float* acc, float inv,
                                                           int64_t n) {
  const __m256 vi = _mm256_set1_ps(inv);
  int64_t i = 0;
  for (; i + 8 <= n; i += 8) {
    const __m128i h = _mm256_cvtps_ph(_mm256_mul_ps(_mm256_loadu_ps(acc + i), vi), _MM_FROUND_TO_NEAREST_INT);
    _mm_storeu_si128(reinterpret_cast<__m128i*>(out + i), h);
  }
  for (; i < n; ++i) out[i] = _cvtss_sh(acc[i] * inv, _MM_FROUND_TO_NEAREST_INT);
}
__attribute__((target("avx2,f16c,fma"))) void widen_f16_v(float* out, const uint16_t* x, int64_t n) {
  int64_t i = 0;
  for (; i + 8 <= n; i += 8)
    _mm256_storeu_ps(out + i, _mm256_cvtph_ps(_mm_loadu_si128(reinterpret_cast<const __m128i*>(x + i))));
  for (; i < n; ++i) out[i] = _cvtsh_ss(x[i]);
}

struct Ops {
  void (*add_f32)(float*, const float*, int64_t);
  void (*add_f32_w)(float*, const float*, float, int64_t);
  void (*add_f16)(float*, const uint16_t*, int64_t);
  void (*add_f16_w)(float*, const uint16_t*, float, int64_t);
  void (*store_f16)(uint16_t*, const float*, float, int64_t);
  void (*widen_f16)(float*, const uint16_t*, int64_t);
  bool vector;
};

const Ops& ops() {
  static const Ops o = [] {
    __builtin_cpu_init();
    if (__builtin_cpu_supports("avx2") && __builtin_cpu_supports("f16c") &&
        __builtin_cpu_supports("fma"))
      return Ops{add_f32_v, add_f32_w_v, add_f16_v, add_f16_w_v, store_f16_v, widen_f16_v, true};
    return Ops{add_f32_s, add_f32_w_s, add_f16_s, add_f16_w_s, store_f16_s, widen_f16_s, false};
  }();
  return o;
}

float weight_at(const void* w, int type, int64_t k) {
  return type == kF16 ? half_bits_to_float(static_cast<const uint16_t*>(w)[k])
                      : static_cast<const float*>(w)[k];
}

// Positions 0..n-1 ordered by key (stable), for work split by key.
std::vector<int64_t> positions_by_key(int64_t n, const void* keys, int key_bytes) {
  std::vector<int64_t> pos((size_t)n);
  std::iota(pos.begin(), pos.end(), (int64_t)0);
  std::stable_sort(pos.begin(), pos.end(), [&](int64_t a, int64_t b) {
    return load_key(keys, key_bytes, a) < load_key(keys, key_bytes, b);
  });
  return pos;
}

// Cuts [0, n) of `pos` into at most `tasks` pieces whose edges fall between
// runs of equal keys; returns the piece edges.
std::vector<int64_t> run_edges(const std::vector<int64_t>& pos, const void* keys, int key_bytes,
                               int64_t tasks) {
  const int64_t n = (int64_t)pos.size();
  std::vector<int64_t> edges{0};
  const int64_t per = std::max<int64_t>(1, ceil_div(n, std::max<int64_t>(1, tasks)));
  int64_t at = 0;
  while (at < n) {
    int64_t e = std::min(n, at + per);
    while (e < n && load_key(keys, key_bytes, pos[(size_t)e]) == load_key(keys, key_bytes, pos[(size_t)e - 1]))
      ++e;
    edges.push_back(e);
    at = e;
  }
  return edges;
}

}  // namespace

bool vector_loops() { return ops().vector; }

void run_tasks(ThreadPool& pool, int64_t num_tasks, const std::function<void(int64_t)>& task) {
  if (num_tasks <= 0) return;
  std::vector<std::future<void>> fs;
  fs.reserve((size_t)num_tasks - 1);
  for (int64_t t = 1; t < num_tasks; ++t) fs.push_back(pool.submit([&task, t] { task(t); }));
  std::exception_ptr first;
  try {
    task(0);
  } catch (...) {
    first = std::current_exception();
  }
  for (auto& f : fs) {
    try {
      f.get();
    } catch (...) {
      if (!first) first = std::current_exception();
    }
  }
  if (first) std::rethrow_exception(first);
}

int64_t gather(ThreadPool& pool, int64_t num_threads, int64_t n, const void* keys, int key_bytes,
               uint64_t* hit_mask, uint8_t* values, int64_t value_stride, const uint8_t* table,
               int64_t row_bytes, uint64_t num_rows) {
  if (n <= 0) return 0;
  num_threads = std::max<int64_t>(1, num_threads);
  // keys per task: ceil(n / threads) rounded up to whole hit-mask words
  const int64_t per = (ceil_div(n, num_threads) + 63) / 64 * 64;
  const int64_t tasks = ceil_div(n, per);
  std::atomic<int64_t> hits{0};
  constexpr int64_t kAhead = 8;  // rows prefetched ahead of the copy
  run_tasks(pool, tasks, [&](int64_t t) {
    const int64_t s = t * per, e = std::min(n, s + per);
    int64_t h = 0;
    for (int64_t i = s; i < std::min(e, s + kAhead); ++i) {
      const int64_t k = load_key(keys, key_bytes, i);
      if (in_range(k, num_rows))
        for (int64_t b = 0; b < row_bytes; b += 64) __builtin_prefetch(table + (uint64_t)k * row_bytes + b);
    }
    for (int64_t i = s; i < e; ++i) {
      if (i + kAhead < e) {
        const int64_t k2 = load_key(keys, key_bytes, i + kAhead);
        if (in_range(k2, num_rows))
          for (int64_t b = 0; b < row_bytes; b += 64)
            __builtin_prefetch(table + (uint64_t)k2 * row_bytes + b);
      }
      const uint64_t bit = 1ull << (i & 63);
      if (hit_mask && (hit_mask[i >> 6] & bit)) continue;
      const int64_t k = load_key(keys, key_bytes, i);
      if (!in_range(k, num_rows)) continue;
      std::memcpy(values + i * value_stride, table + (uint64_t)k * (uint64_t)row_bytes, (size_t)row_bytes);
      ++h;
      if (hit_mask) hit_mask[i >> 6] |= bit;
    }
    hits.fetch_add(h, std::memory_order_relaxed);
  });
  return hits.load();
}

void pool(ThreadPool& tp, int64_t workers, const PoolSpec& sp, int64_t num_bags, const uint8_t* rows,
          int64_t row_stride, uint8_t* out, int64_t out_stride) {
  if (num_bags <= 0) return;
  const Ops& op = ops();
  const bool weighted = sp.pooling == NVE_POOL_WEIGHTED_SUM || sp.pooling == NVE_POOL_WEIGHTED_MEAN;
  const bool mean = sp.pooling == NVE_POOL_MEAN || sp.pooling == NVE_POOL_WEIGHTED_MEAN;
  const int64_t count = sp.count;
  const int oes = sp.out_type == kF16 ? 2 : 4;
  const int64_t per = std::max<int64_t>(1, ceil_div(num_bags, std::max<int64_t>(1, workers)));
  run_tasks(tp, ceil_div(num_bags, per), [&](int64_t t) {
    std::vector<float> acc((size_t)count), tmp((size_t)count);
    const int64_t b1 = std::min(num_bags, (t + 1) * per);
    for (int64_t b = t * per; b < b1; ++b) {
      int64_t s, e;
      if (sp.sparse == NVE_SPARSE_FIXED) {
        s = b * sp.fixed_hotness;
        e = s + sp.fixed_hotness;
      } else {
        s = load_key(sp.offsets, sp.offset_bytes, b);
        e = load_key(sp.offsets, sp.offset_bytes, b + 1);
      }
      uint8_t* orow = out + b * out_stride;
      if (e - s <= 0) {  // empty bag: zero row
        std::memset(orow, 0, (size_t)(count * oes));
        continue;
      }
      std::fill(acc.begin(), acc.end(), 0.0f);
      float wsum = 0.0f;
      for (int64_t k = s; k < e; ++k) {
        const float w = weighted ? weight_at(sp.weights, sp.weight_type, k) : 1.0f;
        wsum += w;
        const uint8_t* row = rows + k * row_stride;
        if (sp.dtype == kF16) {
          const uint16_t* h = reinterpret_cast<const uint16_t*>(row);
          if (weighted)
            op.add_f16_w(acc.data(), h, w, count);
          else
            op.add_f16(acc.data(), h, count);
          continue;
        }
        const float* x;
        if (sp.dtype == kF32 && ((uintptr_t)row & 3) == 0) {
          x = reinterpret_cast<const float*>(row);
        } else {
          decode_row(sp.dtype, count, row, tmp.data());
          x = tmp.data();
        }
        if (weighted)
          op.add_f32_w(acc.data(), x, w, count);
        else
          op.add_f32(acc.data(), x, count);
      }
      float inv = 1.0f;
      if (mean) {
        const float denom = weighted ? wsum : (float)(e - s);
        inv = denom != 0.0f ? 1.0f / denom : 0.0f;
      }
      if (sp.out_type == kF16) {
        op.store_f16(reinterpret_cast<uint16_t*>(orow), acc.data(), inv, count);
      } else {
        float* o = reinterpret_cast<float*>(orow);
        for (int64_t i = 0; i < count; ++i) o[i] = acc[(size_t)i] * inv;
      }
    }
  });
}

void convert(ThreadPool& tp, int64_t workers, int dtype, int64_t count, int out_type, int64_t num_rows,
             const uint8_t* rows, int64_t row_stride, uint8_t* out, int64_t out_stride) {
  if (num_rows <= 0) return;
  const Ops& op = ops();
  const int64_t per = std::max<int64_t>(1, ceil_div(num_rows, std::max<int64_t>(1, workers)));
  run_tasks(tp, ceil_div(num_rows, per), [&](int64_t t) {
    std::vector<float> tmp((size_t)count);
    const int64_t r1 = std::min(num_rows, (t + 1) * per);
    for (int64_t r = t * per; r < r1; ++r) {
      const uint8_t* row = rows + r * row_stride;
      uint8_t* o = out + r * out_stride;
      if (dtype == kF16)
        op.widen_f16(tmp.data(), reinterpret_cast<const uint16_t*>(row), count);
      else
        decode_row(dtype, count, row, tmp.data());
      if (out_type == kF16)
        op.store_f16(reinterpret_cast<uint16_t*>(o), tmp.data(), 1.0f, count);
      else
        std::memcpy(o, tmp.data(), (size_t)count * 4);
    }
  });
}

void copy_rows(ThreadPool& tp, int64_t workers, int64_t num_rows, const uint8_t* src, int64_t src_stride,
               uint8_t* dst, int64_t dst_stride, int64_t row_bytes) {
  if (num_rows <= 0) return;
  const int64_t per = std::max<int64_t>(1, ceil_div(num_rows, std::max<int64_t>(1, workers)));
  run_tasks(tp, ceil_div(num_rows, per), [&](int64_t t) {
    const int64_t r1 = std::min(num_rows, (t + 1) * per);
    for (int64_t r = t * per; r < r1; ++r)
      std::memcpy(dst + r * dst_stride, src + r * src_stride, (size_t)row_bytes);
  });
}

void update_rows(ThreadPool& tp, int64_t num_threads, int64_t n, const void* keys, int key_bytes,
                 const uint8_t* values, int64_t value_stride, uint8_t* table, int64_t row_bytes,
                 uint64_t num_rows) {
  if (n <= 0) return;
  const std::vector<int64_t> pos = positions_by_key(n, keys, key_bytes);
  const std::vector<int64_t> edges = run_edges(pos, keys, key_bytes, num_threads);
  run_tasks(tp, (int64_t)edges.size() - 1, [&](int64_t t) {
    for (int64_t j = edges[(size_t)t]; j < edges[(size_t)t + 1]; ++j) {
      const int64_t i = pos[(size_t)j];
      const int64_t k = load_key(keys, key_bytes, i);
      // a run of one key writes its last position only
      if (j + 1 < edges[(size_t)t + 1] && load_key(keys, key_bytes, pos[(size_t)j + 1]) == k) continue;
      if (!in_range(k, num_rows)) continue;
      std::memcpy(table + (uint64_t)k * row_bytes, values + i * value_stride, (size_t)row_bytes);
    }
  });
}

void accumulate_rows(ThreadPool& tp, int64_t num_threads, int64_t n, const void* keys, int key_bytes,
                     const uint8_t* updates, int64_t update_stride, uint8_t* table,
                     int64_t row_bytes, uint64_t num_rows, int dtype) {
  if (n <= 0) return;
  const bool f16 = dtype == kF16;
  const int64_t count = row_bytes / (f16 ? 2 : 4);
  const std::vector<int64_t> pos = positions_by_key(n, keys, key_bytes);
  const std::vector<int64_t> edges = run_edges(pos, keys, key_bytes, num_threads);
  run_tasks(tp, (int64_t)edges.size() - 1, [&](int64_t t) {
    for (int64_t j = edges[(size_t)t]; j < edges[(size_t)t + 1]; ++j) {
      const int64_t i = pos[(size_t)j];
      const int64_t k = load_key(keys, key_bytes, i);
      if (!in_range(k, num_rows)) continue;
      uint8_t* dst = table + (uint64_t)k * row_bytes;
      const uint8_t* src = updates + i * update_stride;
      if (f16) {
        uint16_t* dh = reinterpret_cast<uint16_t*>(dst);
        for (int64_t e = 0; e < count; ++e)
          dh[e] = float_to_half_bits(half_bits_to_float(dh[e]) + half_bits_to_float(ld_u16(src + 2 * e)));
      } else {
        float* df = reinterpret_cast<float*>(dst);
        for (int64_t e = 0; e < count; ++e) df[e] = df[e] + ld_f32(src + 4 * e);
      }
    }
  });
}

}  // namespace hostk
}  // namespace nve_amd
