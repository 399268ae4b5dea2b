/*
 * nve_oracle.c -- CPU restatement of the NV Embedding Cache lookup path.
 *
 * TEST INFRASTRUCTURE ONLY (see nve_oracle.h): the checker for the MI355X
 * kernels and the timed CPU baseline, never part of the product.
 *
 * Reference citations are to /root/reference (NVE 26.09.0).
 */
#define _GNU_SOURCE
#include "nve_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------- */
/* scalar conversions                                                        */
/* ------------------------------------------------------------------------- */

/* IEEE binary16 -> binary32, exact (every half is a float). */
float orc_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu;
  const uint32_t man = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    /* zero or subnormal: man * 2^-24 is exact in binary32 */
    float v = ldexpf((float)man, -24);
    memcpy(&bits, &v, 4);
    bits |= sign;
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp - 15u + 127u) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

/* binary32 -> binary16, round to nearest even (the rounding of __float2half
 * and of the gfx950 v_cvt_f16_f32 instruction). */
uint16_t orc_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) { /* inf / nan */
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    return (uint16_t)(sign | 0x7c00u);
  }
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
  if (ax < 0x38800000u) {                                   /* below 2^-14: subnormal half */
    float a;
    memcpy(&a, &ax, 4);
    const float scaled = a * 16777216.0f; /* a / 2^-24, exact */
    const uint32_t m = (uint32_t)nearbyintf(scaled); /* default mode: nearest-even */
    return (uint16_t)(sign | m);
  }
  const uint32_t e = (ax >> 23) - 127u + 15u;
  const uint32_t mant = ax & 0x7fffffu;
  uint32_t h = (e << 10) | (mant >> 13);
  const uint32_t rem = mant & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
  return (uint16_t)(sign | h);
}

/* OCP FP8 E4M3FN: bias 7, 3 mantissa bits, no infinities, NaN = S.1111.111.
 * (gfx950 uses this OCP encoding.) */
float orc_e4m3_to_f32(uint8_t v) {
  const int s = v >> 7;
  const int e = (v >> 3) & 0xf;
  const int m = v & 7;
  float r;
  if (e == 15 && m == 7) {
    r = NAN;
  } else if (e == 0) {
    r = ldexpf((float)m, -9); /* m/8 * 2^-6 */
  } else {
    r = ldexpf(1.0f + (float)m / 8.0f, e - 7);
  }
  return s ? -r : r;
}

void orc_f16_to_f32_n(const uint16_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; i++) out[i] = orc_f16_to_f32(in[i]);
}
void orc_f32_to_f16_n(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; i++) out[i] = orc_f32_to_f16(in[i]);
}

/* ------------------------------------------------------------------------- */
/* row layout (nve_types.hpp:143-189, kernels_common.cuh:67-172)             */
/* ------------------------------------------------------------------------- */

int64_t orc_meta_bytes(int dtype) {
  switch (dtype) {
    case ORC_QI8_F32: return 4;
    case ORC_QI8_F16: return 2;
    case ORC_QU8_F32: return 8;
    case ORC_QU8_F16: return 4;
    case ORC_XI8A_F32: return 8;
    case ORC_XE4M3_F32: return 4;
    default: return 0;
  }
}

int64_t orc_value_bytes(int dtype) {
  switch (dtype) {
    case ORC_F32: return 4;
    case ORC_F16: return 2;
    default: return 1;
  }
}

int orc_out_dtype_native(int dtype) {
  switch (dtype) {
    case ORC_F16:
    case ORC_QI8_F16:
    case ORC_QU8_F16: return ORC_F16;
    default: return ORC_F32;
  }
}

/* ------------------------------------------------------------------------- */
/* keys (key_utils.hpp:33-42, sanitize_keys.cuh:30-45)                       */
/* ------------------------------------------------------------------------- */

int orc_key_in_range(int64_t key, uint64_t num_rows) {
  if (key < 0) return 0;
  return (uint64_t)key < num_rows;
}

static int64_t load_key(const void* keys, int key_bytes, int64_t i) {
  if (key_bytes == 4) return (int64_t)((const int32_t*)keys)[i];
  return ((const int64_t*)keys)[i];
}

void orc_sanitize_keys(const void* keys, void* out, int64_t n, int key_bytes, uint64_t num_rows,
                       int64_t default_row) {
  for (int64_t i = 0; i < n; i++) {
    const int64_t k = load_key(keys, key_bytes, i);
    const int64_t r = orc_key_in_range(k, num_rows) ? k : default_row;
    if (key_bytes == 4)
      ((int32_t*)out)[i] = (int32_t)r;
    else
      ((int64_t*)out)[i] = r;
  }
}

/* ------------------------------------------------------------------------- */
/* gather (cpu_gather.hpp:28-80)                                             */
/* ------------------------------------------------------------------------- */

int64_t orc_gather(const void* keys, int key_bytes, int64_t n, uint64_t* hit_mask,
                   const uint8_t* table, uint64_t num_rows, int64_t row_bytes, uint8_t* out,
                   int64_t out_stride) {
  int64_t hits = 0;
  for (int64_t i = 0; i < n; i++) {
    const uint64_t bit = 1ull << (i % 64);
    if (hit_mask && (hit_mask[i / 64] & bit)) continue;
    const int64_t k = load_key(keys, key_bytes, i);
    if (!orc_key_in_range(k, num_rows)) continue;
    memcpy(out + i * out_stride, table + (uint64_t)k * (uint64_t)row_bytes, (size_t)row_bytes);
    hits++;
    if (hit_mask) hit_mask[i / 64] |= bit;
  }
  return hits;
}

void orc_linear_rows(const void* keys, int key_bytes, int64_t n, const uint8_t* table,
                     int64_t row_bytes, const uint8_t** rows) {
  for (int64_t i = 0; i < n; i++) {
    const int64_t k = load_key(keys, key_bytes, i);
    rows[i] = table + (uint64_t)k * (uint64_t)row_bytes;
  }
}

/* ------------------------------------------------------------------------- */
/* dequant (kernels_common.cuh:174-297, find_and_dequant.cuh:41-123)         */
/* ------------------------------------------------------------------------- */

static float ld_f32(const uint8_t* p) {
  float v;
  memcpy(&v, p, 4);
  return v;
}
static uint16_t ld_u16(const uint8_t* p) {
  uint16_t v;
  memcpy(&v, p, 2);
  return v;
}

/* One element in the dtype's native parameter precision.  For the F16-metadata
 * types the value is produced as a half (rounded once), exactly like the
 * reference's dequantize<...F16> specialisations; *is_half tells the caller. */
typedef struct {
  float f;
  uint16_t h;
  int is_half;
} orc_elem;

static orc_elem dequant_elem(const uint8_t* row, int dtype, int64_t count, int64_t e) {
  orc_elem r = {0.0f, 0, 0};
  switch (dtype) {
    case ORC_F32:
      r.f = ld_f32(row + 4 * e);
      break;
    case ORC_F16:
      r.h = ld_u16(row + 2 * e);
      r.is_half = 1;
      break;
    case ORC_QI8_F32: {
      /* float(q)*scale + offset with offset = 0 (kernels_common.cuh:178-183);
       * contracted to one fma as nvcc does by default. */
      const float s = ld_f32(row + count);
      r.f = fmaf((float)(int8_t)row[e], s, 0.0f);
      break;
    }
    case ORC_QU8_F32: {
      const float s = ld_f32(row + count);
      const float o = ld_f32(row + count + 4);
      r.f = fmaf((float)row[e], s, o);
      break;
    }
    case ORC_QI8_F16: {
      /* __float2half(float(q) * __half2float(scale)) (kernels_common.cuh:247-265) */
      const float s = orc_f16_to_f32(ld_u16(row + count));
      r.h = orc_f32_to_f16((float)(int8_t)row[e] * s);
      r.is_half = 1;
      break;
    }
    case ORC_QU8_F16: {
      /* __float2half(float(q)*scale + offset), contracted (kernels_common.cuh:267-288) */
      const float s = orc_f16_to_f32(ld_u16(row + count));
      const float o = orc_f16_to_f32(ld_u16(row + count + 2));
      r.h = orc_f32_to_f16(fmaf((float)row[e], s, o));
      r.is_half = 1;
      break;
    }
    case ORC_XI8A_F32: {
      /* extension: int8 affine, float(q)*scale + offset as one fma */
      const float s = ld_f32(row + count);
      const float o = ld_f32(row + count + 4);
      r.f = fmaf((float)(int8_t)row[e], s, o);
      break;
    }
    case ORC_XE4M3_F32: {
      /* extension: e4m3 value times fp32 scale */
      const float s = ld_f32(row + count);
      r.f = orc_e4m3_to_f32(row[e]) * s;
      break;
    }
    default:
      break;
  }
  return r;
}

static float elem_as_f32(orc_elem x) { return x.is_half ? orc_f16_to_f32(x.h) : x.f; }

void orc_dequant_row(const uint8_t* row, int dtype, int64_t count, int out_dtype, void* out) {
  for (int64_t e = 0; e < count; e++) {
    const orc_elem x = dequant_elem(row, dtype, count, e);
    if (out_dtype == ORC_F16) {
      ((uint16_t*)out)[e] = x.is_half ? x.h : orc_f32_to_f16(x.f);
    } else {
      ((float*)out)[e] = elem_as_f32(x);
    }
  }
}

/* ------------------------------------------------------------------------- */
/* pooling                                                                   */
/* ------------------------------------------------------------------------- */

static float load_weight(const void* w, int wdtype, int64_t k) {
  if (wdtype == ORC_F16) return orc_f16_to_f32(((const uint16_t*)w)[k]);
  return ((const float*)w)[k];
}

static void bag_range(int sparse, const void* offsets, int key_bytes, int64_t b, int64_t hotness,
                      int64_t* s, int64_t* e) {
  if (sparse == ORC_FIXED) {
    *s = b * hotness;
    *e = *s + hotness;
  } else {
    *s = load_key(offsets, key_bytes, b);
    *e = load_key(offsets, key_bytes, b + 1);
  }
}

static void store_out(void* out, int64_t out_stride, int64_t b, int out_dtype, const float* acc,
                      int64_t count) {
  uint8_t* row = (uint8_t*)out + b * out_stride;
  for (int64_t e = 0; e < count; e++) {
    if (out_dtype == ORC_F16)
      ((uint16_t*)row)[e] = orc_f32_to_f16(acc[e]);
    else
      ((float*)row)[e] = acc[e];
  }
}

/* find_and_combine_kernel.cuh:40-154: per bag, per element, fp32 accumulation in
 * key order; weighted: acc += x*w (fused); Mean/WMean: denominator accumulated
 * in fp32 (1.0 per key or w), result = acc / denom, zero denominator -> zero row;
 * output cast round-to-nearest-even. */
void orc_pool(const uint8_t* const* rows, int dtype, int64_t count, int sparse, int pooling,
              int64_t num_keys, const void* offsets, int key_bytes, int64_t num_bags,
              int64_t hotness, const void* weights, int weight_dtype, int out_dtype, void* out,
              int64_t out_stride) {
  (void)num_keys;
  const int weighted = (pooling == ORC_WSUM || pooling == ORC_WMEAN);
  const int mean = (pooling == ORC_MEAN || pooling == ORC_WMEAN);
  float* acc = (float*)malloc(sizeof(float) * (size_t)(count > 0 ? count : 1));
  for (int64_t b = 0; b < num_bags; b++) {
    int64_t s, e;
    bag_range(sparse, offsets, key_bytes, b, hotness, &s, &e);
    for (int64_t i = 0; i < count; i++) acc[i] = 0.0f;
    float denom = 0.0f;
    for (int64_t k = s; k < e; k++) {
      const float w = weighted ? load_weight(weights, weight_dtype, k) : 1.0f;
      for (int64_t i = 0; i < count; i++) {
        const float x = elem_as_f32(dequant_elem(rows[k], dtype, count, i));
        acc[i] = weighted ? fmaf(x, w, acc[i]) : acc[i] + x;
      }
      if (mean) denom = denom + w;
    }
    if (mean) {
      for (int64_t i = 0; i < count; i++) acc[i] = (denom == 0.0f) ? 0.0f : acc[i] / denom;
    }
    store_out(out, out_stride, b, out_dtype, acc, count);
  }
  free(acc);
}

/* One element as the CPU HostLayer widens it to float (cpu_pooling.hpp:68-150
 * float/half, :166-259 and :302-341 quantized): float(x); quantized
 * float(q)*scale + offset taken as one fma (offset 0 for the int8 formats, f16
 * metadata widened first); the extension formats as dequant_elem. */
static float host_value(const uint8_t* row, int dtype, int64_t count, int64_t i) {
  switch (dtype) {
    case ORC_F32: return ld_f32(row + 4 * i);
    case ORC_F16: return orc_f16_to_f32(ld_u16(row + 2 * i));
    case ORC_QI8_F32: return fmaf((float)(int8_t)row[i], ld_f32(row + count), 0.0f);
    case ORC_QI8_F16: return fmaf((float)(int8_t)row[i], orc_f16_to_f32(ld_u16(row + count)), 0.0f);
    case ORC_QU8_F32: return fmaf((float)row[i], ld_f32(row + count), ld_f32(row + count + 4));
    case ORC_QU8_F16:
      return fmaf((float)row[i], orc_f16_to_f32(ld_u16(row + count)),
                  orc_f16_to_f32(ld_u16(row + count + 2)));
    default: return elem_as_f32(dequant_elem(row, dtype, count, i));
  }
}

/* cpu_kernel_concatenate / cpu_kernel_concatenate_quant (cpu_pooling.hpp:272-341):
 * one output row per input row, out = cast(host_value), rounded to nearest even
 * for an f16 output (no half rounding in between, unlike the GPU's f16-metadata
 * dequantize). */
void orc_convert_host(const uint8_t* row, int dtype, int64_t count, int out_dtype, void* out) {
  for (int64_t i = 0; i < count; i++) {
    const float v = host_value(row, dtype, count, i);
    if (out_dtype == ORC_F16)
      ((uint16_t*)out)[i] = orc_f32_to_f16(v);
    else
      ((float*)out)[i] = v;
  }
}

/* cpu_pooling.hpp:68-150 (float/half) and :166-259 (quantized): per bag,
 * v = float(x) [quantized: float(q)*scale + offset, taken as one fma];
 * weighted: v *= w; acc += v; Mean: acc * (1/denom); zero denom -> zero row. */
void orc_pool_host(const uint8_t* const* rows, int dtype, int64_t count, int sparse, int pooling,
                   int64_t num_keys, const void* offsets, int key_bytes, int64_t num_bags,
                   int64_t hotness, const void* weights, int weight_dtype, int out_dtype,
                   void* out, int64_t out_stride) {
  (void)num_keys;
  const int weighted = (pooling == ORC_WSUM || pooling == ORC_WMEAN);
  const int mean = (pooling == ORC_MEAN || pooling == ORC_WMEAN);
  float* acc = (float*)malloc(sizeof(float) * (size_t)(count > 0 ? count : 1));
  for (int64_t b = 0; b < num_bags; b++) {
    int64_t s, e;
    bag_range(sparse, offsets, key_bytes, b, hotness, &s, &e);
    uint8_t* orow = (uint8_t*)out + b * out_stride;
    if (e - s <= 0) {
      memset(orow, 0, (size_t)(count * (out_dtype == ORC_F16 ? 2 : 4)));
      continue;
    }
    for (int64_t i = 0; i < count; i++) acc[i] = 0.0f;
    float wsum = 0.0f;
    for (int64_t k = s; k < e; k++) {
      const float w = weighted ? load_weight(weights, weight_dtype, k) : 1.0f;
      wsum += w;
      const uint8_t* row = rows[k];
      for (int64_t i = 0; i < count; i++) {
        float v = host_value(row, dtype, count, i);
        if (weighted) v *= w;
        acc[i] += v;
      }
    }
    float inv = 1.0f;
    if (mean) {
      const float denom = weighted ? wsum : (float)(e - s);
      inv = (denom != 0.0f) ? 1.0f / denom : 0.0f;
    }
    for (int64_t i = 0; i < count; i++) acc[i] = acc[i] * inv;
    store_out(out, out_stride, b, out_dtype, acc, count);
  }
  free(acc);
}

/* ------------------------------------------------------------------------- */
/* threaded HostLayer lookup (host_embedding_layer.cpp:55-247,               */
/* linear_host_table.hpp:77-108, cpu_gather.hpp:28-80, layer_utils.cpp:331)  */
/* ------------------------------------------------------------------------- */

typedef struct {
  int task;
  int ntasks;
  const void* keys;
  int key_bytes;
  int64_t n;
  const uint8_t* table;
  uint64_t num_rows;
  int64_t row_bytes;
  uint8_t* gather_buf;
  /* pool */
  int dtype, pooling, sparse, weight_dtype, out_dtype;
  const void* offsets;
  int64_t num_bags, hotness, count, out_stride;
  const void* weights;
  void* out;
} host_task;

static void* host_gather_task(void* arg) {
  host_task* t = (host_task*)arg;
  /* keys per task rounded up to 64 (cpu_gather.hpp:37-40) */
  int64_t per = (t->n + t->ntasks - 1) / t->ntasks;
  per = (per + 63) / 64 * 64;
  const int64_t s = (int64_t)t->task * per;
  const int64_t e = (s + per < t->n) ? s + per : t->n;
  for (int64_t i = s; i < e; i++) {
    const int64_t k = load_key(t->keys, t->key_bytes, i);
    if (!orc_key_in_range(k, t->num_rows)) continue;
    memcpy(t->gather_buf + i * t->row_bytes, t->table + (uint64_t)k * (uint64_t)t->row_bytes,
           (size_t)t->row_bytes);
  }
  return NULL;
}

/* Pool bags [b0, b1) of the gathered buffer with cpu_pooling.hpp:68-150 order
 * (same arithmetic as orc_pool_host; a bag range per worker thread). */
static void pool_host_range(const host_task* t, const uint8_t* const* rows, int64_t b0,
                            int64_t b1) {
  const int weighted = (t->pooling == ORC_WSUM || t->pooling == ORC_WMEAN);
  const int mean = (t->pooling == ORC_MEAN || t->pooling == ORC_WMEAN);
  const int64_t count = t->count;
  float* acc = (float*)malloc(sizeof(float) * (size_t)(count > 0 ? count : 1));
  for (int64_t b = b0; b < b1; b++) {
    int64_t s, e;
    bag_range(t->sparse, t->offsets, t->key_bytes, b, t->hotness, &s, &e);
    uint8_t* orow = (uint8_t*)t->out + b * t->out_stride;
    if (e - s <= 0) {
      memset(orow, 0, (size_t)(count * (t->out_dtype == ORC_F16 ? 2 : 4)));
      continue;
    }
    for (int64_t i = 0; i < count; i++) acc[i] = 0.0f;
    float wsum = 0.0f;
    for (int64_t k = s; k < e; k++) {
      const float w = weighted ? load_weight(t->weights, t->weight_dtype, k) : 1.0f;
      wsum += w;
      const uint8_t* row = rows[k];
      if (t->dtype == ORC_F16 && !weighted) {
        const uint16_t* hr = (const uint16_t*)row;
        for (int64_t i = 0; i < count; i++) acc[i] += orc_f16_to_f32(hr[i]);
      } else if (t->dtype == ORC_F32 && !weighted) {
        const float* fr = (const float*)row;
        for (int64_t i = 0; i < count; i++) acc[i] += fr[i];
      } else {
        for (int64_t i = 0; i < count; i++) {
          float v;
          if (t->dtype == ORC_F32)
            v = ld_f32(row + 4 * i);
          else if (t->dtype == ORC_F16)
            v = orc_f16_to_f32(ld_u16(row + 2 * i));
          else
            v = elem_as_f32(dequant_elem(row, t->dtype, count, i));
          if (weighted) v *= w;
          acc[i] += v;
        }
      }
    }
    float inv = 1.0f;
    if (mean) {
      const float denom = weighted ? wsum : (float)(e - s);
      inv = (denom != 0.0f) ? 1.0f / denom : 0.0f;
    }
    for (int64_t i = 0; i < count; i++) acc[i] = acc[i] * inv;
    store_out(t->out, t->out_stride, b, t->out_dtype, acc, count);
  }
  free(acc);
}

static void* host_pool_task2(void* arg) {
  host_task* t = (host_task*)arg;
  int64_t per = (t->num_bags + t->ntasks - 1) / t->ntasks;
  if (per < 1) per = 1;
  const int64_t s = (int64_t)t->task * per;
  if (s >= t->num_bags) return NULL;
  const int64_t e = (s + per < t->num_bags) ? s + per : t->num_bags;
  const int64_t nk = t->n;
  const uint8_t** rows = (const uint8_t**)malloc(sizeof(uint8_t*) * (size_t)(nk > 0 ? nk : 1));
  for (int64_t i = 0; i < nk; i++) rows[i] = t->gather_buf + i * t->row_bytes;
  pool_host_range(t, rows, s, e);
  free(rows);
  return NULL;
}

static void run_tasks(host_task* base, int threads, void* (*fn)(void*)) {
  pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)threads);
  host_task* ts = (host_task*)malloc(sizeof(host_task) * (size_t)threads);
  for (int i = 0; i < threads; i++) {
    ts[i] = *base;
    ts[i].task = i;
    ts[i].ntasks = threads;
  }
  for (int i = 1; i < threads; i++) pthread_create(&th[i], NULL, fn, &ts[i]);
  fn(&ts[0]);
  for (int i = 1; i < threads; i++) pthread_join(th[i], NULL);
  free(ts);
  free(th);
}

void orc_host_layer_lookup(const void* keys, int key_bytes, int64_t n, const uint8_t* table,
                           uint64_t num_rows, int64_t row_bytes, int dtype, int pooling,
                           int sparse, const void* offsets, int64_t num_bags, int64_t hotness,
                           const void* weights, int weight_dtype, int out_dtype,
                           uint8_t* gather_buf, void* out, int64_t out_stride, int threads) {
  if (threads < 1) threads = 1;
  host_task t;
  memset(&t, 0, sizeof(t));
  t.keys = keys;
  t.key_bytes = key_bytes;
  t.n = n;
  t.table = table;
  t.num_rows = num_rows;
  t.row_bytes = row_bytes;
  t.dtype = dtype;
  t.pooling = pooling;
  t.sparse = sparse;
  t.offsets = offsets;
  t.num_bags = num_bags;
  t.hotness = hotness;
  t.weights = weights;
  t.weight_dtype = weight_dtype;
  t.out_dtype = out_dtype;
  t.out = out;
  t.out_stride = out_stride;
  const int64_t meta = orc_meta_bytes(dtype);
  t.count = (row_bytes - meta) / orc_value_bytes(dtype);
  if (pooling == ORC_CONCAT) {
    t.gather_buf = (uint8_t*)out; /* gather straight into the output (stride == row) */
    run_tasks(&t, threads, host_gather_task);
    return;
  }
  t.gather_buf = gather_buf;
  run_tasks(&t, threads, host_gather_task);
  run_tasks(&t, threads, host_pool_task2);
}

/* ------------------------------------------------------------------------- */
/* set-associative cache                                                     */
/* ------------------------------------------------------------------------- */

#define ORC_WAYS 8

static uint64_t align16(uint64_t x) { return (x + 15) / 16 * 16; }

/* ec_set_associative.h:667-685 + ec_set_associative_device_modify.cuh:472-474:
 * per set: align16(8*sizeof(Tag)) + align16(8*row) + align16(8*sizeof(float)). */
uint64_t orc_cache_num_sets(uint64_t cache_bytes, int64_t row_bytes, int key_bytes) {
  const uint64_t per = align16((uint64_t)key_bytes * ORC_WAYS) +
                       align16((uint64_t)row_bytes * ORC_WAYS) + align16(4 * ORC_WAYS);
  return cache_bytes / per;
}

/* ec_set_associative.h:677-683 with get_counter_size_per_set() == 0: the
 * host-metadata cache keeps its counters in host memory. */
uint64_t orc_cache_num_sets_host(uint64_t cache_bytes, int64_t row_bytes, int key_bytes) {
  const uint64_t per = align16((uint64_t)key_bytes * ORC_WAYS) + align16((uint64_t)row_bytes * ORC_WAYS);
  return cache_bytes / per;
}

int orc_cache_init(orc_cache* c, uint64_t cache_bytes, int64_t row_bytes, int key_bytes,
                   int64_t sentinel) {
  return orc_cache_init_ex(c, cache_bytes, row_bytes, key_bytes, sentinel, 0);
}

int orc_cache_init_ex(orc_cache* c, uint64_t cache_bytes, int64_t row_bytes, int key_bytes,
                      int64_t sentinel, int host_modify) {
  memset(c, 0, sizeof(*c));
  c->host_modify = host_modify ? 1 : 0;
  c->num_sets = host_modify ? orc_cache_num_sets_host(cache_bytes, row_bytes, key_bytes)
                            : orc_cache_num_sets(cache_bytes, row_bytes, key_bytes);
  if (c->num_sets == 0) return -1;
  c->row_bytes = row_bytes;
  c->key_bytes = key_bytes;
  c->sentinel = (key_bytes == 4) ? (int64_t)(int32_t)sentinel : sentinel;
  c->decay_rate = 0.95f; /* ec_set_associative.h:120 */
  c->global_ts = 0;
  const uint64_t ways = c->num_sets * ORC_WAYS;
  c->data = (uint8_t*)calloc(ways, (size_t)row_bytes);
  c->tags = (int64_t*)malloc(sizeof(int64_t) * ways);
  c->counters = (float*)calloc(ways, sizeof(float));
  c->set_ts = (int64_t*)calloc(c->num_sets, sizeof(int64_t));
  if (!c->data || !c->tags || !c->counters || !c->set_ts) return -2;
  for (uint64_t i = 0; i < ways; i++) c->tags[i] = c->sentinel;
  return 0;
}

void orc_cache_free(orc_cache* c) {
  free(c->data);
  free(c->tags);
  free(c->counters);
  free(c->set_ts);
  memset(c, 0, sizeof(*c));
}

/* ec_hash.h:36-60: arithmetic in the unsigned counterpart of the key type. */
uint32_t orc_cache_set(const orc_cache* c, int64_t key) {
  if (c->key_bytes == 4) return (uint32_t)((uint32_t)(int32_t)key % (uint32_t)c->num_sets);
  return (uint32_t)((uint64_t)key % c->num_sets);
}

int64_t orc_cache_tag(const orc_cache* c, int64_t key) {
  if (c->key_bytes == 4) return (int64_t)(int32_t)((uint32_t)(int32_t)key / (uint32_t)c->num_sets);
  return (int64_t)((uint64_t)key / c->num_sets);
}

int64_t orc_cache_key_of(const orc_cache* c, int64_t tag, uint32_t set) {
  if (c->key_bytes == 4)
    return (int64_t)(int32_t)((uint32_t)(int32_t)tag * (uint32_t)c->num_sets + set);
  return (int64_t)((uint64_t)tag * c->num_sets + set);
}

/* ec_set_associative.cuh:46-80: compare the rebuilt key of all 8 ways, the
 * lowest matching way wins (__ffs). */
int orc_cache_find_way(const orc_cache* c, int64_t key) {
  if (c->key_bytes == 4) key = (int64_t)(int32_t)key;
  const uint32_t set = orc_cache_set(c, key);
  for (int w = 0; w < ORC_WAYS; w++) {
    if (orc_cache_key_of(c, c->tags[(uint64_t)set * ORC_WAYS + w], set) == key) return w;
  }
  return -1;
}

int64_t orc_cache_resolve(const orc_cache* c, const void* keys, int64_t n, const uint8_t* uvm,
                          const uint8_t** rows, uint64_t* hit_bits) {
  int64_t misses = 0;
  for (int64_t i = 0; i < n; i++) {
    const int64_t k = load_key(keys, c->key_bytes, i);
    const int w = orc_cache_find_way(c, k);
    if (w >= 0) {
      const uint32_t set = orc_cache_set(c, k);
      rows[i] = c->data + ((uint64_t)set * ORC_WAYS + (uint64_t)w) * (uint64_t)c->row_bytes;
      if (hit_bits) hit_bits[i / 64] |= 1ull << (i % 64);
    } else {
      rows[i] = uvm ? uvm + (uint64_t)k * (uint64_t)c->row_bytes : NULL;
      misses++;
    }
  }
  return misses;
}

/* ------------------------------------------------------------------------- */
/* histogram (gather_keys_data_ptrs.cuh:121-191)                             */
/* ------------------------------------------------------------------------- */

typedef struct {
  int64_t key;
  int64_t idx;
} kv_pair;

static int cmp_key_idx(const void* a, const void* b) {
  const kv_pair* x = (const kv_pair*)a;
  const kv_pair* y = (const kv_pair*)b;
  if (x->key != y->key) return x->key < y->key ? -1 : 1;
  return x->idx < y->idx ? -1 : (x->idx > y->idx);
}

typedef struct {
  int64_t count;
  int64_t key;
  int64_t first;
} hist_entry;

static int cmp_hist(const void* a, const void* b) {
  const hist_entry* x = (const hist_entry*)a;
  const hist_entry* y = (const hist_entry*)b;
  if (x->count != y->count) return x->count > y->count ? -1 : 1; /* count descending */
  return x->key < y->key ? -1 : (x->key > y->key);                /* then ascending key */
}

int64_t orc_histogram(const void* keys, int key_bytes, int64_t n, int64_t* ukeys,
                      float* priority, int64_t* first_idx) {
  if (n <= 0) return 0;
  kv_pair* p = (kv_pair*)malloc(sizeof(kv_pair) * (size_t)n);
  for (int64_t i = 0; i < n; i++) {
    p[i].key = load_key(keys, key_bytes, i);
    p[i].idx = i;
  }
  qsort(p, (size_t)n, sizeof(kv_pair), cmp_key_idx); /* (key, idx): a stable key sort */
  hist_entry* h = (hist_entry*)malloc(sizeof(hist_entry) * (size_t)n);
  int64_t u = 0;
  for (int64_t i = 0; i < n; i++) {
    if (i == 0 || p[i].key != p[i - 1].key) {
      h[u].key = p[i].key;
      h[u].first = p[i].idx;
      h[u].count = 0;
      u++;
    }
    h[u - 1].count++;
  }
  qsort(h, (size_t)u, sizeof(hist_entry), cmp_hist);
  const float norm = 1.0f / (float)n;
  for (int64_t i = 0; i < u; i++) {
    ukeys[i] = h[i].key;
    priority[i] = (float)(int32_t)h[i].count * norm;
    first_idx[i] = h[i].first;
  }
  free(h);
  free(p);
  return u;
}

/* ------------------------------------------------------------------------- */
/* replacement policy (ec_set_associative_modify.cuh:36-103,139-297)         */
/* ------------------------------------------------------------------------- */

/* SortBlock (:36-71): bitonic network over 8 lanes; a lane swaps with its
 * partner only when the values differ.  Ends in descending order. */
static void sort_block(float* v, uint32_t* pos) {
  for (uint32_t k = 2; k <= ORC_WAYS; k *= 2) {
    for (uint32_t j = k / 2; j > 0; j /= 2) {
      float nv[ORC_WAYS];
      uint32_t np[ORC_WAYS];
      for (uint32_t x = 0; x < ORC_WAYS; x++) {
        const uint32_t p = x ^ j;
        nv[x] = v[x];
        np[x] = pos[x];
        if (v[x] != v[p]) {
          const int in_order_pos = x > p;
          const int in_order_val = v[x] > v[p];
          const int swap = (x & k) ? (in_order_pos != in_order_val) : (in_order_pos == in_order_val);
          if (swap) {
            nv[x] = v[p];
            np[x] = pos[p];
          }
        }
      }
      memcpy(v, nv, sizeof(nv));
      memcpy(pos, np, sizeof(np));
    }
  }
}

/* MergeBlock (:73-103): take the partner-reversed second list where strictly
 * larger, then a bitonic clean-up with no equality guard (equal values make
 * the lower lane copy its partner -- reproduced as is). The reversed position
 * travels through a float in the reference; exact below 2^24. */
static void merge_block(float* p1, uint32_t* pos1, const float* p2, const uint32_t* pos2) {
  float rp[ORC_WAYS];
  uint32_t rpos[ORC_WAYS];
  for (uint32_t x = 0; x < ORC_WAYS; x++) {
    rp[x] = p2[ORC_WAYS - 1 - x];
    rpos[x] = (uint32_t)(float)pos2[ORC_WAYS - 1 - x];
  }
  for (uint32_t x = 0; x < ORC_WAYS; x++) {
    if (rp[x] > p1[x]) {
      p1[x] = rp[x];
      pos1[x] = rpos[x];
    }
  }
  for (uint32_t j = ORC_WAYS / 2; j > 0; j /= 2) {
    float nv[ORC_WAYS];
    uint32_t np[ORC_WAYS];
    for (uint32_t x = 0; x < ORC_WAYS; x++) {
      const uint32_t p = x ^ j;
      nv[x] = p1[x];
      np[x] = pos1[x];
      const int in_order_pos = x < p;
      const int in_order_val = p1[x] > p1[p];
      if (in_order_pos != in_order_val) {
        nv[x] = p1[p];
        np[x] = pos1[p];
      }
    }
    memcpy(p1, nv, sizeof(nv));
    memcpy(pos1, np, sizeof(np));
  }
}

typedef struct {
  uint32_t set;
  int64_t idx;
} set_pair;

static int cmp_set_pair(const void* a, const void* b) {
  const set_pair* x = (const set_pair*)a;
  const set_pair* y = (const set_pair*)b;
  if (x->set != y->set) return x->set < y->set ? -1 : 1;
  return x->idx < y->idx ? -1 : (x->idx > y->idx);
}

/* Lane-exact model of SetReplaceDataKernel for one set.  cand[] holds the
 * histogram indices mapped to this set, ascending. */
static int64_t replace_one_set(orc_cache* c, uint32_t set, const int64_t* cand, int64_t count,
                               const int64_t* ukeys, const float* priority,
                               const uint8_t* const* src_rows, int64_t* out_set, int64_t* out_way,
                               int64_t n_out, uint8_t** copy_dst, const uint8_t** copy_src,
                               int64_t* new_tags, uint32_t* new_way) {
  int64_t* tags = c->tags + (uint64_t)set * ORC_WAYS;
  float* ctr = c->counters + (uint64_t)set * ORC_WAYS;

  /* lazy decay (:172-183): delta = ts - set_ts; factor defined as
   * (float)pow((double)rate, (double)delta) -- the reference's __powf bits are
   * not published, so this part is parity-unpinned. */
  const int64_t delta = c->global_ts - c->set_ts[set];
  if (delta > 0 && c->decay_rate != 1.0f) {
    const float f = (float)pow((double)c->decay_rate, (double)delta);
    for (int x = 0; x < ORC_WAYS; x++) ctr[x] *= f;
  }
  c->set_ts[set] = c->global_ts;

  const uint32_t num_repl = (uint32_t)(count < ORC_WAYS ? count : ORC_WAYS);
  float hp[ORC_WAYS];
  uint32_t pos[ORC_WAYS];
  int64_t processed = 0;
  int first = 1;
  while (first || processed < count) {
    float hp2[ORC_WAYS];
    uint32_t pos2[ORC_WAYS];
    for (int x = 0; x < ORC_WAYS; x++) {
      hp2[x] = 0.0f;
      pos2[x] = 0;
      if (processed + x < count) {
        const int64_t loc = cand[processed + x];
        const int64_t key = ukeys[loc];
        int hit = 0;
        for (int w = 0; w < ORC_WAYS; w++) {
          if (orc_cache_key_of(c, tags[w], set) == key) {
            ctr[w] += priority[loc];
            hit = 1;
          }
        }
        /* a candidate without a source row (a key outside the backing table
         * of insert_from_uvm) is not inserted; a resident one still gains */
        if (!hit && (src_rows == NULL || src_rows[loc] != NULL)) {
          pos2[x] = (uint32_t)loc;
          hp2[x] = priority[loc];
        }
      }
    }
    sort_block(hp2, pos2);
    if (first) {
      memcpy(hp, hp2, sizeof(hp));
      memcpy(pos, pos2, sizeof(pos));
      first = 0;
    } else {
      merge_block(hp, pos, hp2, pos2);
    }
    processed += ORC_WAYS;
  }

  /* order the ways by counter (empty ways count 0), ascending after the reversal */
  float cv[ORC_WAYS];
  uint32_t dpos[ORC_WAYS];
  for (int x = 0; x < ORC_WAYS; x++) {
    dpos[x] = (uint32_t)x;
    cv[x] = (tags[x] == c->sentinel) ? 0.0f : ctr[x];
  }
  sort_block(cv, dpos);
  float rc[ORC_WAYS];
  uint32_t rd[ORC_WAYS];
  for (int x = 0; x < ORC_WAYS; x++) {
    rc[x] = cv[ORC_WAYS - 1 - x];
    rd[x] = dpos[ORC_WAYS - 1 - x];
  }
  int64_t written = 0;
  for (uint32_t x = 0; x < num_repl; x++) {
    if (hp[x] > rc[x]) {
      const int64_t key = ukeys[pos[x]];
      const uint32_t way = rd[x];
      const int64_t k = n_out + written;
      if (out_set) out_set[k] = set;
      if (out_way) out_way[k] = way;
      copy_dst[k] = c->data + ((uint64_t)set * ORC_WAYS + way) * (uint64_t)c->row_bytes;
      copy_src[k] = src_rows[pos[x]];
      new_tags[k] = orc_cache_tag(c, key);
      new_way[k] = (uint32_t)((uint64_t)set * ORC_WAYS + way);
      ctr[way] = hp[x];
      written++;
    }
  }
  return written;
}

int64_t orc_cache_insert_hist(orc_cache* c, const int64_t* ukeys, const float* priority,
                              const uint8_t* const* src_rows, int64_t m, int64_t* out_set,
                              int64_t* out_way) {
  if (m <= 0) return 0;
  c->global_ts++; /* ++global_ts_ per insert (ec_set_associative_device_modify.cuh:262) */
  set_pair* sp = (set_pair*)malloc(sizeof(set_pair) * (size_t)m);
  for (int64_t i = 0; i < m; i++) {
    sp[i].set = orc_cache_set(c, ukeys[i]);
    sp[i].idx = i;
  }
  qsort(sp, (size_t)m, sizeof(set_pair), cmp_set_pair); /* stable sort by set */
  int64_t* cand = (int64_t*)malloc(sizeof(int64_t) * (size_t)m);
  for (int64_t i = 0; i < m; i++) cand[i] = sp[i].idx;
  /* each candidate yields at most one record per lane; a set yields <= 8 */
  const int64_t cap = m * 2 + 8;
  uint8_t** dst = (uint8_t**)malloc(sizeof(uint8_t*) * (size_t)cap);
  const uint8_t** src = (const uint8_t**)malloc(sizeof(uint8_t*) * (size_t)cap);
  int64_t* ntag = (int64_t*)malloc(sizeof(int64_t) * (size_t)cap);
  uint32_t* nway = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)cap);
  int64_t n_out = 0;
  int64_t i = 0;
  while (i < m) {
    int64_t j = i;
    while (j < m && sp[j].set == sp[i].set) j++;
    n_out += replace_one_set(c, sp[i].set, cand + i, j - i, ukeys, priority, src_rows, out_set,
                             out_way, n_out, dst, src, ntag, nway);
    i = j;
  }
  /* invalidate -> copy rows -> commit tags (ec_set_associative_device_modify.cuh:275-280) */
  for (int64_t k = 0; k < n_out; k++) memcpy(dst[k], src[k], (size_t)c->row_bytes);
  for (int64_t k = 0; k < n_out; k++) c->tags[nway[k]] = ntag[k];
  free(nway);
  free(ntag);
  free(src);
  free(dst);
  free(cand);
  free(sp);
  return n_out;
}

int64_t orc_cache_insert_keys(orc_cache* c, const void* keys, int64_t n, const uint8_t* uvm,
                              uint64_t uvm_rows, const uint8_t* values, int64_t value_stride,
                              int64_t max_modify_size) {
  if (n <= 0) return 0;
  int64_t* uk = (int64_t*)malloc(sizeof(int64_t) * (size_t)n);
  float* pr = (float*)malloc(sizeof(float) * (size_t)n);
  int64_t* fi = (int64_t*)malloc(sizeof(int64_t) * (size_t)n);
  int64_t u = orc_histogram(keys, c->key_bytes, n, uk, pr, fi);
  const int64_t m = (u < max_modify_size) ? u : max_modify_size;
  const uint8_t** rows = (const uint8_t**)malloc(sizeof(uint8_t*) * (size_t)(m > 0 ? m : 1));
  for (int64_t i = 0; i < m; i++) {
    if (uvm)
      rows[i] = (uint64_t)uk[i] < uvm_rows ? uvm + (uint64_t)uk[i] * (uint64_t)c->row_bytes : NULL;
    else
      rows[i] = values + fi[i] * value_stride;
  }
  const int64_t r = orc_cache_insert_hist(c, uk, pr, rows, m, NULL, NULL);
  free(rows);
  free(fi);
  free(pr);
  free(uk);
  return r;
}

/* SetUpdateDataKernel<invalidate_only> (ec_set_associative_modify.cuh:516-561) */
int64_t orc_cache_erase(orc_cache* c, const void* keys, int64_t n) {
  int64_t cnt = 0;
  for (int64_t i = 0; i < n; i++) {
    int64_t k = load_key(keys, c->key_bytes, i);
    const uint32_t set = orc_cache_set(c, k);
    for (int w = 0; w < ORC_WAYS; w++) {
      int64_t* t = &c->tags[(uint64_t)set * ORC_WAYS + w];
      if (orc_cache_key_of(c, *t, set) == k) {
        *t = c->sentinel;
        cnt++;
      }
    }
  }
  return cnt;
}

void orc_cache_clear(orc_cache* c) {
  const uint64_t ways = c->num_sets * ORC_WAYS;
  for (uint64_t i = 0; i < ways; i++) c->tags[i] = c->sentinel;
  if (c->host_modify) memset(c->counters, 0, sizeof(float) * ways);
  memset(c->set_ts, 0, sizeof(int64_t) * c->num_sets);
  c->global_ts = 0;
}

/* ------------------------------------------------------------------------- */
/* host-metadata insert (modify_on_gpu = false)                              */
/* ------------------------------------------------------------------------- */

typedef struct {
  int64_t key;
  int64_t first; /* first position, also the bin's creation order */
  int64_t count;
} host_bin;

static int cmp_host_bin_key(const void* a, const void* b) {
  const host_bin* x = (const host_bin*)a;
  const host_bin* y = (const host_bin*)b;
  if (x->key != y->key) return x->key < y->key ? -1 : 1;
  return x->first < y->first ? -1 : (x->first > y->first);
}

/* count descending; equal counts in order of first occurrence */
static int cmp_host_bin_count(const void* a, const void* b) {
  const host_bin* x = (const host_bin*)a;
  const host_bin* y = (const host_bin*)b;
  if (x->count != y->count) return x->count > y->count ? -1 : 1;
  return x->first < y->first ? -1 : (x->first > y->first);
}

/* embed_cache.h:199-229 */
int64_t orc_histogram_host(const void* keys, int key_bytes, int64_t n, int64_t* ukeys,
                           float* priority, int64_t* first_idx) {
  if (n <= 0) return 0;
  host_bin* b = (host_bin*)malloc(sizeof(host_bin) * (size_t)n);
  for (int64_t i = 0; i < n; i++) {
    b[i].key = load_key(keys, key_bytes, i);
    b[i].first = i;
    b[i].count = 1;
  }
  qsort(b, (size_t)n, sizeof(host_bin), cmp_host_bin_key);
  int64_t u = 0;
  for (int64_t i = 0; i < n; i++) {
    if (u > 0 && b[u - 1].key == b[i].key) {
      b[u - 1].count++; /* the bin keeps its first position */
    } else {
      b[u++] = b[i];
    }
  }
  qsort(b, (size_t)u, sizeof(host_bin), cmp_host_bin_count);
  for (int64_t i = 0; i < u; i++) {
    ukeys[i] = b[i].key;
    priority[i] = (float)b[i].count / (float)n; /* Bin::count is a float counting by 1 */
    first_idx[i] = b[i].first;
  }
  free(b);
  return u;
}

/* ec_set_associative_host_modify.h:218-296 plus modify() (:428-480): the tags
 * and counters change on the host as candidates are visited; the recorded
 * ways then get their rows copied and their tags committed. */
int64_t orc_cache_insert_host(orc_cache* c, const int64_t* ukeys, const float* priority,
                              const uint8_t* const* src_rows, int64_t m, int64_t max_update,
                              int64_t* out_set, int64_t* out_way) {
  const int64_t now = ++c->global_ts; /* advanced once per insert call */
  const uint64_t ways = c->num_sets * ORC_WAYS;
  /* one record per (set, way) in this call: the reference's insertMap */
  int64_t* rec_of_slot = (int64_t*)malloc(sizeof(int64_t) * ways);
  for (uint64_t i = 0; i < ways; i++) rec_of_slot[i] = -1;
  int64_t cap = max_update < m ? max_update : m;
  if (cap < 1) cap = 1;
  uint64_t* rslot = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)cap);
  const uint8_t** rsrc = (const uint8_t**)malloc(sizeof(uint8_t*) * (size_t)cap);
  int64_t nrec = 0;
  for (int64_t i = 0; i < m && nrec < max_update; i++) {
    int64_t key = ukeys[i];
    if (c->key_bytes == 4) key = (int64_t)(int32_t)key;
    const uint32_t set = orc_cache_set(c, key);
    int64_t* st = c->tags + (uint64_t)set * ORC_WAYS;
    float* sc = c->counters + (uint64_t)set * ORC_WAYS;
    if (c->set_ts[set] != now) {
      const int64_t delta = now - c->set_ts[set];
      const float f = (float)pow((double)c->decay_rate, (double)delta);
      for (int w = 0; w < ORC_WAYS; w++) sc[w] *= f;
      c->set_ts[set] = now;
    }
    int hit = 0;
    for (int w = 0; w < ORC_WAYS; w++) {
      if (orc_cache_key_of(c, st[w], set) == key) {
        sc[w] += priority[i];
        hit = 1;
        break;
      }
    }
    if (hit) continue;
    /* a key outside the backing table of insert_from_uvm has no source row:
     * it is not a candidate */
    if (src_rows != NULL && src_rows[i] == NULL) continue;
    int wmin = 0; /* std::min_element: the first smallest counter */
    for (int w = 1; w < ORC_WAYS; w++)
      if (sc[w] < sc[wmin]) wmin = w;
    if (sc[wmin] > priority[i]) continue;
    const uint64_t slot = (uint64_t)set * ORC_WAYS + (uint64_t)wmin;
    if (rec_of_slot[slot] >= 0) continue;
    sc[wmin] = priority[i];
    st[wmin] = orc_cache_tag(c, key);
    rec_of_slot[slot] = nrec;
    rslot[nrec] = slot;
    rsrc[nrec] = src_rows ? src_rows[i] : NULL;
    nrec++;
  }
  for (int64_t r = 0; r < nrec; r++) {
    if (rsrc[r])
      memcpy(c->data + rslot[r] * (uint64_t)c->row_bytes, rsrc[r], (size_t)c->row_bytes);
    if (out_set) out_set[r] = (int64_t)(rslot[r] / ORC_WAYS);
    if (out_way) out_way[r] = (int64_t)(rslot[r] % ORC_WAYS);
  }
  free(rsrc);
  free(rslot);
  free(rec_of_slot);
  return nrec;
}

int64_t orc_cache_insert_keys_host(orc_cache* c, const void* keys, int64_t n, const uint8_t* uvm,
                                   uint64_t uvm_rows, const uint8_t* values, int64_t value_stride,
                                   int64_t max_modify_size) {
  if (n <= 0) return 0;
  int64_t* uk = (int64_t*)malloc(sizeof(int64_t) * (size_t)n);
  float* pr = (float*)malloc(sizeof(float) * (size_t)n);
  int64_t* fi = (int64_t*)malloc(sizeof(int64_t) * (size_t)n);
  const int64_t u = orc_histogram_host(keys, c->key_bytes, n, uk, pr, fi);
  const uint8_t** rows = (const uint8_t**)malloc(sizeof(uint8_t*) * (size_t)u);
  for (int64_t i = 0; i < u; i++) {
    if (uvm)
      rows[i] = (uint64_t)uk[i] < uvm_rows ? uvm + (uint64_t)uk[i] * (uint64_t)c->row_bytes : NULL;
    else
      rows[i] = values + fi[i] * value_stride;
  }
  const int64_t r = orc_cache_insert_host(c, uk, pr, rows, u, max_modify_size, NULL, NULL);
  free(rows);
  free(fi);
  free(pr);
  free(uk);
  return r;
}

/* ------------------------------------------------------------------------- */
/* training backprop (gradient_calculator.cuh:238-301, dedup_grads_kernel.cuh)*/
/* ------------------------------------------------------------------------- */

static float load_f(const void* p, int dtype, int64_t i) {
  return dtype == ORC_F16 ? orc_f16_to_f32(((const uint16_t*)p)[i]) : ((const float*)p)[i];
}

/* bag holding position p: p / hotness (Fixed), else the b with
 * offsets[b] <= p < offsets[b+1] found by binary search; -1 for none */
static int64_t bag_of_pos(int64_t p, int sparse, const void* offsets, int key_bytes,
                          int64_t num_bags, int64_t hotness) {
  if (sparse == ORC_FIXED) {
    const int64_t b = hotness > 0 ? p / hotness : -1;
    return (b >= 0 && b < num_bags) ? b : -1;
  }
  int64_t lo = 0, hi = num_bags; /* largest b in [0, num_bags) with offsets[b] <= p */
  if (num_bags <= 0 || load_key(offsets, key_bytes, 0) > p) return -1;
  while (hi - lo > 1) {
    const int64_t mid = (lo + hi) / 2;
    if (load_key(offsets, key_bytes, mid) <= p) lo = mid; else hi = mid;
  }
  return p < load_key(offsets, key_bytes, lo + 1) ? lo : -1;
}

#define PIECE_FAN_IN 8 /* sub-sequences of a key's pieces */

int64_t orc_pooling_backprop(const void* keys, int key_bytes, int64_t n, int pooling, int sparse,
                             const void* offsets, int64_t num_bags, int64_t hotness,
                             const void* weights, int weight_dtype, const void* grads_in,
                             int grad_dtype, int64_t dim, int64_t block, void* unique_out,
                             void* grads_out) {
  if (n <= 0) return 0;
  if (block < 1) block = 1;
  int64_t* uq = (int64_t*)malloc(sizeof(int64_t) * (size_t)n);
  int64_t* ct = (int64_t*)malloc(sizeof(int64_t) * (size_t)n);
  int64_t* inv = (int64_t*)malloc(sizeof(int64_t) * (size_t)n);
  int64_t* off = (int64_t*)malloc(sizeof(int64_t) * (size_t)n);
  const int64_t u = orc_dedup(keys, key_bytes, n, uq, ct, inv, off);
  const int concat = pooling == ORC_CONCAT;
  const int weighted = pooling == ORC_WSUM || pooling == ORC_WMEAN;
  const int normalized = pooling == ORC_MEAN || pooling == ORC_WMEAN;
  float* denom = NULL;
  if (!concat && normalized) {
    denom = (float*)calloc((size_t)(num_bags > 0 ? num_bags : 1), sizeof(float));
    for (int64_t b = 0; b < num_bags; b++) {
      int64_t s, e;
      if (sparse == ORC_FIXED) {
        s = b * hotness;
        e = s + hotness;
      } else {
        s = load_key(offsets, key_bytes, b);
        e = load_key(offsets, key_bytes, b + 1);
      }
      if (pooling == ORC_MEAN) {
        denom[b] = (float)(e - s);
      } else {
        float acc = 0.0f;
        for (int64_t p = s; p < e; p++) acc += load_f(weights, weight_dtype, p);
        denom[b] = acc;
      }
    }
  }
  float* part = (float*)malloc(sizeof(float) * (size_t)dim);
  float* quarter = (float*)malloc(sizeof(float) * (size_t)dim);
  float* tot = (float*)malloc(sizeof(float) * (size_t)dim);
  for (int64_t k = 0; k < u; k++) {
    /* pieces: key k's positions [d, e) of the dedup order cut at multiples of block */
    const int64_t d = off[k], e = off[k] + ct[k];
    const int64_t first_block = d / block;
    const int64_t pieces = (e - 1) / block - first_block + 1;
    const int64_t per_part = (pieces + PIECE_FAN_IN - 1) / PIECE_FAN_IN;
    for (int64_t c = 0; c < dim; c++) tot[c] = 0.0f;
    for (int64_t q = 0; q < PIECE_FAN_IN; q++) {
      for (int64_t c = 0; c < dim; c++) quarter[c] = 0.0f;
      const int64_t j_end = (q + 1) * per_part < pieces ? (q + 1) * per_part : pieces;
      for (int64_t j = q * per_part; j < j_end; j++) {
        const int64_t b_lo = (first_block + j) * block, b_hi = b_lo + block;
        const int64_t ps = d > b_lo ? d : b_lo, pe = e < b_hi ? e : b_hi;
        for (int64_t c = 0; c < dim; c++) part[c] = 0.0f;
        for (int64_t pos = ps; pos < pe; pos++) {
          const int64_t p = inv[pos];
          int64_t row;
          float w = 1.0f;
          if (concat) {
            row = p;
          } else {
            row = bag_of_pos(p, sparse, offsets, key_bytes, num_bags, hotness);
            if (row < 0) continue; /* a position in no bag adds nothing */
            if (weighted) w = load_f(weights, weight_dtype, p);
            if (normalized) w = (pooling == ORC_MEAN ? 1.0f : w) / denom[row];
          }
          for (int64_t c = 0; c < dim; c++) {
            const float g = load_f(grads_in, grad_dtype, row * dim + c);
            part[c] = (concat || pooling == ORC_SUM) ? part[c] + g : fmaf(g, w, part[c]);
          }
        }
        for (int64_t c = 0; c < dim; c++) quarter[c] = quarter[c] + part[c];
      }
      for (int64_t c = 0; c < dim; c++) tot[c] = tot[c] + quarter[c];
    }
    for (int64_t c = 0; c < dim; c++) {
      if (grad_dtype == ORC_F16)
        ((uint16_t*)grads_out)[k * dim + c] = orc_f32_to_f16(tot[c]);
      else
        ((float*)grads_out)[k * dim + c] = tot[c];
    }
    if (key_bytes == 4)
      ((int32_t*)unique_out)[k] = (int32_t)uq[k];
    else
      ((int64_t*)unique_out)[k] = uq[k];
  }
  free(tot);
  free(quarter);
  free(part);
  free(denom);
  free(off);
  free(inv);
  free(ct);
  free(uq);
  return u;
}

/* ------------------------------------------------------------------------- */
/* dedup (deduper.cuh:136-221)                                               */
/* ------------------------------------------------------------------------- */

int64_t orc_dedup(const void* keys, int key_bytes, int64_t n, int64_t* unique, int64_t* counts,
                  int64_t* inverse, int64_t* offsets) {
  if (n <= 0) return 0;
  kv_pair* p = (kv_pair*)malloc(sizeof(kv_pair) * (size_t)n);
  for (int64_t i = 0; i < n; i++) {
    p[i].key = load_key(keys, key_bytes, i);
    p[i].idx = i;
  }
  qsort(p, (size_t)n, sizeof(kv_pair), cmp_key_idx);
  int64_t u = 0;
  for (int64_t i = 0; i < n; i++) {
    inverse[i] = p[i].idx;
    if (i == 0 || p[i].key != p[i - 1].key) {
      unique[u] = p[i].key;
      offsets[u] = i;
      counts[u] = 0;
      u++;
    }
    counts[u - 1]++;
  }
  free(p);
  return u;
}

/* ------------------------------------------------------------------------- */
/* key generator                                                             */
/* ------------------------------------------------------------------------- */

/* pytorch_samples_common.py:21-28 (translateToPowerLaw): gamma is a float32
 * tensor, so max^gamma, min^gamma and 1/gamma are float32 values; the affine
 * map and the final pow run in float64; y >= max clamps to max-1; the int64
 * cast truncates. */
void orc_power_law(const double* x, int64_t n, double min_v, double max_v, double alpha,
                   int64_t* out) {
  const float g = (float)(1.0 - alpha);
  const float maxg = powf((float)max_v, g);
  const float ming = powf((float)min_v, g);
  const float invg = 1.0f / g;
  for (int64_t i = 0; i < n; i++) {
    double y = pow(x[i] * ((double)maxg - (double)ming) + (double)ming, (double)invg);
    if (y >= max_v) y = max_v - 1.0;
    out[i] = (int64_t)y;
  }
}
