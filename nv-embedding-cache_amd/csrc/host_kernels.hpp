// host_kernels.hpp -- the CPU row kernels of the host layer: threaded gather,
// per-bag fp32 pooling, per-row conversion / dequantization, row updates.
//
// Reference counterparts (file:line in /root/reference):
//   gather                 cpu_ops/cpu_gather.hpp:28-80
//   pooling                cpu_ops/cpu_pooling.hpp:68-150 (float / half rows),
//                          :166-259 (rowwise-quantized rows)
//   conversion             cpu_ops/cpu_pooling.hpp:272-341
//   update / accumulate    cpu_ops/cpu_update.hpp:28-129
//
// Arithmetic per element, fixed so that every host and every instruction set
// produces the same bits (the translation unit is built without contraction):
//   value    = float(x) for f32 / f16 rows; fma(float(q), scale, offset) for
//              rowwise-quantized rows (offset 0 for the int8 formats, scale and
//              offset widened from f16 for the f16-metadata formats);
//              e4m3(q) * scale for the fp8 extension format
//   weighted = value * w, rounded, then added: acc += value (* w)
//   mean     = acc * (1 / denom), denom = count or the weights added in order,
//              a zero denominator giving a zero row; the output is rounded to
//              nearest even once.
// A host with AVX2 + F16C + FMA runs 8-wide loops, any other the scalar ones;
// the results are identical.
#pragma once

#include <stdint.h>

#include <functional>

#include "runtime.hpp"

namespace nve_amd {
namespace hostk {

// Runs task(0 .. num_tasks-1): task 0 on the calling thread, the others on
// `pool`; returns when all are done and rethrows the first exception.
void run_tasks(ThreadPool& pool, int64_t num_tasks, const std::function<void(int64_t)>& task);

// cpu_kernel_gather: row keys[i] of `table` to values + i*value_stride for
// keys in [0, num_rows) whose hit bit is not set yet; sets their hit bits
// (hit_mask may be null) and returns how many rows were copied.  Keys are
// split into num_threads tasks of a multiple of 64 keys, so no two tasks
// write the same hit-mask word.
int64_t gather(ThreadPool& pool, int64_t num_threads, int64_t n, const void* keys, int key_bytes,
               uint64_t* hit_mask, uint8_t* values, int64_t value_stride, const uint8_t* table,
               int64_t row_bytes, uint64_t num_rows);

struct PoolSpec {
  int dtype = 0;            // stored row format (dtypes.hpp)
  int64_t count = 0;        // values per row
  int pooling = 0;          // NVE_POOL_SUM .. NVE_POOL_WEIGHTED_MEAN
  int sparse = 0;           // NVE_SPARSE_FIXED / NVE_SPARSE_CSR
  int64_t fixed_hotness = 0;
  const void* offsets = nullptr;  // CSR: num_bags + 1 entries
  int offset_bytes = 8;
  const void* weights = nullptr;  // per key (weighted pooling)
  int weight_type = 0;            // kF32 / kF16
  int out_type = 0;               // kF32 / kF16
};

// Pools bag b of `rows` (one gathered row per key, row_stride bytes apart)
// into out + b*out_stride for b < num_bags, bags split over `workers` tasks.
void pool(ThreadPool& pool, int64_t workers, const PoolSpec& spec, int64_t num_bags,
          const uint8_t* rows, int64_t row_stride, uint8_t* out, int64_t out_stride);

// One output row per input row: values converted (f32 <-> f16) or
// dequantized to out_type (kF32 / kF16).
void convert(ThreadPool& pool, int64_t workers, int dtype, int64_t count, int out_type,
             int64_t num_rows, const uint8_t* rows, int64_t row_stride, uint8_t* out,
             int64_t out_stride);

// Copies of whole rows: dst + i*dst_stride <- src + i*src_stride.
void copy_rows(ThreadPool& pool, int64_t workers, int64_t num_rows, const uint8_t* src,
               int64_t src_stride, uint8_t* dst, int64_t dst_stride, int64_t row_bytes);

// cpu_kernel_update: table row keys[i] <- values + i*value_stride (keys out of
// range skipped; a repeated key takes its last value).
void update_rows(ThreadPool& pool, int64_t num_threads, int64_t n, const void* keys, int key_bytes,
                 const uint8_t* values, int64_t value_stride, uint8_t* table, int64_t row_bytes,
                 uint64_t num_rows);

// cpu_kernel_update_accumulate: table row keys[i] += update i, rows of f32
// (dtype kF32) or f16 (kF16: each element widened, added in f32, rounded
// back).  Work is split by key, so every row has one writer and a repeated
// key's updates are added in position order: the result is deterministic.
void accumulate_rows(ThreadPool& pool, int64_t num_threads, int64_t n, const void* keys,
                     int key_bytes, const uint8_t* updates, int64_t update_stride, uint8_t* table,
                     int64_t row_bytes, uint64_t num_rows, int dtype);

// true when the 8-wide AVX2 + F16C + FMA loops are in use on this host
bool vector_loops();

}  // namespace hostk
}  // namespace nve_amd
