// update.cpp -- row updates: GpuTable::update / update_accumulate and the
// layers' update / accumulate entry points.
//
// Reference behaviour restated:
//   GpuTable::update             src/gpu_table.cu:579-681
//   GpuTable::update_accumulate  src/gpu_table.cu:683-1046 (uvm_cpu_accumulate branch)
//   GPUEmbeddingLayer            src/gpu_embedding_layer.cu:500-639
//   LinearUVMEmbeddingLayer      src/linear_embedding_layer.cu:230-285
//
// Order of work for a table with a backing table, all under the table's
// modify lock (no insert can interleave): the backing rows change first (all
// lookups drained, new ones held off by the table's exclusive lock), then the
// cache rows of resident keys go through invalidate -> drain -> copy or add ->
// commit.  A lookup that runs in the window sees the invalidated tag and reads
// the already changed backing row.
// Accumulating into the backing table is done by host threads whatever
// uvm_cpu_accumulate says: the alternative is GPU atomics over the host link.
#include <algorithm>
#include <vector>

#include "kernels/cache_launch.hpp"
#include "kernels/modify_launch.hpp"
#include "host_kernels.hpp"
#include "kernels/update_launch.hpp"
#include "layers.hpp"
#include "trace.hpp"

namespace nve_amd {

namespace {

template <typename T>
T* carve(uint8_t*& p, size_t count) {
  T* r = reinterpret_cast<T*>(p);
  p += (count * sizeof(T) + 255) / 256 * 256;
  return r;
}

// rows[key] += vals[i] on the host for keys inside [0, num_rows), in the
// table's float type, split over the pool's workers by key: each row has one
// writer and a repeated key's additions are made in position order.
void host_accumulate(ThreadPool& pool, const void* keys, int key_bytes, int64_t n,
                     const uint8_t* vals, int64_t stride, uint8_t* rows, int64_t row_bytes,
                     uint64_t num_rows, int dtype) {
  hostk::accumulate_rows(pool, pool.num_workers(), n, keys, key_bytes, vals, stride, rows, row_bytes,
                         num_rows, dtype);
}

void check_update_args(int64_t n, const void* keys, const void* values, int64_t stride,
                       int64_t size) {
  NVE_CHECK_ARG(n >= 0, "Invalid num_keys");
  NVE_CHECK_ARG(n == 0 || (keys != nullptr && values != nullptr), "keys and values must not be null");
  NVE_CHECK_ARG(stride >= size, "value_stride is smaller than value_size");
}

}  // namespace

// ---------------------------------------------------------------------------
// GpuTable
// ---------------------------------------------------------------------------
// Caller holds modify_mu_.
void GpuTable::modify_rows(ExecutionContext& ctx, hipStream_t s, int64_t n, const void* d_keys,
                           const uint8_t* d_vals, int64_t value_stride, bool accumulate,
                           int dtype) {
  const int64_t chunk = std::max<int64_t>(1, std::min<int64_t>(n, cfg_.max_modify_size));
  uint8_t* p = static_cast<uint8_t*>(ctx.buffer("update_records", (size_t)chunk * 8 * 3 + 768));
  uint64_t* slot = carve<uint64_t>(p, (size_t)chunk);
  int64_t* tag = carve<int64_t>(p, (size_t)chunk);
  uint64_t* src = carve<uint64_t>(p, (size_t)chunk);
  // set by the records kernel when a key matches more than one way
  volatile uint32_t* multi = static_cast<volatile uint32_t*>(ctx.buffer("update_multi", 64, true));
  const int src_align = (int)(((uint64_t)d_vals | (uint64_t)value_stride) & 15u) == 0
                            ? 16
                            : ((((uint64_t)d_vals | (uint64_t)value_stride) & 3u) == 0 ? 4 : 1);
  const uint64_t row_bytes = (uint64_t)cfg_.row_size_in_bytes;
  auto apply = [&](const uint32_t* num, uint32_t cap, const uint64_t* sl, const uint64_t* sr) {
    if (accumulate)
      NVE_HIP(launch_accumulate_rows(num, cap, sl, sr, data_, row_bytes, dtype, s));
    else
      NVE_HIP(launch_copy_rows(num, cap, sl, sr, src_align, data_, row_bytes, s));
  };
  for (int64_t k0 = 0; k0 < n; k0 += chunk) {
    const int64_t cn = std::min(chunk, n - k0);
    const uint32_t m = (uint32_t)cn;
    const uint8_t* ck = static_cast<const uint8_t*>(d_keys) + k0 * key_bytes_;
    const uint8_t* cv = d_vals + k0 * value_stride;
    // record i for key i (empty when no way matches it); the device policy
    // commits the key's own tag into every matching way
    // (ec_set_associative_modify.cuh:541-561), the host policy the first
    // matching way's current tag (ec_set_associative_host_modify.h:489-512)
    *multi = 0;
    NVE_HIP(launch_update_records(ck, cn, key_bytes_, tags_, num_sets_, cv, value_stride, slot, tag, src,
                                  const_cast<uint32_t*>(multi), cfg_.modify_on_gpu, s));
    NVE_HIP(launch_invalidate(nullptr, m, slot, tags_, key_bytes_, cfg_.invalid_key, s));
    // lookups queued before the invalidation may still read these rows
    NVE_HIP(hipStreamSynchronize(s));
    // keys matching several ways (only a key equal to the rebuilt key of the
    // empty ways of its set): records of their further ways, invalidated too
    // (device policy; the host policy stops at a key's first matching way)
    uint32_t* more_num = nullptr;
    uint64_t* more_slot = nullptr;
    int64_t* more_tag = nullptr;
    uint64_t* more_src = nullptr;
    const uint32_t more_cap = (uint32_t)std::min<uint64_t>(7ull * m, 0xffffffffull);
    if (*multi != 0 && cfg_.modify_on_gpu) {
      uint8_t* q = static_cast<uint8_t*>(ctx.buffer("update_more_records", 256 + (size_t)more_cap * 8 * 3 + 768));
      more_num = carve<uint32_t>(q, 1);
      more_slot = carve<uint64_t>(q, more_cap);
      more_tag = carve<int64_t>(q, more_cap);
      more_src = carve<uint64_t>(q, more_cap);
      NVE_HIP(launch_fill_u32(more_num, 1, 0, s));
      NVE_HIP(launch_update_more_records(ck, cn, key_bytes_, tags_, num_sets_, cv, value_stride, more_slot,
                                         more_tag, more_src, more_num, more_cap, s));
      NVE_HIP(launch_invalidate(more_num, more_cap, more_slot, tags_, key_bytes_, cfg_.invalid_key, s));
      NVE_HIP(hipStreamSynchronize(s));
    }
    lookups_->order_before(s);
    apply(nullptr, m, slot, src);
    if (more_num != nullptr) apply(more_num, more_cap, more_slot, more_src);
    NVE_HIP(launch_commit(nullptr, m, slot, tag, tags_, key_bytes_, s));
    if (more_num != nullptr) NVE_HIP(launch_commit(more_num, more_cap, more_slot, more_tag, tags_, key_bytes_, s));
    NVE_HIP(hipStreamSynchronize(s));  // the records are reused by the next chunk
  }
}

void GpuTable::update(ExecutionContext& ctx, int64_t n, const void* keys, int64_t value_stride,
                      int64_t value_size, const void* values) {
  ScopedDevice sd(cfg_.device_id);
  check_update_args(n, keys, values, value_stride, value_size);
  if (n == 0) return;
  NVE_CHECK(value_size == cfg_.row_size_in_bytes, "Unsupported update_size");
  // one modify at a time, for the whole update: an insert in between could
  // copy a backing row into the cache after it changed and before the cache did
  std::lock_guard<std::mutex> mk(modify_mu_);
  StreamQueue q(ctx.modify_stream(), cfg_.private_stream);
  const hipStream_t s = q.stream;
  const void* d_keys = device_input(ctx, "modify_keys", keys, (size_t)n * key_bytes_, s);
  const uint8_t* d_vals = static_cast<const uint8_t*>(device_input(
      ctx, "update_values", values, (size_t)(n - 1) * value_stride + value_size, s));
  if (cfg_.uvm_table != nullptr && !cfg_.disable_uvm_update) {
    std::unique_lock<std::shared_mutex> lk(uvm_mu_);
    lookups_->order_before(s);  // queued lookups read the old backing rows
    NVE_HIP(launch_table_update(d_keys, n, key_bytes_, d_vals, value_stride,
                                static_cast<uint8_t*>(cfg_.uvm_table),
                                (uint64_t)cfg_.row_size_in_bytes, (uint64_t)cfg_.uvm_num_rows, s));
    NVE_HIP(hipStreamSynchronize(s));
  }
  modify_rows(ctx, s, n, d_keys, d_vals, value_stride, false, kUnknown);
}

void GpuTable::update_accumulate(ExecutionContext& ctx, int64_t n, const void* keys,
                                 int64_t value_stride, int64_t value_size, const void* values,
                                 int update_dtype) {
  ScopedDevice sd(cfg_.device_id);
  check_update_args(n, keys, values, value_stride, value_size);
  if (n == 0) return;
  NVE_CHECK(value_size == cfg_.row_size_in_bytes, "Row/update size mismatch");
  NVE_CHECK(update_dtype == cfg_.value_dtype && (update_dtype == kF32 || update_dtype == kF16),
            "Unsupported update type combination");
  std::lock_guard<std::mutex> mk(modify_mu_);  // see update
  StreamQueue q(ctx.modify_stream(), cfg_.private_stream);
  const hipStream_t s = q.stream;
  if (cfg_.uvm_table != nullptr && !cfg_.disable_uvm_update) {
    const void* h_keys = host_input(ctx, "accumulate_keys_host", keys, (size_t)n * key_bytes_, s);
    const uint8_t* h_vals = static_cast<const uint8_t*>(host_input(
        ctx, "accumulate_values_host", values, (size_t)(n - 1) * value_stride + value_size, s));
    std::unique_lock<std::shared_mutex> lk(uvm_mu_);
    lookups_->drain();  // host threads write the rows queued lookups may read
    host_accumulate(ctx.pool(), h_keys, key_bytes_, n, h_vals, value_stride,
                    static_cast<uint8_t*>(cfg_.uvm_table), cfg_.row_size_in_bytes,
                    (uint64_t)cfg_.uvm_num_rows, update_dtype);
  }
  const void* d_keys = device_input(ctx, "modify_keys", keys, (size_t)n * key_bytes_, s);
  const uint8_t* d_vals = static_cast<const uint8_t*>(device_input(
      ctx, "update_values", values, (size_t)(n - 1) * value_stride + value_size, s));
  modify_rows(ctx, s, n, d_keys, d_vals, value_stride, true, update_dtype);
}

// ---------------------------------------------------------------------------
// GPUEmbeddingLayer
// ---------------------------------------------------------------------------
// gpu_embedding_layer.cu:500-505,628-640: no effect on a linear table, with a
// warning that says so
void GPUEmbeddingLayer::insert(ExecutionContext&, int64_t, const void*, int64_t, int64_t,
                               const void*, int64_t) {
  NVE_LOG_WARNING("insert method has no effect for GPU layer, use update to change table content");
}

void GPUEmbeddingLayer::clear(ExecutionContext&) { NVE_LOG_WARNING("clear method has no effect for GPU layer"); }

void GPUEmbeddingLayer::erase(ExecutionContext&, int64_t, const void*, int64_t) {
  NVE_LOG_WARNING("erase method has no effect for GPU layer");
}

void GPUEmbeddingLayer::update(ExecutionContext& ctx, int64_t n, const void* keys,
                               int64_t value_stride, int64_t value_size, const void* values,
                               int64_t table_id) {
  ScopedDevice sd(cfg_.device_id);
  check_update_args(n, keys, values, value_stride, value_size);
  NVE_CHECK_ARG(value_size == cfg_.embedding_width_in_bytes, "Invalid value size");
  NVE_CHECK_ARG(table_id < num_tables(), "Invalid table_id");
  if (n == 0) return;
  const hipStream_t s = ctx.modify_stream();
  const void* d_keys = device_input(ctx, "modify_keys", keys, (size_t)n * key_bytes_, s);
  const uint8_t* d_vals = static_cast<const uint8_t*>(device_input(
      ctx, "update_values", values, (size_t)(n - 1) * value_stride + value_size, s));
  std::lock_guard<std::mutex> lk(launch_mu_);
  lookups_->order_before(s);  // lookups issued before this call read the old rows
  NVE_HIP(launch_table_update(d_keys, n, key_bytes_, d_vals, value_stride,
                              static_cast<uint8_t*>(cfg_.embedding_table),
                              (uint64_t)cfg_.embedding_width_in_bytes,
                              (uint64_t)cfg_.num_embeddings, s));
  NVE_HIP(hipStreamSynchronize(s));  // and lookups issued after it read the new ones
}

void GPUEmbeddingLayer::accumulate(ExecutionContext& ctx, int64_t n, const void* keys,
                                   int64_t value_stride, int64_t value_size, const void* values,
                                   int value_type, int64_t table_id) {
  ScopedDevice sd(cfg_.device_id);
  check_update_args(n, keys, values, value_stride, value_size);
  NVE_CHECK(!is_rowwise(cfg_.value_dtype),
            "Accumulate is not supported for quantized GPU embedding tables");
  NVE_CHECK_ARG(value_size == cfg_.embedding_width_in_bytes, "Invalid value size");
  NVE_CHECK_ARG(table_id < num_tables(), "Invalid table_id");
  NVE_CHECK_ARG(value_type == kF32 || value_type == kF16, "Unsupported Data type");
  NVE_CHECK_ARG(value_type == cfg_.value_dtype, "Accumulated values must have the table's type");
  if (n == 0) return;
  const hipStream_t s = ctx.modify_stream();
  const void* d_keys = device_input(ctx, "modify_keys", keys, (size_t)n * key_bytes_, s);
  const uint8_t* d_vals = static_cast<const uint8_t*>(device_input(
      ctx, "update_values", values, (size_t)(n - 1) * value_stride + value_size, s));
  std::lock_guard<std::mutex> lk(launch_mu_);
  lookups_->order_before(s);  // see update
  NVE_HIP(launch_table_accumulate(d_keys, n, key_bytes_, d_vals, value_stride,
                                  static_cast<uint8_t*>(cfg_.embedding_table),
                                  (uint64_t)cfg_.embedding_width_in_bytes,
                                  (uint64_t)cfg_.num_embeddings, value_type, s));
  NVE_HIP(hipStreamSynchronize(s));
}

// ---------------------------------------------------------------------------
// LinearUVMEmbeddingLayer
// ---------------------------------------------------------------------------
void LinearUVMEmbeddingLayer::update(ExecutionContext& ctx, int64_t n, const void* keys,
                                     int64_t value_stride, int64_t value_size, const void* values,
                                     int64_t table_id) {
  check_update_args(n, keys, values, value_stride, value_size);
  NVE_CHECK_ARG(value_size == table_->config().row_size_in_bytes, "Invalid value size");
  NVE_CHECK_ARG(table_id < num_tables(), "Invalid table_id");
  {
    std::lock_guard<std::mutex> lk(collect_mu_);
    reset_collection();  // collected lookup rows may predate the new values
  }
  table_->update(ctx, n, keys, value_stride, value_size, values);
}

void LinearUVMEmbeddingLayer::accumulate(ExecutionContext& ctx, int64_t n, const void* keys,
                                         int64_t value_stride, int64_t value_size,
                                         const void* values, int value_type, int64_t table_id) {
  check_update_args(n, keys, values, value_stride, value_size);
  NVE_CHECK_ARG(value_size == table_->config().row_size_in_bytes, "Invalid value size");
  NVE_CHECK_ARG(table_id < num_tables(), "Invalid table_id");
  {
    std::lock_guard<std::mutex> lk(collect_mu_);
    reset_collection();  // collected lookup rows may predate the new values
  }
  table_->update_accumulate(ctx, n, keys, value_stride, value_size, values, value_type);
}

}  // namespace nve_amd
