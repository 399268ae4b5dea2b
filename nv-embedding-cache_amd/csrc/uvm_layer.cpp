// uvm_layer.cpp -- LinearUVMEmbeddingLayer: GPU cache over a host-linear table.
//
// Lookup flow (linear_embedding_layer.cu:91-209): sanitize keys against the
// backing table, reset the context's miss counter, run the fused
// find-and-pool (or the raw find), read the miss count (a stream sync) to get
// the hit rate, then hand the keys to the auto-insert protocol
// (layer_utils.cpp:94-275): once the heuristic fires, keys are collected
// until min_insert_size_gpu of them exist, and the insert runs as a task on
// the context's thread pool.  Plain lookups also keep their output rows (a
// device-to-device copy) and the insert takes them from HBM; a pooled lookup
// has no per-key rows, so a collection it joins promotes the rows from the
// backing table (linear_embedding_layer.cu:197-206).
#include <climits>
#include <cstring>

#include "layers.hpp"
#include "trace.hpp"

namespace nve_amd {

LinearUVMEmbeddingLayer::LinearUVMEmbeddingLayer(int key_bytes, const LinearUVMLayerConfig& cfg,
                                                 std::shared_ptr<GpuTable> table)
    : EmbeddingLayer(key_bytes, table ? table->config().device_id : 0),
      cfg_(cfg),
      table_(std::move(table)) {
  NVE_CHECK(table_ != nullptr, "Invalid GPU table");
  NVE_CHECK(table_->key_bytes() == key_bytes, "GPU table key type does not match the layer");
  NVE_CHECK(table_->config().uvm_table != nullptr, "LinearUVM layer requires a GPU table with a uvm_table");
  NVE_CHECK(table_->config().uvm_num_rows > 0, "uvm_num_rows must be >0");
  NVE_CHECK((uint64_t)table_->config().uvm_num_rows <= (key_bytes == 4 ? (uint64_t)INT32_MAX : (uint64_t)INT64_MAX),
            "Number of UVM rows cannot be represented by the layer key type");
  NVE_CHECK(cfg_.default_row_index < table_->config().uvm_num_rows,
            "Default row index must be less than the UVM table's row count");
  if (!cfg_.insert_heuristic)
    cfg_.insert_heuristic = std::make_shared<DefaultInsertHeuristic>(std::vector<float>{0.75f});
}

void LinearUVMEmbeddingLayer::lookup(ExecutionContext& ctx, int64_t num_keys, const void* keys,
                                     void* output, int64_t output_stride, uint64_t* hitmask,
                                     const PoolingParams* pp, float* hitrates) {
  const GPUTableConfig& tc = table_->config();
  ScopedDevice sd(tc.device_id);
  NVE_CHECK_ARG(num_keys >= 0, "Invalid num_keys");
  NVE_CHECK_ARG(keys != nullptr, "Invalid keys buffer");
  NVE_CHECK_ARG(output != nullptr, "Invalid output buffer");
  NVE_CHECK_ARG(hitmask == nullptr, "Hitmask is not supported for the UVM layer");
  NVE_CHECK_ARG(num_keys <= INT_MAX, "Number of keys exceeding max int value is not supported");
  const hipStream_t stream = ctx.lookup_stream();
  if (pp) validate_pool_params(*pp);
  const bool raw_concat = pp && pp->pooling_type == NVE_POOL_CONCATENATE &&
                          pp->output_type == tc.value_dtype;
  if (raw_concat)
    NVE_CHECK_ARG(output_stride >= tc.row_size_in_bytes,
                  "Raw Concatenate output stride is smaller than the stored row width");
  const bool pooled = pp && !raw_concat;
  if (pooled) {
    // find_and_pool.cuh:29-86: the output precision follows the stored type
    const int vdt = tc.value_dtype;
    const bool ext = vdt == kXI8AF32 || vdt == kXE4M3F32;
    NVE_CHECK_ARG(ext ? (pp->output_type == kF32 || pp->output_type == kF16)
                      : pp->output_type == native_out(vdt),
                  "Unsupported find_and_pool value/output type combination: value type ", vdt,
                  " output type ", pp->output_type);
    const int oes = dtype_size(pp->output_type);
    NVE_CHECK_ARG(output_stride > 0 && output_stride % oes == 0,
                  "Pooled/dequantized output stride must be a whole number of output elements");
    const int64_t vcount = output_stride / oes;
    const int64_t stored = is_rowwise(vdt) ? value_elem_bytes(vdt) : oes;
    NVE_CHECK_ARG(vcount * stored + meta_bytes(vdt) <= tc.row_size_in_bytes,
                  "Pooled/dequantized output stride implies more value elements than the stored row holds");
    if (pp->pooling_type != NVE_POOL_CONCATENATE && is_weighted_pooling(pp->pooling_type))
      NVE_CHECK_ARG(pp->weight_type == kF32 || pp->weight_type == kF16,
                    "Unsupported find_and_pool weight type ", pp->weight_type);
  }
  const int64_t out_rows = lookup_output_rows(num_keys, pp);
  const size_t out_bytes = (size_t)out_rows * (size_t)output_stride;
  const void* d_keys = device_input(ctx, "keys", keys, (size_t)num_keys * key_bytes_, stream);
  if (cfg_.default_row_index >= 0 && num_keys > 0) {
    void* s = ctx.buffer("sanitized_keys", (size_t)num_keys * key_bytes_);
    NVE_HIP(launch_sanitize(d_keys, s, num_keys, key_bytes_, (uint64_t)tc.uvm_num_rows,
                            cfg_.default_row_index, stream));
    d_keys = s;
  }
  const bool never = dynamic_cast<NeverInsertHeuristic*>(cfg_.insert_heuristic.get()) != nullptr;
  const bool collect = hitrates != nullptr || !never;
  if (collect) {
    NVE_CHECK(tc.count_misses, "GPU table was not configured to report hit counts");
    ctx.prepare_misses();
  }
  void* d_out = device_output(ctx, "output", output, out_bytes);
  if (pooled) {
    PoolingParams dp = *pp;
    if (pp->pooling_type != NVE_POOL_CONCATENATE) {
      if (pp->sparse_type == NVE_SPARSE_CSR)
        dp.csr_offsets = device_input(ctx, "offsets", pp->csr_offsets,
                                      (size_t)pp->num_csr_offsets * key_bytes_, stream);
      if (pp->weights)
        dp.weights = device_input(ctx, "weights", pp->weights,
                                  (size_t)num_keys * dtype_size(pp->weight_type), stream);
    }
    table_->find_and_pool(ctx, num_keys, d_keys, dp, d_out, output_stride);
  } else {
    table_->find(ctx, num_keys, d_keys, nullptr, output_stride, d_out, nullptr);
  }
  finish_output(output, d_out, out_bytes, stream);
  if (collect) {
    const int64_t misses = ctx.take_misses();  // syncs the lookup stream, leaves the counter at 0
    const float hitrate =
        num_keys > 0 ? 1.0f - (float)misses / (float)num_keys : 1.0f;
    if (hitrates) *hitrates = hitrate;
    if (!never && num_keys > 0) auto_insert(ctx, num_keys, d_keys, d_out, output_stride, pooled, hitrate);
  }
}

struct LinearUVMEmbeddingLayer::CollectedRows {
  void* ptr = nullptr;
  size_t bytes = 0;
  explicit CollectedRows(size_t b) : bytes(b) { NVE_HIP(hipMalloc(&ptr, b)); }
  ~CollectedRows() { (void)hipFree(ptr); }
  CollectedRows(const CollectedRows&) = delete;
  CollectedRows& operator=(const CollectedRows&) = delete;
};

void LinearUVMEmbeddingLayer::reset_collection() {
  collected_.clear();
  collected_n_ = 0;
  collection_is_uvm_ = false;
}

// Auto-insert (layer_utils.cpp:94-143): collect keys, and the output rows of
// plain lookups, once the heuristic fires; insert when min_insert_size_gpu
// keys are collected.
void LinearUVMEmbeddingLayer::auto_insert(ExecutionContext& ctx, int64_t n, const void* d_keys,
                                          const void* d_out, int64_t out_stride, bool from_uvm,
                                          float hitrate) {
  std::unique_lock<std::mutex> lk(collect_mu_, std::try_to_lock);
  if (!lk.owns_lock()) return;  // an insert is being collected or launched elsewhere
  if (in_flight_ && in_flight_->load()) return;  // the previous insert still runs
  const int64_t min_size = cfg_.min_insert_size_gpu > 0 ? cfg_.min_insert_size_gpu : 1;
  if (collected_n_ > 0) {
    // a pooled lookup joining a collection of rows turns it into one that
    // promotes from the backing table for good, and its rows are dropped
    collection_is_uvm_ = collection_is_uvm_ || from_uvm;
    NVE_CHECK(collection_is_uvm_ || out_stride == collected_stride_,
              "Output stride must be fixed during accumulation");
  } else {
    // min_insert_freq_gpu lookups pass between inserts (layer_utils.cpp:120-131)
    if (--insert_wait_ >= 0) return;
    insert_wait_ = 0;
    if (!cfg_.insert_heuristic->insert_needed(hitrate, 0)) return;
    collection_is_uvm_ = from_uvm;
    collected_stride_ = out_stride;
  }
  const int64_t total = collected_n_ == 0 ? std::max(n, min_size) : min_size;
  const int64_t part = std::min(n, total - collected_n_);
  if (part <= 0) return;
  const hipStream_t s = ctx.lookup_stream();
  const size_t stride = (size_t)collected_stride_;
  uint8_t* rows = nullptr;
  if (!collection_is_uvm_) {
    // sized for the whole collection when it starts, so later parts never
    // move it; an insert task still holding the previous buffer keeps it
    if (collected_n_ == 0 &&
        (!collected_rows_ || collected_rows_.use_count() > 1 || collected_rows_->bytes < (size_t)total * stride))
      collected_rows_ = std::make_shared<CollectedRows>((size_t)total * stride);
    rows = static_cast<uint8_t*>(collected_rows_->ptr);
    NVE_HIP(hipMemcpyAsync(rows + (size_t)collected_n_ * stride, d_out, (size_t)part * stride,
                           hipMemcpyDeviceToDevice, s));
  }
  collected_.resize((size_t)(collected_n_ + part) * key_bytes_);
  NVE_HIP(hipMemcpyAsync(collected_.data() + (size_t)collected_n_ * key_bytes_, d_keys,
                         (size_t)part * key_bytes_, hipMemcpyDefault, s));
  NVE_HIP(hipStreamSynchronize(s));
  // keys outside the backing table (no default row configured) have no row
  // to promote and no defined lookup row: drop them here, with their rows
  {
    const uint64_t num_rows = (uint64_t)table_->config().uvm_num_rows;
    uint8_t* base = collected_.data() + (size_t)collected_n_ * key_bytes_;
    int64_t kept = 0;
    int64_t run = -1;  // first part position of the current run of kept keys
    // a run that moved down gets its rows again from the lookup's output
    auto flush = [&](int64_t end) {
      const int64_t len = end - run;
      if (rows && run >= 0 && kept - len != run)
        NVE_HIP(hipMemcpyAsync(rows + (size_t)(collected_n_ + kept - len) * stride,
                               static_cast<const uint8_t*>(d_out) + (size_t)run * stride,
                               (size_t)len * stride, hipMemcpyDeviceToDevice, s));
      run = -1;
    };
    for (int64_t i = 0; i < part; ++i) {
      int64_t k;
      if (key_bytes_ == 4) {
        int32_t k32;
        std::memcpy(&k32, base + (size_t)i * 4, 4);
        k = k32;
      } else {
        std::memcpy(&k, base + (size_t)i * 8, 8);
      }
      if ((uint64_t)k >= num_rows) {
        flush(i);
        continue;
      }
      if (kept != i) std::memmove(base + (size_t)kept * key_bytes_, base + (size_t)i * key_bytes_, key_bytes_);
      if (run < 0) run = i;
      ++kept;
    }
    flush(part);
    if (rows && kept != part) NVE_HIP(hipStreamSynchronize(s));
    collected_n_ += kept;
    collected_.resize((size_t)collected_n_ * key_bytes_);
  }
  if (collected_n_ < min_size) return;
  std::vector<uint8_t> keys;
  keys.swap(collected_);
  const int64_t nk = collected_n_;
  std::shared_ptr<CollectedRows> data = collection_is_uvm_ ? nullptr : collected_rows_;
  collected_n_ = 0;
  collection_is_uvm_ = false;
  // the insert itself runs as a pool task; wait() on the context joins it
  insert_wait_ = cfg_.min_insert_freq_gpu;
  if (!in_flight_) in_flight_ = std::make_shared<std::atomic<bool>>(false);
  in_flight_->store(true);
  std::shared_ptr<GpuTable> table = table_;
  std::shared_ptr<std::atomic<bool>> flag = in_flight_;
  ExecutionContext* c = &ctx;
  NVE_LOG_PERF("auto-insert of ", nk, " keys launched (hit rate ", hitrate, ", rows from the ",
               data ? "lookups" : "backing table", ")");
  ctx.add_pending(ctx.pool().submit([table, c, nk, flag, data, stride, keys = std::move(keys)]() mutable {
    // the task (with its captures) lives on in the context's future until
    // wait(): hand the rows back to the next collection before the flag drops
    struct Done {
      std::atomic<bool>* f;
      std::shared_ptr<CollectedRows>* d;
      ~Done() {
        d->reset();
        f->store(false);
      }
    } done{flag.get(), &data};
    if (data)
      table->insert(*c, nk, keys.data(), (int64_t)stride, table->config().row_size_in_bytes, data->ptr);
    else
      table->insert_from_uvm(*c, nk, keys.data());
  }));
}

void LinearUVMEmbeddingLayer::insert(ExecutionContext& ctx, int64_t n, const void* keys,
                                     int64_t value_stride, int64_t value_size, const void* values,
                                     int64_t table_id) {
  NVE_CHECK_ARG(table_id <= 0, "Invalid table id ", table_id);
  {
    std::lock_guard<std::mutex> lk(collect_mu_);
    reset_collection();
  }
  table_->insert(ctx, n, keys, value_stride, value_size, values);
}

void LinearUVMEmbeddingLayer::clear(ExecutionContext& ctx) {
  std::lock_guard<std::mutex> lk(collect_mu_);
  reset_collection();
  table_->clear(ctx);
}

void LinearUVMEmbeddingLayer::erase(ExecutionContext& ctx, int64_t n, const void* keys,
                                    int64_t table_id) {
  NVE_CHECK_ARG(table_id <= 0, "Invalid table id ", table_id);
  std::lock_guard<std::mutex> lk(collect_mu_);
  reset_collection();
  table_->erase(ctx, n, keys);
}

}  // namespace nve_amd
