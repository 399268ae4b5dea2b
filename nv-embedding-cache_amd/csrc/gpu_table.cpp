// gpu_table.cpp -- GpuTable: 8-way set-associative cache in HBM over an
// optional host-linear backing table.
//
// Layout (EmbedCacheSA<Key, Key>, ec_set_associative.h:104-178, :327-403,
// :667-685): per set 8 tags of the key type, 8 rows, 8 float counters and one
// int64 timestamp.  num_sets = cache_size / (align16(8*sizeof(Key)) +
// align16(8*row) + align16(8*4)), the device-modify counter bytes included in
// the per-set size (ec_set_associative_device_modify.cuh:472-474).  With
// modify_on_gpu = false (CacheSAHostModify) the counters and timestamps live
// in host memory and the per-set size has no counter term
// (ec_set_associative_host_modify.h:519-534).  Rows live set-major at
// data + (set*8 + way)*row so one set's 8 rows are contiguous.
#include <algorithm>
#include <climits>
#include <cstring>

#include "kernels/cache_launch.hpp"
#include "kernels/modify_launch.hpp"
#include "layers.hpp"
#include "trace.hpp"

namespace nve_amd {

namespace {
uint64_t align16(uint64_t x) { return (x + 15) / 16 * 16; }
}  // namespace

GpuTable::GpuTable(int key_bytes, const GPUTableConfig& cfg) : key_bytes_(key_bytes), cfg_(cfg) {
  ScopedDevice sd(cfg_.device_id);
  if (cfg_.private_stream) lookups_->add(cfg_.private_stream);  // lookups run there
  NVE_CHECK(key_bytes == 4 || key_bytes == 8, "Unsupported key size ", key_bytes);
  NVE_CHECK(cfg_.row_size_in_bytes > 0, "Invalid row size");
  NVE_CHECK(cfg_.uvm_table == nullptr || cfg_.uvm_num_rows > 0,
            "uvm_num_rows must be set to the number of rows in uvm_table");
  NVE_CHECK(cfg_.max_modify_size > 0, "max_modify_size must be positive");
  // an unknown kernel_mode_type is accepted here and reported as not
  // implemented by the first lookup that needs a mode (gpu_table.cu:271-287)
  if (cfg_.kernel_mode_type == 3 && cfg_.kernel_mode_value != 0) {
    // PipelineGather: kernel_mode_value points at {task_size, num_aux_streams}
    // (GatherKernelPipelineParams, pipeline_gather.cuh:33-36), read once here
    const uint64_t* params = reinterpret_cast<const uint64_t*>(cfg_.kernel_mode_value);
    if (params[0] > 0) pipeline_task_size_ = params[0];
  }
  if (is_rowwise(cfg_.value_dtype))
    NVE_CHECK(cfg_.row_size_in_bytes % 2 == 0, "Quantized rows must have an even width");
  const uint64_t per_set = align16((uint64_t)key_bytes * kWays) +
                           align16((uint64_t)cfg_.row_size_in_bytes * kWays) +
                           (cfg_.modify_on_gpu ? align16(sizeof(float) * kWays) : 0);
  num_sets_ = cfg_.cache_size / per_set;
  NVE_CHECK(num_sets_ > 0, "Memory allocated to the cache is too small");
  NVE_CHECK(num_sets_ <= UINT32_MAX, "Too many cache sets");
  const uint64_t ways = num_sets_ * kWays;
  const size_t data_bytes = (size_t)ways * (size_t)cfg_.row_size_in_bytes;
  NVE_LOG_INFO("GpuTable on device ", cfg_.device_id, ": ", num_sets_, " sets of 8 ways, ",
               data_bytes, " bytes of rows in ", cfg_.data_storage_on_host ? "host" : "device",
               " memory, ", cfg_.uvm_table ? "with" : "without", " a backing table, ",
               cfg_.modify_on_gpu ? "device" : "host", " replacement policy");
  if (cfg_.data_storage_on_host)
    NVE_HIP(hipHostMalloc((void**)&data_, data_bytes, hipHostMallocDefault));
  else
    NVE_HIP(hipMalloc((void**)&data_, data_bytes));
  NVE_HIP(hipMalloc(&tags_, (size_t)ways * key_bytes));
  NVE_HIP(launch_fill_tags(tags_, (int64_t)ways, key_bytes, cfg_.invalid_key, nullptr));
  if (cfg_.modify_on_gpu) {
    NVE_HIP(hipMalloc((void**)&counters_, (size_t)ways * sizeof(float)));
    NVE_HIP(hipMalloc((void**)&set_ts_, (size_t)num_sets_ * sizeof(int64_t)));
    NVE_HIP(launch_fill_u32(reinterpret_cast<uint32_t*>(counters_), (int64_t)ways, 0, nullptr));
    NVE_HIP(launch_fill_u64(reinterpret_cast<uint64_t*>(set_ts_), (int64_t)num_sets_, 0, nullptr));
    NVE_HIP(hipMalloc((void**)&set_word_, (size_t)num_sets_ * sizeof(uint64_t)));
    NVE_HIP(launch_fill_u64(set_word_, (int64_t)num_sets_, kSetClean, nullptr));
    build_decay_table();
  } else {
    h_tags_.resize((size_t)ways * key_bytes);
    for (uint64_t w = 0; w < ways; ++w) set_h_tag(w, cfg_.invalid_key);
    h_counters_.assign((size_t)ways, 0.0f);
    h_set_ts_.assign((size_t)num_sets_, 0);
  }
  NVE_HIP(hipDeviceSynchronize());
}

GpuTable::~GpuTable() {
  ScopedDevice sd(cfg_.device_id);
  (void)hipDeviceSynchronize();
  if (cfg_.data_storage_on_host)
    (void)hipHostFree(data_);
  else
    (void)hipFree(data_);
  (void)hipFree(tags_);
  (void)hipFree(counters_);
  (void)hipFree(set_ts_);
  (void)hipFree(set_word_);
  (void)hipFree(decay_table_);
}

RowSource GpuTable::row_source(bool with_uvm) const {
  RowSource s{};
  s.table = with_uvm ? static_cast<const uint8_t*>(cfg_.uvm_table) : nullptr;
  s.num_rows = with_uvm ? (uint64_t)cfg_.uvm_num_rows : 0;  // misses outside it read nothing
  s.row_bytes = (uint64_t)cfg_.row_size_in_bytes;
  s.load_indices = 1;
  s.cache_data = data_;
  s.cache_tags = tags_;
  s.num_sets = num_sets_;
  return s;
}

// GpuTable::find (gpu_table.cu:375-413).  With a backing table every key is
// resolved (cache hit or backing row) and the hit mask is left alone; without
// one, hits are copied and flagged in the mask, misses keep their output.
void GpuTable::find(ExecutionContext& ctx, int64_t n, const void* keys, uint64_t* hit_mask,
                    int64_t value_stride, void* values, int64_t* value_sizes) {
  ScopedDevice sd(cfg_.device_id);
  NVE_CHECK(value_sizes == nullptr, "value_sizes must be nullptr for GPU table");
  if (n <= 0) return;
  NVE_CHECK_ARG(keys != nullptr, "keys must not be null");
  StreamQueue q(ctx.lookup_stream(), cfg_.private_stream);
  const hipStream_t stream = q.stream;
  const void* d_keys = device_input(ctx, "keys", keys, (size_t)n * key_bytes_, stream);
  const bool uvm = cfg_.uvm_table != nullptr;
  uint64_t* d_mask = nullptr;
  const size_t mask_bytes = (size_t)((n + 63) / 64) * 8;
  if (!uvm && hit_mask) {
    d_mask = static_cast<uint64_t*>(
        const_cast<void*>(device_input(ctx, "hit_mask", hit_mask, mask_bytes, stream)));
  }
  if (values) NVE_CHECK_ARG(value_stride >= cfg_.row_size_in_bytes, "value_stride is smaller than a row");
  const size_t out_bytes = values ? (size_t)(n - 1) * value_stride + cfg_.row_size_in_bytes : 0;
  void* d_vals = values ? device_output(ctx, "values", values, out_bytes) : nullptr;
  if (d_vals != values && values) {
    // rows that miss keep the caller's content: start from a copy of it
    NVE_HIP(hipMemcpyAsync(d_vals, values, out_bytes, hipMemcpyHostToDevice, stream));
  }

  std::shared_lock<std::shared_mutex> lk(uvm_mu_, std::defer_lock);
  // backing-table writers (update, accumulate, erase, clear) take it exclusively
  if (uvm) lk.lock();
  GatherLaunch g{};
  g.keys = d_keys;
  g.key_bytes = key_bytes_;
  g.n = n;
  g.src = row_source(uvm);
  g.stored_dtype = cfg_.value_dtype;
  g.raw = 1;
  g.out = d_vals;
  g.out_stride = value_stride;
  g.hitmask = d_mask;
  g.miss_counter = cfg_.count_misses ? ctx.miss_counter() : nullptr;
  if (d_vals == nullptr) {
    // existence check only: resolve into a scratch row per key
    NVE_CHECK_ARG(d_mask != nullptr || uvm, "find needs values or a hit mask");
    g.out = ctx.buffer("find_scratch", (size_t)n * cfg_.row_size_in_bytes);
    g.out_stride = cfg_.row_size_in_bytes;
  }
  if (uvm && d_vals != nullptr) {
    switch (uvm_mode(n)) {
      case UvmMode::Lookup: NVE_HIP(launch_gather(g, stream)); break;
      case UvmMode::SortGather: find_sort_gather(ctx, g, stream); break;
      case UvmMode::PipelineGather: find_pipeline_gather(ctx, g, stream); break;
    }
  } else {
    NVE_HIP(launch_gather(g, stream));
  }
  if (d_mask && d_mask != hit_mask)
    NVE_HIP(hipMemcpyAsync(hit_mask, d_mask, mask_bytes, hipMemcpyDeviceToHost, stream));
  if (values) finish_output(values, d_vals, out_bytes, stream);
  if (d_mask != hit_mask || d_vals != values) NVE_HIP(hipStreamSynchronize(stream));
}

// GpuTable::find_and_pool (gpu_table.cu:1049-1104): fused resolve + dequant +
// pool; rows that miss are read from the backing table in host memory.
void GpuTable::find_and_pool(ExecutionContext& ctx, int64_t n, const void* d_keys,
                             const PoolingParams& pp, void* d_output, int64_t output_stride) {
  ScopedDevice sd(cfg_.device_id);
  StreamQueue q(ctx.lookup_stream(), cfg_.private_stream);
  const hipStream_t stream = q.stream;
  const int vdt = cfg_.value_dtype;
  const int64_t count =
      is_rowwise(vdt) ? (cfg_.row_size_in_bytes - meta_bytes(vdt)) / value_elem_bytes(vdt)
                      : cfg_.row_size_in_bytes / std::max(1, dtype_size(vdt));
  std::shared_lock<std::shared_mutex> lk(uvm_mu_, std::defer_lock);
  lk.lock();  // held off while the backing table is written
  if (pp.pooling_type == NVE_POOL_CONCATENATE) {
    GatherLaunch g{};
    g.keys = d_keys;
    g.key_bytes = key_bytes_;
    g.n = n;
    g.src = row_source(true);
    g.stored_dtype = vdt;
    g.count = output_stride / dtype_size(pp.output_type);
    g.raw = 0;
    g.out = d_output;
    g.out_stride = output_stride;
    g.out_dtype = pp.output_type;
    g.miss_counter = cfg_.count_misses ? ctx.miss_counter() : nullptr;
    NVE_HIP(launch_gather(g, stream));
    return;
  }
  PoolLaunch p{};
  p.keys = d_keys;
  p.key_bytes = key_bytes_;
  p.num_keys = n;
  if (pp.sparse_type == NVE_SPARSE_CSR) {
    p.offsets = pp.csr_offsets;
    p.num_bags = pp.num_csr_offsets - 1;
  } else {
    p.hotness = pp.fixed_hotness;
    p.num_bags = n / pp.fixed_hotness;
  }
  p.weighted = is_weighted_pooling(pp.pooling_type);
  p.mean = is_mean_pooling(pp.pooling_type);
  p.weights = pp.weights;
  p.weight_dtype = pp.weight_type;
  p.src = row_source(true);
  p.stored_dtype = vdt;
  p.count = output_stride / dtype_size(pp.output_type);
  NVE_CHECK_ARG(p.count <= count, "Output stride implies more values than a stored row holds");
  p.out = d_output;
  p.out_stride = output_stride;
  p.out_dtype = pp.output_type;
  p.miss_counter = cfg_.count_misses ? ctx.miss_counter() : nullptr;
  NVE_HIP(launch_pool(p, stream));
}

void GpuTable::erase(ExecutionContext& ctx, int64_t n, const void* keys) {
  ScopedDevice sd(cfg_.device_id);
  if (n <= 0) return;
  NVE_CHECK_ARG(keys != nullptr, "keys must not be null");
  std::lock_guard<std::mutex> mk(modify_mu_);
  std::unique_lock<std::shared_mutex> lk(uvm_mu_);
  StreamQueue q(ctx.modify_stream(), cfg_.private_stream);
  const hipStream_t stream = q.stream;
  if (!cfg_.modify_on_gpu) {
    // CacheSAHostModify::invalidate (ec_set_associative_host_modify.h:134-178):
    // every matching way of the host tags is emptied (its counter stays) and
    // the device tags follow
    const uint8_t* hk = static_cast<const uint8_t*>(
        host_input(ctx, "modify_keys_host", keys, (size_t)n * key_bytes_, stream));
    std::vector<uint64_t> slot;
    std::vector<int64_t> tag;
    std::vector<uint64_t> src;
    for (int64_t i = 0; i < n; ++i) {
      const int64_t k = load_key(hk, i);
      const uint64_t set = set_of(k);
      for (int w = 0; w < kWays; ++w) {
        const uint64_t sl = set * kWays + (uint64_t)w;
        if (key_of(h_tag(sl), set) == k) {
          set_h_tag(sl, cfg_.invalid_key);
          slot.push_back(sl);
          tag.push_back(cfg_.invalid_key);
          src.push_back(0);
        }
      }
    }
    apply_records(ctx, stream, slot, tag, src, true);
    return;
  }
  const void* d_keys = device_input(ctx, "modify_keys", keys, (size_t)n * key_bytes_, stream);
  NVE_HIP(launch_cache_erase(tags_, d_keys, n, key_bytes_, num_sets_, cfg_.invalid_key, stream));
  NVE_HIP(hipStreamSynchronize(stream));
}

// clear_cache: all ways empty, the insert clock and the set timestamps back to
// 0 (ec_set_associative_device_modify.cuh:205-222); the host-policy cache also
// zeroes its counters (ec_set_associative_host_modify.h:192-211).  The device
// policy leaves the counters: an empty way counts as 0 there whatever it holds.
void GpuTable::clear(ExecutionContext& ctx) {
  ScopedDevice sd(cfg_.device_id);
  std::lock_guard<std::mutex> mk(modify_mu_);
  std::unique_lock<std::shared_mutex> lk(uvm_mu_);
  StreamQueue q(ctx.modify_stream(), cfg_.private_stream);
  const hipStream_t stream = q.stream;
  const int64_t ways = (int64_t)num_sets_ * kWays;
  NVE_HIP(launch_fill_tags(tags_, ways, key_bytes_, cfg_.invalid_key, stream));
  if (cfg_.modify_on_gpu) {
    NVE_HIP(launch_fill_u64(reinterpret_cast<uint64_t*>(set_ts_), (int64_t)num_sets_, 0, stream));
  } else {
    for (int64_t w = 0; w < ways; ++w) set_h_tag((uint64_t)w, cfg_.invalid_key);
    std::fill(h_counters_.begin(), h_counters_.end(), 0.0f);
    std::fill(h_set_ts_.begin(), h_set_ts_.end(), 0);
  }
  global_ts_ = 0;
  NVE_HIP(hipStreamSynchronize(stream));
}

void GpuTable::export_state(void* tags, float* counters, int64_t* set_ts, int64_t* global_ts) {
  ScopedDevice sd(cfg_.device_id);
  std::lock_guard<std::mutex> mk(modify_mu_);  // modifies end with their stream synchronized
  const size_t ways = (size_t)num_sets_ * kWays;
  if (tags) NVE_HIP(hipMemcpy(tags, tags_, ways * key_bytes_, hipMemcpyDefault));
  if (cfg_.modify_on_gpu) {
    if (counters) NVE_HIP(hipMemcpy(counters, counters_, ways * sizeof(float), hipMemcpyDefault));
    if (set_ts) NVE_HIP(hipMemcpy(set_ts, set_ts_, num_sets_ * sizeof(int64_t), hipMemcpyDefault));
  } else {
    if (counters) std::memcpy(counters, h_counters_.data(), ways * sizeof(float));
    if (set_ts) std::memcpy(set_ts, h_set_ts_.data(), num_sets_ * sizeof(int64_t));
  }
  if (global_ts) *global_ts = global_ts_;
}

void GpuTable::import_state(const void* tags, const float* counters, const int64_t* set_ts,
                            int64_t global_ts) {
  ScopedDevice sd(cfg_.device_id);
  std::lock_guard<std::mutex> mk(modify_mu_);
  std::unique_lock<std::shared_mutex> lk(uvm_mu_);
  lookups_->drain();  // lookups queued so far read the old tags to the end
  const size_t ways = (size_t)num_sets_ * kWays;
  // copies on the null stream, then waited for: a copy from pageable memory
  // may still be in flight when hipMemcpy returns, and lookups queued after
  // this call must see the imported state
  const hipStream_t s = nullptr;
  if (tags) NVE_HIP(hipMemcpyAsync(tags_, tags, ways * key_bytes_, hipMemcpyDefault, s));
  if (cfg_.modify_on_gpu) {
    if (counters)
      NVE_HIP(hipMemcpyAsync(counters_, counters, ways * sizeof(float), hipMemcpyDefault, s));
    if (set_ts)
      NVE_HIP(hipMemcpyAsync(set_ts_, set_ts, num_sets_ * sizeof(int64_t), hipMemcpyDefault, s));
  } else {
    if (tags) NVE_HIP(hipMemcpyAsync(h_tags_.data(), tags, ways * key_bytes_, hipMemcpyDefault, s));
    if (counters)
      NVE_HIP(hipMemcpyAsync(h_counters_.data(), counters, ways * sizeof(float), hipMemcpyDefault, s));
    if (set_ts)
      NVE_HIP(hipMemcpyAsync(h_set_ts_.data(), set_ts, num_sets_ * sizeof(int64_t), hipMemcpyDefault, s));
  }
  NVE_HIP(hipStreamSynchronize(s));
  global_ts_ = global_ts;
}

}  // namespace nve_amd
