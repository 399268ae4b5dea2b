// layers.hpp -- embedding layers and the GPU table (set-associative cache).
//
// Reference counterparts (file:line in /root/reference):
//   EmbeddingLayerBase, PoolingParams   include/embedding_layer.hpp:34-213
//   GPUEmbeddingLayer                   include/gpu_embedding_layer.hpp:29-41,
//                                       src/gpu_embedding_layer.cu:296-499
//   GpuTable / GPUTableConfig           include/gpu_table.hpp:44-74, src/gpu_table.cu
//   LinearUVMEmbeddingLayer             include/linear_embedding_layer.hpp:34-43,
//                                       src/linear_embedding_layer.cu:48-209
//   insert heuristics                   include/insert_heuristic.hpp, src/insert_heuristic.cpp
#pragma once

#include <atomic>
#include <memory>
#include <mutex>
#include <random>
#include <shared_mutex>
#include <string>
#include <vector>

#include "dtypes.hpp"
#include "kernels/launch.hpp"
#include "runtime.hpp"

namespace nve_amd {

// PoolingParams (embedding_layer.hpp:44-64): ids are the C ABI's enum values.
struct PoolingParams {
  int pooling_type = NVE_POOL_CONCATENATE;
  int sparse_type = NVE_SPARSE_FIXED;
  const void* csr_offsets = nullptr;
  int64_t num_csr_offsets = 0;
  int64_t fixed_hotness = 0;
  const void* weights = nullptr;
  int weight_type = kUnknown;
  int output_type = kUnknown;
};

inline bool is_weighted_pooling(int p) {
  return p == NVE_POOL_WEIGHTED_SUM || p == NVE_POOL_WEIGHTED_MEAN;
}
inline bool is_mean_pooling(int p) { return p == NVE_POOL_MEAN || p == NVE_POOL_WEIGHTED_MEAN; }

// layer_utils.cpp:277-305 / :307-328
void validate_pool_params(const PoolingParams& pp);
int64_t lookup_output_rows(int64_t num_keys, const PoolingParams* pp);

// ---------------------------------------------------------------------------
class EmbeddingLayer {
 public:
  explicit EmbeddingLayer(int key_bytes, int device) : key_bytes_(key_bytes), device_(device) {}
  virtual ~EmbeddingLayer() = default;

  virtual void lookup(ExecutionContext& ctx, int64_t num_keys, const void* keys, void* output,
                      int64_t output_stride, uint64_t* hitmask, const PoolingParams* pp,
                      float* hitrates) = 0;
  virtual void insert(ExecutionContext& ctx, int64_t n, const void* keys, int64_t value_stride,
                      int64_t value_size, const void* values, int64_t table_id);
  virtual void update(ExecutionContext& ctx, int64_t n, const void* keys, int64_t value_stride,
                      int64_t value_size, const void* values, int64_t table_id);
  virtual void accumulate(ExecutionContext& ctx, int64_t n, const void* keys,
                          int64_t value_stride, int64_t value_size, const void* values,
                          int value_type, int64_t table_id);
  virtual void clear(ExecutionContext& ctx);
  virtual void erase(ExecutionContext& ctx, int64_t n, const void* keys, int64_t table_id);
  virtual std::shared_ptr<ExecutionContext> create_execution_context(
      hipStream_t lookup, hipStream_t modify, std::shared_ptr<ThreadPool> pool);
  virtual int64_t num_tables() const { return 1; }
  // the registry a context of this layer adds its lookup stream to (none: the
  // layer's modifies need no lookup ordered before them)
  virtual std::shared_ptr<LookupStreams> lookup_streams() const { return nullptr; }

  int key_bytes() const { return key_bytes_; }
  int device() const { return device_; }

 protected:
  int key_bytes_;
  int device_;
};

// ---------------------------------------------------------------------------
// GPUEmbeddingLayer: linear table fully in HBM.
// ---------------------------------------------------------------------------
struct GPUEmbeddingLayerConfig {
  std::string layer_name;
  int device_id = 0;
  void* embedding_table = nullptr;
  int64_t num_embeddings = 0;
  int64_t embedding_width_in_bytes = 0;
  int value_dtype = kUnknown;
  int64_t default_row_index = -1;
};

class GPUEmbeddingLayer : public EmbeddingLayer {
 public:
  GPUEmbeddingLayer(int key_bytes, const GPUEmbeddingLayerConfig& cfg);
  void lookup(ExecutionContext& ctx, int64_t num_keys, const void* keys, void* output,
              int64_t output_stride, uint64_t* hitmask, const PoolingParams* pp,
              float* hitrates) override;
  // gpu_embedding_layer.cu:500-639: update / accumulate write the HBM table;
  // insert, clear and erase have no effect on a linear table.
  void insert(ExecutionContext& ctx, int64_t n, const void* keys, int64_t value_stride,
              int64_t value_size, const void* values, int64_t table_id) override;
  void update(ExecutionContext& ctx, int64_t n, const void* keys, int64_t value_stride,
              int64_t value_size, const void* values, int64_t table_id) override;
  void accumulate(ExecutionContext& ctx, int64_t n, const void* keys, int64_t value_stride,
                  int64_t value_size, const void* values, int value_type,
                  int64_t table_id) override;
  void clear(ExecutionContext& ctx) override;
  void erase(ExecutionContext& ctx, int64_t n, const void* keys, int64_t table_id) override;
  const GPUEmbeddingLayerConfig& config() const { return cfg_; }
  std::shared_ptr<LookupStreams> lookup_streams() const override { return lookups_; }

 private:
  GPUEmbeddingLayerConfig cfg_;
  std::mutex launch_mu_;  // lookups are serialised like kernel_launch_mutex_
  std::shared_ptr<LookupStreams> lookups_ = std::make_shared<LookupStreams>();
};

// ---------------------------------------------------------------------------
// GpuTable: one 8-way set-associative cache in HBM plus an optional
// host-linear backing table (misses read from it directly).
// ---------------------------------------------------------------------------
struct GPUTableConfig {
  int device_id = 0;
  uint64_t cache_size = 0;
  int64_t row_size_in_bytes = 0;
  void* uvm_table = nullptr;
  int64_t uvm_num_rows = 0;
  bool count_misses = true;
  int64_t max_modify_size = 1 << 20;
  int value_dtype = kUnknown;
  hipStream_t private_stream = nullptr;
  bool disable_uvm_update = false;
  bool uvm_cpu_accumulate = true;
  bool data_storage_on_host = false;
  bool modify_on_gpu = true;
  uint64_t kernel_mode_type = 0;
  uint64_t kernel_mode_value = 0;
  int64_t invalid_key = -1;
};

class GpuTable {
 public:
  static constexpr int kWays = 8;
  GpuTable(int key_bytes, const GPUTableConfig& cfg);
  ~GpuTable();

  const GPUTableConfig& config() const { return cfg_; }
  int key_bytes() const { return key_bytes_; }
  uint64_t num_sets() const { return num_sets_; }
  RowSource row_source(bool with_uvm) const;

  // Table API (table.hpp:130-180)
  void find(ExecutionContext& ctx, int64_t n, const void* keys, uint64_t* hit_mask,
            int64_t value_stride, void* values, int64_t* value_sizes);
  void insert(ExecutionContext& ctx, int64_t n, const void* keys, int64_t value_stride,
              int64_t value_size, const void* values);
  void insert_from_uvm(ExecutionContext& ctx, int64_t n, const void* keys);  // gpu_table.cu:494-576
  void erase(ExecutionContext& ctx, int64_t n, const void* keys);
  void clear(ExecutionContext& ctx);
  // gpu_table.cu:579-681 / :683-1046: resident keys' cache rows are
  // overwritten (update) or added to (update_accumulate, f32/f16 of the
  // table's type); the backing table gets the same change unless
  // disable_uvm_update is set.
  void update(ExecutionContext& ctx, int64_t n, const void* keys, int64_t value_stride,
              int64_t value_size, const void* values);
  void update_accumulate(ExecutionContext& ctx, int64_t n, const void* keys, int64_t value_stride,
                         int64_t value_size, const void* values, int update_dtype);

  // GpuTable::find_and_pool (gpu_table.cu:1049-1104), keys already on the device.
  void find_and_pool(ExecutionContext& ctx, int64_t n, const void* d_keys, const PoolingParams& pp,
                     void* d_output, int64_t output_stride);

  // state transfer for checkpoint-like restore and tests: tags (num_sets*8 of
  // the key type), counters (num_sets*8 float), set timestamps (num_sets int64)
  void export_state(void* tags, float* counters, int64_t* set_ts, int64_t* global_ts);
  void import_state(const void* tags, const float* counters, const int64_t* set_ts,
                    int64_t global_ts);
  void* data_ptr() const { return data_; }

  std::shared_mutex& uvm_mutex() { return uvm_mu_; }
  // lookup streams of every context that reads this table (the private
  // stream included): inserts, updates and erases order themselves after them
  const std::shared_ptr<LookupStreams>& lookup_streams() const { return lookups_; }

 private:
  // runs on stream s (the modify stream or the table's private stream)
  void modify_insert(ExecutionContext& ctx, hipStream_t s, int64_t n, const void* keys,
                     const uint8_t* rows, int64_t row_stride, bool from_uvm);
  // modify_on_gpu = false (CacheSAHostModify): the policy runs on the host
  // over a host copy of the tags and the counters, then the chosen ways go
  // through the same invalidate -> drain -> copy -> commit kernels
  void host_modify_insert(ExecutionContext& ctx, hipStream_t s, int64_t n, const void* keys,
                          const uint8_t* rows, int64_t row_stride, bool from_uvm);
  // records (slot = set*8 + way, new tag, source row) to the device; with
  // invalidate_only the ways are emptied and nothing is copied
  void apply_records(ExecutionContext& ctx, hipStream_t s, const std::vector<uint64_t>& slot,
                     const std::vector<int64_t>& tag, const std::vector<uint64_t>& src,
                     bool invalidate_only);
  int64_t h_tag(uint64_t slot) const;
  void set_h_tag(uint64_t slot, int64_t tag);
  // ec_hash.h:36-60 on the host (unsigned arithmetic in the key's width)
  int64_t load_key(const uint8_t* keys, int64_t i) const;
  uint64_t set_of(int64_t key) const;
  int64_t tag_of(int64_t key) const;
  int64_t key_of(int64_t tag, uint64_t set) const;
  // lookup modes over the backing table (gpu_table.cu:271-287): the direct
  // lookup, SortGather (misses and hits sorted apart) and PipelineGather
  // (host threads copy the missed rows); all write the same output
  enum class UvmMode { Lookup, SortGather, PipelineGather };
  UvmMode uvm_mode(int64_t n) const;
  void find_sort_gather(ExecutionContext& ctx, const GatherLaunch& g, hipStream_t s);
  void find_pipeline_gather(ExecutionContext& ctx, const GatherLaunch& g, hipStream_t s);
  // cache rows of resident keys: invalidate -> drain -> copy or add -> commit
  void modify_rows(ExecutionContext& ctx, hipStream_t s, int64_t n, const void* d_keys,
                   const uint8_t* d_vals, int64_t value_stride, bool accumulate, int dtype);
  void build_decay_table();
  // the device-policy insert with the hashed histogram (large caches); false:
  // a set had too many candidates and nothing changed (the sorted histogram redoes it)
  bool hashed_insert(ExecutionContext& ctx, hipStream_t s, int64_t n, const void* d_keys,
                     const uint8_t* rows, int64_t row_stride, bool from_uvm);
  int key_bytes_;
  GPUTableConfig cfg_;
  uint64_t num_sets_ = 0;
  uint8_t* data_ = nullptr;
  void* tags_ = nullptr;
  float* counters_ = nullptr;
  int64_t* set_ts_ = nullptr;
  // per-set words of the hashed histogram (device policy): kSetClean between
  // inserts; an insert that failed part way leaves them to be cleaned first
  uint64_t* set_word_ = nullptr;
  bool set_words_dirty_ = false;
  int64_t global_ts_ = 0;
  // host policy state (modify_on_gpu = false): a copy of the device tags kept
  // in step by every modify, the way counters and the set timestamps
  std::vector<uint8_t> h_tags_;
  std::vector<float> h_counters_;
  std::vector<int64_t> h_set_ts_;
  float decay_rate_ = 0.95f;  // EmbedCacheSA::CacheConfig default (ec_set_associative.h:120)
  float* decay_table_ = nullptr;
  int64_t decay_len_ = 0;
  uint64_t pipeline_task_size_ = 1024;  // PipelineGather keys per host task
  std::mutex modify_mu_;        // one modify at a time
  std::shared_mutex uvm_mu_;    // lookups shared, modifies exclusive
  std::shared_ptr<LookupStreams> lookups_ = std::make_shared<LookupStreams>();
};

// ---------------------------------------------------------------------------
// insert heuristics (insert_heuristic.hpp:28-60)
// ---------------------------------------------------------------------------
class InsertHeuristic {
 public:
  virtual ~InsertHeuristic() = default;
  virtual bool insert_needed(float hitrate, size_t table_id) = 0;
};

// DefaultInsertHeuristic (insert_heuristic.cpp:27-36): draw u in [0,1) from a
// seeded mt19937; insert when u < (1-h) below the threshold, else u < (1-h)^3.
class DefaultInsertHeuristic : public InsertHeuristic {
 public:
  explicit DefaultInsertHeuristic(std::vector<float> thresholds);
  bool insert_needed(float hitrate, size_t table_id) override;

 private:
  std::vector<float> thresholds_;
  std::mt19937 gen_;                           // seed 98437598437 (insert_heuristic.hpp:48)
  std::uniform_real_distribution<double> dis_;  // [0, 1)
  std::mutex mu_;
};

class NeverInsertHeuristic : public InsertHeuristic {
 public:
  bool insert_needed(float, size_t) override { return false; }
};

// ---------------------------------------------------------------------------
// LinearUVMEmbeddingLayer: GPU cache over a host-linear table.
// ---------------------------------------------------------------------------
struct LinearUVMLayerConfig {
  std::string layer_name;
  std::shared_ptr<InsertHeuristic> insert_heuristic;
  int64_t min_insert_freq_gpu = 0;
  int64_t min_insert_size_gpu = 1 << 16;
  int64_t default_row_index = -1;
};

class LinearUVMEmbeddingLayer : public EmbeddingLayer {
 public:
  LinearUVMEmbeddingLayer(int key_bytes, const LinearUVMLayerConfig& cfg,
                          std::shared_ptr<GpuTable> table);
  void lookup(ExecutionContext& ctx, int64_t num_keys, const void* keys, void* output,
              int64_t output_stride, uint64_t* hitmask, const PoolingParams* pp,
              float* hitrates) override;
  void insert(ExecutionContext& ctx, int64_t n, const void* keys, int64_t value_stride,
              int64_t value_size, const void* values, int64_t table_id) override;
  void update(ExecutionContext& ctx, int64_t n, const void* keys, int64_t value_stride,
              int64_t value_size, const void* values, int64_t table_id) override;
  void accumulate(ExecutionContext& ctx, int64_t n, const void* keys, int64_t value_stride,
                  int64_t value_size, const void* values, int value_type,
                  int64_t table_id) override;
  void clear(ExecutionContext& ctx) override;
  void erase(ExecutionContext& ctx, int64_t n, const void* keys, int64_t table_id) override;

  GpuTable& table() { return *table_; }
  std::shared_ptr<LookupStreams> lookup_streams() const override { return table_->lookup_streams(); }

 private:
  void auto_insert(ExecutionContext& ctx, int64_t n, const void* d_keys, const void* d_out,
                   int64_t out_stride, bool from_uvm, float hitrate);
  void reset_collection();  // with collect_mu_ held
  struct CollectedRows;     // device copy of the collected lookups' output rows
  LinearUVMLayerConfig cfg_;
  std::shared_ptr<GpuTable> table_;
  std::mutex collect_mu_;
  std::vector<uint8_t> collected_;  // keys gathered for the next insert
  int64_t collected_n_ = 0;
  // A collection of plain lookups keeps their output rows and inserts those;
  // one that a pooled lookup joined inserts from the backing table.
  bool collection_is_uvm_ = false;
  int64_t collected_stride_ = 0;                   // output stride of a collection of rows
  std::shared_ptr<CollectedRows> collected_rows_;  // shared with the insert task that reads it
  int64_t insert_wait_ = 0;                       // lookups to skip before the next collection
  std::shared_ptr<std::atomic<bool>> in_flight_;  // an auto-insert task is running
};

}  // namespace nve_amd
