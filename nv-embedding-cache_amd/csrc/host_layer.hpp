// host_layer.hpp -- the CPU-only tier: a linear table in host memory and the
// host embedding layer over it.  Neither enters the HIP runtime when every
// buffer it is given is host memory, so both run on machines without a GPU.
//
// Reference counterparts (file:line in /root/reference):
//   LinearHostTable, LinearHostTableConfig   include/linear_host_table.hpp:36-183,
//                                            src/linear_host_table.cpp:21-28
//   HostEmbeddingLayer                       include/host_embedding_layer.hpp:32-85,
//                                            src/host_embedding_layer.cpp:29-320
//   pool_gathered_host                       src/layer_utils.cpp:331-515
#pragma once

#include <memory>
#include <string>
#include <vector>

#include "layers.hpp"

namespace nve_amd {

struct LinearHostTableConfig {
  void* emb_table = nullptr;  // num_rows * row_bytes bytes of host memory, owned by the caller
  int64_t num_rows = 0;
  int64_t row_bytes = 0;  // max_value_size: bytes of one stored row
  int value_dtype = kUnknown;
  int64_t max_threads = INT64_MAX;  // tasks per operation at most this many
  int64_t invalid_key = -1;
};

// Dense host table indexed by key: row k at emb_table + k * row_bytes.
// Keys outside [0, num_rows) resolve to nothing.  Insert, erase and clear have
// no effect (linear_host_table.hpp:75-76,84-87,113-117).
class LinearHostTable {
 public:
  LinearHostTable(int key_bytes, const LinearHostTableConfig& cfg);

  int key_bytes() const { return key_bytes_; }
  const LinearHostTableConfig& config() const { return cfg_; }

  // find (linear_host_table.hpp:89-121): rows of the keys whose hit bit is not
  // set yet into values + i*value_stride, their hit bits set; the context's
  // lookup counter grows by the number of rows found.  keys, hit_mask and
  // values are host memory.
  int64_t find(ExecutionContext& ctx, int64_t n, const void* keys, uint64_t* hit_mask,
               int64_t value_stride, void* values);
  // find through the table C API: buffers may be device memory (staged).
  void find_any(ExecutionContext& ctx, int64_t n, const void* keys, uint64_t* hit_mask,
                int64_t value_stride, void* values, int64_t* value_sizes);
  void update(ExecutionContext& ctx, int64_t n, const void* keys, int64_t value_stride,
              int64_t value_size, const void* values);
  void update_accumulate(ExecutionContext& ctx, int64_t n, const void* keys, int64_t value_stride,
                         int64_t value_size, const void* values, int value_type);
  std::shared_ptr<ExecutionContext> create_execution_context(hipStream_t lookup, hipStream_t modify,
                                                             std::shared_ptr<ThreadPool> pool);

 private:
  int64_t threads(ExecutionContext& ctx) const;
  int key_bytes_;
  LinearHostTableConfig cfg_;
};

struct HostEmbeddingLayerConfig {
  std::string layer_name;
  std::vector<uint8_t> default_embedding;  // one row, or empty: missed keys left as they are
};

class HostEmbeddingLayer : public EmbeddingLayer {
 public:
  HostEmbeddingLayer(int key_bytes, const HostEmbeddingLayerConfig& cfg,
                     std::shared_ptr<LinearHostTable> table);
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
  std::shared_ptr<ExecutionContext> create_execution_context(
      hipStream_t lookup, hipStream_t modify, std::shared_ptr<ThreadPool> pool) override;

  LinearHostTable& table() { return *table_; }

 private:
  // pool_gathered_host (layer_utils.cpp:331-515): `gathered` holds one stored
  // row per key (host memory); the result goes to `out` (host memory).
  void pool_gathered(ExecutionContext& ctx, const PoolingParams& pp, const uint8_t* gathered,
                     int64_t num_keys, uint8_t* out, int64_t output_stride, int64_t out_rows);
  HostEmbeddingLayerConfig cfg_;
  std::shared_ptr<LinearHostTable> table_;
};

}  // namespace nve_amd
