/* nve_amd.hpp -- the reference's C++ layer and table classes (namespace nve)
 * over this library's C ABI, header-only.
 *
 * Reference interfaces mirrored (file:line in the reference):
 *   EmbeddingLayerBase, PoolingParams   include/embedding_layer.hpp:34-213
 *   GPUEmbeddingLayerConfig / Layer<K>  include/gpu_embedding_layer.hpp:29-88
 *   GPUTableConfig, GpuTable<K>         include/gpu_table.hpp:44-240
 *   LinearUVMEmbeddingLayer<K>::Config  include/linear_embedding_layer.hpp:30-80
 *   HostEmbeddingLayer<K>, LinearHostTable<K>
 *                                       include/host_embedding_layer.hpp,
 *                                       include/linear_host_table.hpp:36-183
 *   context_ptr_t, thread_pool_ptr_t, allocator_ptr_t, DataType_t,
 *   PoolingType_t, SparseType_t         include/nve_types.hpp:34-271
 *   InsertHeuristic, DefaultInsertHeuristic, NeverInsertHeuristic
 *                                       include/insert_heuristic.hpp:28-60
 *
 * A C++ host written against those classes compiles against this header and
 * links with -lnve_amd: every method forwards to the C entry point of the
 * same name and throws nve::Exception (the C status and the library's
 * message) when it fails.  Differences from the reference's classes:
 *   - streams are hipStream_t;
 *   - table methods take either buffer_ptr<T> (BufferWrapper, as the
 *     reference's do) or plain pointers; host or device memory is accepted
 *     either way and staged by the library; BufferWrapper's memory types are
 *     hipMemoryType and its staging copies belong to the wrapper;
 *   - custom allocators are not supported (pass nullptr / {});
 *   - DataType_t's numeric values are the C ABI's (the names are the
 *     reference's). */
#pragma once

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#include <memory>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <vector>

#include "nve_amd_ext.h"
#include "nve_c_api.h"

namespace nve {

using bitmask64_t = uint64_t;

enum class DataType_t : uint64_t {
  Unknown = NVE_DTYPE_UNKNOWN,
  Float32 = NVE_DTYPE_FLOAT32,
  BFloat16 = NVE_DTYPE_BFLOAT16,
  Float16 = NVE_DTYPE_FLOAT16,
  E4M3 = NVE_DTYPE_E4M3,
  E5M2 = NVE_DTYPE_E5M2,
  Float64 = NVE_DTYPE_FLOAT64,
  QInt8RowwiseF32 = NVE_DTYPE_QINT8_ROWWISE_F32,
  QInt8RowwiseF16 = NVE_DTYPE_QINT8_ROWWISE_F16,
  QUint8RowwiseF32 = NVE_DTYPE_QUINT8_ROWWISE_F32,
  QUint8RowwiseF16 = NVE_DTYPE_QUINT8_ROWWISE_F16,
};
enum class SparseType_t : uint64_t { Fixed = NVE_SPARSE_FIXED, CSR = NVE_SPARSE_CSR };
enum class PoolingType_t : uint64_t {
  Concatenate = NVE_POOL_CONCATENATE,
  Sum = NVE_POOL_SUM,
  Mean = NVE_POOL_MEAN,
  WeightedSum = NVE_POOL_WEIGHTED_SUM,
  WeightedMean = NVE_POOL_WEIGHTED_MEAN,
};

class Exception : public std::runtime_error {
 public:
  Exception(nve_status_t status, const std::string& msg) : std::runtime_error(msg), status_(status) {}
  nve_status_t status() const { return status_; }

 private:
  nve_status_t status_;
};

namespace detail {
inline void check(nve_status_t s) {
  if (s == NVE_SUCCESS) return;
  const char* msg = nullptr;
  nve_get_last_error(&msg);
  throw Exception(s, msg ? msg : "nve error");
}
template <typename K>
constexpr nve_key_type_t key_type() {
  static_assert(std::is_same_v<K, int32_t> || std::is_same_v<K, int64_t>, "keys are int32_t or int64_t");
  return std::is_same_v<K, int32_t> ? NVE_KEY_INT32 : NVE_KEY_INT64;
}
inline nve_data_type_t dt(DataType_t t) { return (nve_data_type_t)t; }
}  // namespace detail

// Custom allocators are not supported by this build: allocator_ptr_t is kept
// for signatures and must be empty.
class Allocator {};
using allocator_ptr_t = std::shared_ptr<Allocator>;

class ThreadPool {
 public:
  // json_config as nve_thread_pool_create takes it, e.g. {"num_workers": 8}
  explicit ThreadPool(const std::string& json_config = "{}") {
    detail::check(nve_thread_pool_create(&h_, json_config.c_str()));
  }
  ~ThreadPool() { nve_thread_pool_destroy(h_); }
  ThreadPool(const ThreadPool&) = delete;
  ThreadPool& operator=(const ThreadPool&) = delete;
  int64_t num_workers() const {
    int64_t n = 0;
    detail::check(nve_thread_pool_num_workers(h_, &n));
    return n;
  }
  nve_thread_pool_t handle() const { return h_; }

 private:
  nve_thread_pool_t h_ = nullptr;
};
using thread_pool_ptr_t = std::shared_ptr<ThreadPool>;

class ExecutionContext {
 public:
  explicit ExecutionContext(nve_context_t h) : h_(h) {}
  ~ExecutionContext() {
    nve_context_wait(h_);
    nve_context_destroy(h_);
  }
  ExecutionContext(const ExecutionContext&) = delete;
  ExecutionContext& operator=(const ExecutionContext&) = delete;
  hipStream_t get_lookup_stream() const {
    void* s = nullptr;
    detail::check(nve_context_get_lookup_stream(h_, &s));
    return (hipStream_t)s;
  }
  hipStream_t get_modify_stream() const {
    void* s = nullptr;
    detail::check(nve_context_get_modify_stream(h_, &s));
    return (hipStream_t)s;
  }
  // waits for pending work, tasks offloaded to the thread pool included
  void wait() { detail::check(nve_context_wait(h_)); }
  nve_context_t handle() const { return h_; }

 private:
  nve_context_t h_;
};
using context_ptr_t = std::shared_ptr<ExecutionContext>;

// A named view of a caller's buffer (the reference's BufferWrapper<T>,
// include/buffer_wrapper.hpp:34-123): what the reference's table methods take
// for keys, values, hit masks and sizes.  The table methods below hand the
// caller's own pointer to the library, which reads host, pinned or device
// memory itself.  access_buffer gives a caller the buffer in another memory
// type as the reference's does (allocated on first access, contents copied
// when asked, a const buffer copied only once); those copies belong to the
// wrapper and are freed with it (the reference's belong to the context).
template <typename T>
class BufferWrapper {
 public:
  BufferWrapper(context_ptr_t& ctx, const std::string name, T* buffer, const size_t size_in_bytes)
      : ctx_(ctx), name_(std::move(name)), size_(size_in_bytes) {
    if (!ctx_) throw Exception(NVE_ERROR_INVALID_ARGUMENT, "Invalid context");
    if (!buffer) throw Exception(NVE_ERROR_INVALID_ARGUMENT, "Invalid buffer");
    last_access_ = type_of(buffer);
    slots_.push_back({last_access_, buffer, false});
  }
  BufferWrapper(const BufferWrapper&) = delete;
  BufferWrapper& operator=(const BufferWrapper&) = delete;
  ~BufferWrapper() {
    for (auto& s : slots_) {
      if (!s.owned) continue;
      void* p = const_cast<void*>(static_cast<const void*>(s.ptr));
      if (s.type == hipMemoryTypeHost)
        (void)hipHostFree(p);
      else
        (void)hipFree(p);
    }
  }

  T* access_buffer(hipMemoryType mem_type, bool copy_content, hipStream_t stream) {
    if (mem_type == hipMemoryTypeUnregistered) mem_type = hipMemoryTypeHost;
    if (mem_type != hipMemoryTypeHost && mem_type != hipMemoryTypeDevice && !get_buffer(mem_type))
      throw Exception(NVE_ERROR_INVALID_ARGUMENT, "BufferWrapper '" + name_ + "': cannot allocate this memory type");
    bool fresh = false;
    if (!get_buffer(mem_type)) {
      if (std::is_const<T>::value && !copy_content)
        throw Exception(NVE_ERROR_INVALID_ARGUMENT,
                        "BufferWrapper '" + name_ + "': a const buffer must be accessed with copy_content");
      void* p = nullptr;
      hipError_t e = mem_type == hipMemoryTypeHost ? hipHostMalloc(&p, size_ ? size_ : 1)
                                                   : hipMalloc(&p, size_ ? size_ : 1);
      if (e != hipSuccess) throw Exception(NVE_ERROR_OUT_OF_MEMORY, "BufferWrapper '" + name_ + "': allocation failed");
      slots_.push_back({mem_type, static_cast<T*>(p), true});
      fresh = true;
    }
    T* dst = get_buffer(mem_type);
    if (copy_content && (!std::is_const<T>::value || fresh)) {
      const void* src = static_cast<const void*>(get_buffer(last_access_));
      void* d = const_cast<void*>(static_cast<const void*>(dst));
      if (src != d && size_) {
        if (hipMemcpyAsync(d, src, size_, hipMemcpyDefault, stream) != hipSuccess ||
            (mem_type != hipMemoryTypeDevice && hipStreamSynchronize(stream) != hipSuccess))
          throw Exception(NVE_ERROR_CUDA, "BufferWrapper '" + name_ + "': copy failed");
      }
    }
    last_access_ = mem_type;
    return dst;
  }
  hipMemoryType get_last_access() const { return last_access_; }
  // the buffer of that memory type if the wrapper has one, else nullptr
  T* get_buffer(hipMemoryType mem_type) const {
    for (const auto& s : slots_)
      if (s.type == mem_type) return s.ptr;
    return nullptr;
  }
  // the caller's own buffer, which the table methods pass on
  T* data() const { return slots_.front().ptr; }
  size_t size() const { return size_; }
  const std::string& name() const { return name_; }

 private:
  struct Slot {
    hipMemoryType type;
    T* ptr;
    bool owned;
  };
  static hipMemoryType type_of(const void* p) {
    hipPointerAttribute_t a;
    if (hipPointerGetAttributes(&a, p) != hipSuccess) {
      (void)hipGetLastError();
      return hipMemoryTypeUnregistered;
    }
    return a.type;
  }
  context_ptr_t ctx_;
  std::string name_;
  size_t size_;
  hipMemoryType last_access_ = hipMemoryTypeUnregistered;
  std::vector<Slot> slots_;
};
template <typename T>
using buffer_ptr = std::shared_ptr<BufferWrapper<T>>;

namespace detail {
template <typename T>
T* ptr_of(const buffer_ptr<T>& b) {
  return b ? b->data() : nullptr;
}
inline nve_thread_pool_t pool_of(const thread_pool_ptr_t& p) { return p ? p->handle() : nullptr; }
inline void no_allocator(const allocator_ptr_t& a) {
  if (a) throw Exception(NVE_ERROR_INVALID_ARGUMENT, "Custom allocators are not supported by this build");
}
}  // namespace detail

// ---------------------------------------------------------------------------
// insert heuristics
// ---------------------------------------------------------------------------
class InsertHeuristic {
 public:
  virtual ~InsertHeuristic() {
    if (h_) nve_heuristic_destroy(h_);
  }
  nve_heuristic_t handle() const { return h_; }

 protected:
  nve_heuristic_t h_ = nullptr;
};
class DefaultInsertHeuristic : public InsertHeuristic {
 public:
  explicit DefaultInsertHeuristic(const std::vector<float>& thresholds = {}) {
    detail::check(nve_heuristic_create_default(&h_, thresholds.empty() ? nullptr : thresholds.data(),
                                               (int64_t)thresholds.size()));
  }
};
class NeverInsertHeuristic : public InsertHeuristic {
 public:
  NeverInsertHeuristic() { detail::check(nve_heuristic_create_never(&h_)); }
};

// ---------------------------------------------------------------------------
// tables
// ---------------------------------------------------------------------------
struct GPUTableConfig {
  int device_id{0};
  size_t cache_size{0};
  int64_t row_size_in_bytes{0};
  void* uvm_table{nullptr};
  int64_t uvm_num_rows{0};
  bool count_misses{true};
  int64_t max_modify_size{1 << 20};
  DataType_t value_dtype{DataType_t::Unknown};
  hipStream_t private_stream{nullptr};
  bool disable_uvm_update{false};
  bool uvm_cpu_accumulate{true};
  bool data_storage_on_host{false};
  bool modify_on_gpu{true};
  uint64_t kernel_mode_type{0};
  uint64_t kernel_mode_value{0};
  int64_t invalid_key{-1};
};

// Operations shared by the table classes (the reference's Table interface).
class Table {
 public:
  virtual ~Table() {
    if (h_) nve_table_destroy(h_);
  }
  Table(const Table&) = delete;
  Table& operator=(const Table&) = delete;

  void find(context_ptr_t& ctx, int64_t num_keys, const void* keys, bitmask64_t* hit_mask,
            int64_t value_stride, void* values, int64_t* value_sizes) const {
    detail::check(nve_table_find(h_, ctx->handle(), num_keys, keys, hit_mask, value_stride, values,
                                 value_sizes));
  }
  void insert(context_ptr_t& ctx, int64_t num_keys, const void* keys, int64_t value_stride,
              int64_t value_size, const void* values) {
    detail::check(nve_table_insert(h_, ctx->handle(), num_keys, keys, value_stride, value_size, values));
  }
  void update(context_ptr_t& ctx, int64_t num_keys, const void* keys, int64_t update_stride,
              int64_t update_size, const void* updates) {
    detail::check(nve_table_update(h_, ctx->handle(), num_keys, keys, update_stride, update_size, updates));
  }
  void update_accumulate(context_ptr_t& ctx, int64_t num_keys, const void* keys, int64_t update_stride,
                         int64_t update_size, const void* updates, DataType_t update_dtype) {
    detail::check(nve_table_update_accumulate(h_, ctx->handle(), num_keys, keys, update_stride,
                                              update_size, updates, detail::dt(update_dtype)));
  }
  void erase(context_ptr_t& ctx, int64_t num_keys, const void* keys) {
    detail::check(nve_table_erase(h_, ctx->handle(), num_keys, keys));
  }

  // the reference's signatures (include/table.hpp:104-180)
  template <typename T>
  using buffer_ptr = nve::buffer_ptr<T>;
  void find(context_ptr_t& ctx, int64_t n, buffer_ptr<const void> keys, buffer_ptr<bitmask64_t> hit_mask,
            int64_t value_stride, buffer_ptr<void> values, buffer_ptr<int64_t> value_sizes) const {
    find(ctx, n, detail::ptr_of(keys), detail::ptr_of(hit_mask), value_stride, detail::ptr_of(values),
         detail::ptr_of(value_sizes));
  }
  void insert(context_ptr_t& ctx, int64_t n, buffer_ptr<const void> keys, int64_t value_stride,
              int64_t value_size, buffer_ptr<const void> values) {
    insert(ctx, n, detail::ptr_of(keys), value_stride, value_size, detail::ptr_of(values));
  }
  void update(context_ptr_t& ctx, int64_t n, buffer_ptr<const void> keys, int64_t value_stride,
              int64_t value_size, buffer_ptr<const void> values) {
    update(ctx, n, detail::ptr_of(keys), value_stride, value_size, detail::ptr_of(values));
  }
  void update_accumulate(context_ptr_t& ctx, int64_t n, buffer_ptr<const void> keys, int64_t update_stride,
                         int64_t update_size, buffer_ptr<const void> updates, DataType_t update_dtype) {
    update_accumulate(ctx, n, detail::ptr_of(keys), update_stride, update_size, detail::ptr_of(updates),
                      update_dtype);
  }
  void erase(context_ptr_t& ctx, int64_t n, buffer_ptr<const void> keys) {
    erase(ctx, n, detail::ptr_of(keys));
  }
  void clear(context_ptr_t& ctx) { detail::check(nve_table_clear(h_, ctx->handle())); }
  context_ptr_t create_execution_context(hipStream_t lookup_stream, hipStream_t modify_stream,
                                         thread_pool_ptr_t thread_pool = {},
                                         allocator_ptr_t allocator = {}) {
    detail::no_allocator(allocator);
    nve_context_t c = nullptr;
    detail::check(nve_table_create_execution_context(h_, &c, (void*)lookup_stream, (void*)modify_stream,
                                                     detail::pool_of(thread_pool), nullptr));
    return std::make_shared<ExecutionContext>(c);
  }
  int32_t get_device_id() const {
    int32_t d = 0;
    detail::check(nve_table_get_device_id(h_, &d));
    return d;
  }
  int64_t get_max_row_size() const {
    int64_t r = 0;
    detail::check(nve_table_get_max_row_size(h_, &r));
    return r;
  }
  int64_t get_key_size() const {
    int64_t r = 0;
    detail::check(nve_table_get_key_size(h_, &r));
    return r;
  }
  nve_table_t handle() const { return h_; }

 protected:
  Table() = default;
  nve_table_t h_ = nullptr;
};
using table_ptr_t = std::shared_ptr<Table>;

template <typename KeyType>
class GpuTable : public Table {
 public:
  using key_type = KeyType;
  using config_type = GPUTableConfig;

  explicit GpuTable(const GPUTableConfig& config, allocator_ptr_t allocator = {}) {
    detail::no_allocator(allocator);
    nve_gpu_table_config_t c = nve_gpu_table_config_default();
    c.device_id = config.device_id;
    c.cache_size = config.cache_size;
    c.row_size_in_bytes = config.row_size_in_bytes;
    c.uvm_table = config.uvm_table;
    c.uvm_num_rows = config.uvm_num_rows;
    c.count_misses = config.count_misses;
    c.max_modify_size = config.max_modify_size;
    c.value_dtype = detail::dt(config.value_dtype);
    c.private_stream = (void*)config.private_stream;
    c.disable_uvm_update = config.disable_uvm_update;
    c.uvm_cpu_accumulate = config.uvm_cpu_accumulate;
    c.data_storage_on_host = config.data_storage_on_host;
    c.modify_on_gpu = config.modify_on_gpu;
    c.kernel_mode_type = config.kernel_mode_type;
    c.kernel_mode_value = config.kernel_mode_value;
    c.invalid_key = config.invalid_key;
    detail::check(nve_gpu_table_create(&h_, detail::key_type<KeyType>(), &c, nullptr));
  }
  // GpuTable::insert_from_uvm (gpu_table.hpp:160-167): rows come from the
  // backing table at uvm_table + key * row_size_in_bytes
  void insert_from_uvm(context_ptr_t& ctx, int64_t num_keys, const void* keys) {
    detail::check(nve_amd_table_insert_from_uvm(h_, ctx->handle(), num_keys, keys));
  }
};

// LinearHostTable over caller-owned host rows (row k at emb_table + k * max_value_size)
struct LinearHostTableConfig {
  void* emb_table{nullptr};
  int64_t num_rows{0};
  int64_t max_value_size{0};
  DataType_t value_dtype{DataType_t::Unknown};
  int64_t max_threads{0};  // tasks per operation, <= 0: no limit beyond the thread pool
  int64_t invalid_key{-1};
};

template <typename KeyType>
class LinearHostTable : public Table {
 public:
  using key_type = KeyType;
  explicit LinearHostTable(const LinearHostTableConfig& config) {
    nve_host_table_config_t c = nve_host_table_config_default();
    c.key_size = sizeof(KeyType);
    c.max_value_size = config.max_value_size;
    c.value_dtype = detail::dt(config.value_dtype);
    c.invalid_key = config.invalid_key;
    detail::check(nve_amd_linear_host_table_create(&h_, detail::key_type<KeyType>(), &c, config.emb_table,
                                                   config.num_rows, config.max_threads));
  }
};

// ---------------------------------------------------------------------------
// layers
// ---------------------------------------------------------------------------
class EmbeddingLayerBase {
 public:
  struct PoolingParams {
    PoolingType_t pooling_type{PoolingType_t::Concatenate};
    SparseType_t sparse_type{SparseType_t::Fixed};
    const void* csr_offsets{nullptr};  // of the layer's key type; CSR only
    int64_t num_csr_offsets{0};
    int64_t fixed_hotness{0};           // Fixed only
    const void* weights{nullptr};
    DataType_t weight_type{DataType_t::Unknown};
    DataType_t output_type{DataType_t::Unknown};
  };

  virtual ~EmbeddingLayerBase() {
    if (h_) nve_layer_destroy(h_);
  }
  EmbeddingLayerBase(const EmbeddingLayerBase&) = delete;
  EmbeddingLayerBase& operator=(const EmbeddingLayerBase&) = delete;

  virtual void lookup(context_ptr_t& ctx, const int64_t num_keys, const void* keys, void* output,
                      const int64_t output_stride, bitmask64_t* hitmask, const PoolingParams* pool_params,
                      float* hitrates) {
    if (pool_params == nullptr) {
      detail::check(nve_layer_lookup(h_, ctx->handle(), num_keys, keys, output, output_stride, hitmask,
                                     hitrates));
      return;
    }
    const PoolingParams& p = *pool_params;
    detail::check(nve_layer_lookup_pooled(
        h_, ctx->handle(), num_keys, keys, output, output_stride, hitmask,
        (nve_pooling_type_t)p.pooling_type, (nve_sparse_type_t)p.sparse_type, p.csr_offsets,
        p.num_csr_offsets, p.fixed_hotness, p.weights, detail::dt(p.weight_type),
        detail::dt(p.output_type), hitrates));
  }
  virtual void insert(context_ptr_t& ctx, const int64_t num_keys, const void* keys, const int64_t value_stride,
                      const int64_t value_size, const void* values, const int64_t table_id) {
    detail::check(nve_layer_insert(h_, ctx->handle(), num_keys, keys, value_stride, value_size, values,
                                   table_id));
  }
  virtual void update(context_ptr_t& ctx, const int64_t num_keys, const void* keys,
                      const int64_t vector_stride, const int64_t value_size, const void* values,
                      const int64_t table_id) {
    detail::check(nve_layer_update(h_, ctx->handle(), num_keys, keys, vector_stride, value_size, values,
                                   table_id));
  }
  virtual void accumulate(context_ptr_t& ctx, const int64_t num_keys, const void* keys,
                          const int64_t vector_stride, const int64_t value_size, const void* values,
                          DataType_t value_type, const int64_t table_id) {
    detail::check(nve_layer_accumulate(h_, ctx->handle(), num_keys, keys, vector_stride, value_size,
                                       values, detail::dt(value_type), table_id));
  }
  virtual void clear(context_ptr_t& ctx) { detail::check(nve_layer_clear(h_, ctx->handle())); }
  virtual void erase(context_ptr_t& ctx, const int64_t num_keys, const void* keys, const int64_t table_id) {
    detail::check(nve_layer_erase(h_, ctx->handle(), num_keys, keys, table_id));
  }
  virtual context_ptr_t create_execution_context(hipStream_t lookup_stream, hipStream_t modify_stream,
                                                 thread_pool_ptr_t thread_pool, allocator_ptr_t allocator) {
    detail::no_allocator(allocator);
    nve_context_t c = nullptr;
    detail::check(nve_layer_create_execution_context(h_, &c, (void*)lookup_stream, (void*)modify_stream,
                                                     detail::pool_of(thread_pool), nullptr));
    return std::make_shared<ExecutionContext>(c);
  }
  virtual int64_t get_num_tables() const {
    int64_t n = 0;
    detail::check(nve_layer_get_num_tables(h_, &n));
    return n;
  }
  nve_layer_t handle() const { return h_; }

 protected:
  EmbeddingLayerBase() = default;
  nve_layer_t h_ = nullptr;
};

struct GPUEmbeddingLayerConfig {
  std::string layer_name;
  int device_id{0};
  void* embedding_table{nullptr};
  int64_t num_embeddings{0};
  int64_t embedding_width_in_bytes{0};
  DataType_t value_dtype{DataType_t::Unknown};
  int64_t default_row_index{-1};
};

template <typename KeyType>
class GPUEmbeddingLayer : public EmbeddingLayerBase {
 public:
  using key_type = KeyType;
  explicit GPUEmbeddingLayer(const GPUEmbeddingLayerConfig& config, allocator_ptr_t allocator = {})
      : config_(config) {
    detail::no_allocator(allocator);
    nve_gpu_embedding_layer_config_t c = nve_gpu_embedding_layer_config_default();
    c.layer_name = config_.layer_name.c_str();
    c.device_id = config_.device_id;
    c.embedding_table = config_.embedding_table;
    c.num_embeddings = config_.num_embeddings;
    c.embedding_width_in_bytes = config_.embedding_width_in_bytes;
    c.value_dtype = detail::dt(config_.value_dtype);
    c.default_row_index = config_.default_row_index;
    detail::check(nve_gpu_embedding_layer_create(&h_, detail::key_type<KeyType>(), &c, nullptr));
  }
  int64_t get_num_tables() const override { return 1; }

 private:
  GPUEmbeddingLayerConfig config_;
};

template <typename KeyType>
class LinearUVMEmbeddingLayer : public EmbeddingLayerBase {
 public:
  struct Config {
    std::string layer_name;
    std::shared_ptr<InsertHeuristic> insert_heuristic = nullptr;  // nullptr: the default heuristic
    int64_t min_insert_freq_gpu{0};
    int64_t min_insert_size_gpu{1 << 16};
    int64_t default_row_index{-1};
  };
  using gpu_table_ptr_t = std::shared_ptr<GpuTable<KeyType>>;
  using key_type = KeyType;

  LinearUVMEmbeddingLayer(const Config& cfg, gpu_table_ptr_t gpu_table, allocator_ptr_t allocator = {})
      : config_(cfg), gpu_table_(std::move(gpu_table)) {
    detail::no_allocator(allocator);
    nve_linear_uvm_layer_config_t c = nve_linear_uvm_layer_config_default();
    c.layer_name = config_.layer_name.c_str();
    c.insert_heuristic = config_.insert_heuristic ? config_.insert_heuristic->handle() : nullptr;
    c.min_insert_freq_gpu = config_.min_insert_freq_gpu;
    c.min_insert_size_gpu = config_.min_insert_size_gpu;
    c.default_row_index = config_.default_row_index;
    detail::check(nve_linear_uvm_layer_create(&h_, detail::key_type<KeyType>(), &c, gpu_table_->handle(),
                                              nullptr));
  }
  // contexts and the layer go before the table they read
  ~LinearUVMEmbeddingLayer() override {
    nve_layer_destroy(h_);
    h_ = nullptr;
  }
  int64_t get_num_tables() const override { return 1; }
  const Config& get_config() const { return config_; }

 private:
  const Config config_;
  gpu_table_ptr_t gpu_table_;
};

template <typename KeyType>
class HostEmbeddingLayer : public EmbeddingLayerBase {
 public:
  struct Config {
    std::string layer_name;
    std::vector<uint8_t> default_embedding;  // empty: a missed key reads zeros
  };
  HostEmbeddingLayer(const Config& cfg, std::shared_ptr<LinearHostTable<KeyType>> table,
                     allocator_ptr_t allocator = {})
      : config_(cfg), table_(std::move(table)) {
    detail::no_allocator(allocator);
    nve_host_embedding_layer_config_t c = nve_host_embedding_layer_config_default();
    c.layer_name = config_.layer_name.c_str();
    c.default_embedding = config_.default_embedding.empty() ? nullptr : config_.default_embedding.data();
    c.default_embedding_size = (int64_t)config_.default_embedding.size();
    detail::check(nve_host_embedding_layer_create(&h_, detail::key_type<KeyType>(), &c, table_->handle(),
                                                  nullptr));
  }
  ~HostEmbeddingLayer() override {
    nve_layer_destroy(h_);
    h_ = nullptr;
  }
  int64_t get_num_tables() const override { return 1; }

 private:
  Config config_;
  std::shared_ptr<LinearHostTable<KeyType>> table_;
};

}  // namespace nve
