// c_api.cpp -- the extern "C" boundary (include/nve_c_api.h).
//
// Restates the reference's C-ABI conventions (src/nve_c_api_*.cpp): null
// handles are rejected with NVE_ERROR_INVALID_ARGUMENT before any work; every
// exception becomes a status (nve_c_api_internal.hpp:48-92) with its message
// kept in thread-local storage for nve_get_last_error.
#include <algorithm>
#include <cstring>
#include <new>

#include "../../include/nve_amd_ext.h"
#include "backprop.hpp"
#include "dedup.hpp"
#include "host_layer.hpp"
#include "kernels/noalloc_launch.hpp"
#include "layers.hpp"
#include "trace.hpp"

using namespace nve_amd;

struct nve_context_s {
  std::shared_ptr<ExecutionContext> ptr;
};
// A table handle holds a GPU table (8-way cache) or a linear host table.
struct nve_table_s {
  std::shared_ptr<GpuTable> ptr;
  std::shared_ptr<LinearHostTable> host;
};
struct nve_layer_s {
  std::shared_ptr<EmbeddingLayer> ptr;
};
struct nve_thread_pool_s {
  std::shared_ptr<ThreadPool> ptr;
};
struct nve_heuristic_s {
  std::shared_ptr<InsertHeuristic> ptr;
};
struct nve_allocator_s {
  int unused;
};
struct nve_table_factory_s {
  int unused;
};

namespace {

thread_local std::string g_last_error;

nve_status_t set_error(nve_status_t s, const std::string& m) {
  g_last_error = m;
  // rejected arguments and unsupported features are the caller's to handle
  const bool expected = s == NVE_ERROR_INVALID_ARGUMENT || s == NVE_ERROR_NOT_IMPLEMENTED;
  log_at(expected ? LogLevel::Info : LogLevel::Error, "status ", (int)s, ": ", m);
  return s;
}

#define C_TRY try {
#define C_CATCH                                                             \
  }                                                                         \
  catch (const Error& e) {                                                  \
    return set_error(e.status(), e.what());                                 \
  }                                                                         \
  catch (const std::bad_alloc&) {                                           \
    return set_error(NVE_ERROR_OUT_OF_MEMORY, "Out of memory");             \
  }                                                                         \
  catch (const std::invalid_argument& e) {                                  \
    return set_error(NVE_ERROR_INVALID_ARGUMENT, e.what());                 \
  }                                                                         \
  catch (const std::exception& e) {                                         \
    return set_error(NVE_ERROR_RUNTIME, e.what());                          \
  }                                                                         \
  catch (...) {                                                             \
    return set_error(NVE_ERROR_RUNTIME, "Unknown error");                   \
  }

int key_bytes_of(nve_key_type_t t) {
  if (t == NVE_KEY_INT32) return 4;
  if (t == NVE_KEY_INT64) return 8;
  throw Error(NVE_ERROR_INVALID_ARGUMENT, cat("Unsupported key type ", (int)t));
}

std::shared_ptr<ThreadPool> unwrap(nve_thread_pool_t p) { return p ? p->ptr : nullptr; }

int dtype_in(nve_data_type_t d) {
  switch (d) {
    case NVE_DTYPE_UNKNOWN:
    case NVE_DTYPE_FLOAT32:
    case NVE_DTYPE_BFLOAT16:
    case NVE_DTYPE_FLOAT16:
    case NVE_DTYPE_E4M3:
    case NVE_DTYPE_E5M2:
    case NVE_DTYPE_FLOAT64:
    case NVE_DTYPE_QINT8_ROWWISE_F32:
    case NVE_DTYPE_QINT8_ROWWISE_F16:
    case NVE_DTYPE_QUINT8_ROWWISE_F32:
    case NVE_DTYPE_QUINT8_ROWWISE_F16:
    case kXI8AF32:
    case kXE4M3F32: return (int)d;
    default: return kUnknown;
  }
}

}  // namespace

extern "C" {

nve_status_t nve_get_last_error(const char** message) {
  if (message) *message = g_last_error.c_str();
  return NVE_SUCCESS;
}

// ---- config defaults (nve_c_api_util.cpp:49-129) ----
nve_gpu_table_config_t nve_gpu_table_config_default(void) {
  nve_gpu_table_config_t c;
  std::memset(&c, 0, sizeof(c));
  c.device_id = 0;
  c.count_misses = 1;
  c.max_modify_size = 1 << 20;
  c.value_dtype = NVE_DTYPE_UNKNOWN;
  c.uvm_cpu_accumulate = 1;
  c.modify_on_gpu = 1;
  c.invalid_key = -1;
  return c;
}

nve_gpu_embedding_layer_config_t nve_gpu_embedding_layer_config_default(void) {
  nve_gpu_embedding_layer_config_t c;
  std::memset(&c, 0, sizeof(c));
  c.layer_name = "";
  c.value_dtype = NVE_DTYPE_UNKNOWN;
  c.default_row_index = -1;
  return c;
}

nve_linear_uvm_layer_config_t nve_linear_uvm_layer_config_default(void) {
  nve_linear_uvm_layer_config_t c;
  std::memset(&c, 0, sizeof(c));
  c.layer_name = "";
  c.min_insert_size_gpu = 1 << 16;
  c.default_row_index = -1;
  return c;
}

nve_hierarchical_layer_config_t nve_hierarchical_layer_config_default(void) {
  nve_hierarchical_layer_config_t c;
  std::memset(&c, 0, sizeof(c));
  c.layer_name = "";
  c.min_insert_size_gpu = 1 << 16;
  return c;
}

nve_host_embedding_layer_config_t nve_host_embedding_layer_config_default(void) {
  nve_host_embedding_layer_config_t c;
  std::memset(&c, 0, sizeof(c));
  c.layer_name = "";
  return c;
}

nve_overflow_policy_config_t nve_overflow_policy_config_default(void) {
  nve_overflow_policy_config_t c;
  std::memset(&c, 0, sizeof(c));
  c.overflow_margin = INT64_MAX - 1023;  // disables overflow checks
  c.handler = NVE_OVERFLOW_EVICT_RANDOM;
  c.resolution_margin = 0.8;
  return c;
}

nve_host_table_config_t nve_host_table_config_default(void) {
  nve_host_table_config_t c;
  std::memset(&c, 0, sizeof(c));
  c.key_size = 8;
  c.max_value_size = 8;
  c.value_dtype = NVE_DTYPE_UNKNOWN;
  c.invalid_key = -1;
  return c;
}

// ---- version ----
nve_status_t nve_version(int32_t* major, int32_t* minor, int32_t* patch) {
  if (!major || !minor || !patch)
    return set_error(NVE_ERROR_INVALID_ARGUMENT, "Output pointers must not be NULL");
  *major = 26;  // API level of the reference release this library replaces (26.09.0)
  *minor = 9;
  *patch = 0;
  return NVE_SUCCESS;
}

nve_status_t nve_abi_version(int32_t* major, int32_t* minor) {
  if (!major || !minor) return set_error(NVE_ERROR_INVALID_ARGUMENT, "Output pointers must not be NULL");
  *major = NVE_C_ABI_VERSION_MAJOR;
  *minor = NVE_C_ABI_VERSION_MINOR;
  return NVE_SUCCESS;
}

// ---- thread pool ----
// thread_pool.cpp:46-68: "simple" (the default) and "numa" name the reference's
// implementations; a NUMA-pinned pool is not part of this build, so "numa"
// makes the same worker pool as "simple".
static int64_t thread_pool_workers(const char* json_config) {
  const std::string impl = json_string_field(json_config, "implementation", "simple");
  NVE_CHECK(impl == "simple" || impl == "numa", "Thread pool implementation '", impl, "' not found!");
  const int64_t n = json_int_field(json_config, "num_workers", 0);
  NVE_CHECK_ARG(n >= 0, "num_workers must not be negative");
  return n;
}

nve_status_t nve_thread_pool_create(nve_thread_pool_t* out, const char* json_config) {
  if (!out || !json_config)
    return set_error(NVE_ERROR_INVALID_ARGUMENT, "out and json_config must not be NULL");
  *out = nullptr;
  C_TRY
  *out = new nve_thread_pool_s{std::make_shared<ThreadPool>(thread_pool_workers(json_config))};
  return NVE_SUCCESS;
  C_CATCH
}

nve_status_t nve_thread_pool_destroy(nve_thread_pool_t pool) {
  if (!pool) return set_error(NVE_ERROR_INVALID_ARGUMENT, "pool must not be NULL");
  C_TRY
  delete pool;
  return NVE_SUCCESS;
  C_CATCH
}

nve_status_t nve_thread_pool_num_workers(nve_thread_pool_t pool, int64_t* out) {
  if (!pool || !pool->ptr || !out)
    return set_error(NVE_ERROR_INVALID_ARGUMENT, "pool and out must not be NULL");
  *out = pool->ptr->num_workers();
  return NVE_SUCCESS;
}

nve_status_t nve_configure_default_thread_pool(const char* json_config) {
  if (!json_config) return set_error(NVE_ERROR_INVALID_ARGUMENT, "json_config must not be NULL");
  C_TRY
  ThreadPool::configure_default(thread_pool_workers(json_config));
  return NVE_SUCCESS;
  C_CATCH
}

// ---- heuristics ----
nve_status_t nve_heuristic_create_default(nve_heuristic_t* out, const float* thresholds,
                                          int64_t num_thresholds) {
  if (!out) return set_error(NVE_ERROR_INVALID_ARGUMENT, "out must not be NULL");
  if (num_thresholds < 0 || (num_thresholds > 0 && !thresholds))
    return set_error(NVE_ERROR_INVALID_ARGUMENT, "thresholds must hold num_thresholds values");
  C_TRY
  std::vector<float> t;
  if (num_thresholds == 0)
    t.push_back(0.75f);
  else
    t.assign(thresholds, thresholds + num_thresholds);
  for (float v : t) NVE_CHECK_ARG(v >= 0.0f && v <= 1.0f, "thresholds must be in [0, 1]");
  *out = new nve_heuristic_s{std::make_shared<DefaultInsertHeuristic>(std::move(t))};
  return NVE_SUCCESS;
  C_CATCH
}

nve_status_t nve_heuristic_create_never(nve_heuristic_t* out) {
  if (!out) return set_error(NVE_ERROR_INVALID_ARGUMENT, "out must not be NULL");
  C_TRY
  *out = new nve_heuristic_s{std::make_shared<NeverInsertHeuristic>()};
  return NVE_SUCCESS;
  C_CATCH
}

nve_status_t nve_heuristic_destroy(nve_heuristic_t heuristic) {
  if (!heuristic) return set_error(NVE_ERROR_INVALID_ARGUMENT, "heuristic must not be NULL");
  delete heuristic;
  return NVE_SUCCESS;
}

// ---- contexts ----
nve_status_t nve_context_destroy(nve_context_t ctx) {
  if (!ctx) return set_error(NVE_ERROR_INVALID_ARGUMENT, "ctx must not be NULL");
  C_TRY
  delete ctx;
  return NVE_SUCCESS;
  C_CATCH
}

nve_status_t nve_context_wait(nve_context_t ctx) {
  if (!ctx || !ctx->ptr) return set_error(NVE_ERROR_INVALID_ARGUMENT, "ctx must not be NULL");
  C_TRY
  ctx->ptr->wait();
  return NVE_SUCCESS;
  C_CATCH
}

nve_status_t nve_context_get_lookup_stream(nve_context_t ctx, void** out_stream) {
  if (!ctx || !ctx->ptr || !out_stream)
    return set_error(NVE_ERROR_INVALID_ARGUMENT, "ctx and out_stream must not be NULL");
  *out_stream = (void*)ctx->ptr->lookup_stream();
  return NVE_SUCCESS;
}

nve_status_t nve_context_get_modify_stream(nve_context_t ctx, void** out_stream) {
  if (!ctx || !ctx->ptr || !out_stream)
    return set_error(NVE_ERROR_INVALID_ARGUMENT, "ctx and out_stream must not be NULL");
  *out_stream = (void*)ctx->ptr->modify_stream();
  return NVE_SUCCESS;
}

// ---- GPU table ----
nve_status_t nve_gpu_table_create(nve_table_t* out, nve_key_type_t key_type,
                                  const nve_gpu_table_config_t* config, nve_allocator_t allocator) {
  if (!out || !config) return set_error(NVE_ERROR_INVALID_ARGUMENT, "out and config must not be NULL");
  C_TRY
  NVE_CHECK_ARG(allocator == nullptr, "Custom allocators are not supported by this build");
  GPUTableConfig c;
  c.device_id = config->device_id;
  c.cache_size = config->cache_size;
  c.row_size_in_bytes = config->row_size_in_bytes;
  c.uvm_table = config->uvm_table;
  c.uvm_num_rows = config->uvm_num_rows;
  c.count_misses = config->count_misses != 0;
  c.max_modify_size = config->max_modify_size;
  c.value_dtype = dtype_in(config->value_dtype);
  c.private_stream = (hipStream_t)config->private_stream;
  c.disable_uvm_update = config->disable_uvm_update != 0;
  c.uvm_cpu_accumulate = config->uvm_cpu_accumulate != 0;
  c.data_storage_on_host = config->data_storage_on_host != 0;
  c.modify_on_gpu = config->modify_on_gpu != 0;
  c.kernel_mode_type = config->kernel_mode_type;
  c.kernel_mode_value = config->kernel_mode_value;
  c.invalid_key = config->invalid_key;
  *out = new nve_table_s{std::make_shared<GpuTable>(key_bytes_of(key_type), c)};
  return NVE_SUCCESS;
  C_CATCH
}

nve_status_t nve_table_destroy(nve_table_t table) {
  if (!table) return set_error(NVE_ERROR_INVALID_ARGUMENT, "table must not be NULL");
  C_TRY
  delete table;
  return NVE_SUCCESS;
  C_CATCH
}

#define NEED_TABLE_CTX                                                       \
  if (!table || (!table->ptr && !table->host) || !ctx || !ctx->ptr)          \
    return set_error(NVE_ERROR_INVALID_ARGUMENT, "table and ctx must not be NULL");

// keys is the one buffer these calls cannot do without (nve_c_api_tables.cpp:97-99)
#define NEED_KEYS                                                            \
  if (n > 0 && !keys)                                                        \
    return set_error(NVE_ERROR_INVALID_ARGUMENT, "keys must not be NULL when n > 0");

nve_status_t nve_table_find(nve_table_t table, nve_context_t ctx, int64_t n, const void* keys,
                            uint64_t* hit_mask, int64_t value_stride, void* values,
                            int64_t* value_sizes) {
  NEED_TABLE_CTX
  NEED_KEYS
  C_TRY
  NVE_TRACE("nve_table_find");
  if (table->host)
    table->host->find_any(*ctx->ptr, n, keys, hit_mask, value_stride, values, value_sizes);
  else
    table->ptr->find(*ctx->ptr, n, keys, hit_mask, value_stride, values, value_sizes);
  return NVE_SUCCESS;
  C_CATCH
}

nve_status_t nve_table_insert(nve_table_t table, nve_context_t ctx, int64_t n, const void* keys,
                              int64_t value_stride, int64_t value_size, const void* values) {
  NEED_TABLE_CTX
  NEED_KEYS
  C_TRY
  NVE_TRACE("nve_table_insert");
  if (table->host) {  // a linear host table holds every row: no effect
    NVE_LOG_INFO("Inserting into linear host table has no effect");
    return NVE_SUCCESS;
  }
  table->ptr->insert(*ctx->ptr, n, keys, value_stride, value_size, values);
  return NVE_SUCCESS;
  C_CATCH
}

nve_status_t nve_table_update(nve_table_t table, nve_context_t ctx, int64_t n, const void* keys,
                              int64_t value_stride, int64_t value_size, const void* values) {
  NEED_TABLE_CTX
  NEED_KEYS
  C_TRY
  NVE_TRACE("nve_table_update");
  if (table->host)
    table->host->update(*ctx->ptr, n, keys, value_stride, value_size, values);
  else
    table->ptr->update(*ctx->ptr, n, keys, value_stride, value_size, values);
  return NVE_SUCCESS;
  C_CATCH
}

nve_status_t nve_table_update_accumulate(nve_table_t table, nve_context_t ctx, int64_t n,
                                         const void* keys, int64_t value_stride,
                                         int64_t value_size, const void* values,
                                         nve_data_type_t value_type) {
  NEED_TABLE_CTX
  NEED_KEYS
  C_TRY
  NVE_TRACE("nve_table_update_accumulate");
  if (table->host)
    table->host->update_accumulate(*ctx->ptr, n, keys, value_stride, value_size, values,
                                   dtype_in(value_type));
  else
    table->ptr->update_accumulate(*ctx->ptr, n, keys, value_stride, value_size, values,
                                  dtype_in(value_type));
  return NVE_SUCCESS;
  C_CATCH
}

nve_status_t nve_table_clear(nve_table_t table, nve_context_t ctx) {
  NEED_TABLE_CTX
  C_TRY
  NVE_TRACE("nve_table_clear");
  if (table->host) {
    NVE_LOG_INFO("Clearing linear host table has no effect");
    return NVE_SUCCESS;
  }
  table->ptr->clear(*ctx->ptr);
  return NVE_SUCCESS;
  C_CATCH
}

nve_status_t nve_table_erase(nve_table_t table, nve_context_t ctx, int64_t n, const void* keys) {
  NEED_TABLE_CTX
  NEED_KEYS
  C_TRY
  NVE_TRACE("nve_table_erase");
  if (table->host) {
    NVE_LOG_INFO("Erasing from linear host table has no effect");
    return NVE_SUCCESS;
  }
  table->ptr->erase(*ctx->ptr, n, keys);
  return NVE_SUCCESS;
  C_CATCH
}

nve_status_t nve_table_create_execution_context(nve_table_t table, nve_context_t* out,
                                                void* lookup_stream, void* modify_stream,
                                                nve_thread_pool_t thread_pool,
                                                nve_allocator_t allocator) {
  if (!table || (!table->ptr && !table->host) || !out)
    return set_error(NVE_ERROR_INVALID_ARGUMENT, "table and out must not be NULL");
  C_TRY
  NVE_CHECK_ARG(allocator == nullptr, "Custom allocators are not supported by this build");
  if (table->host) {
    *out = new nve_context_s{table->host->create_execution_context(
        (hipStream_t)lookup_stream, (hipStream_t)modify_stream, unwrap(thread_pool))};
    return NVE_SUCCESS;
  }
  auto ctx = std::make_shared<ExecutionContext>(table->ptr->config().device_id,
                                                (hipStream_t)lookup_stream,
                                                (hipStream_t)modify_stream, unwrap(thread_pool));
  ctx->watch(table->ptr->lookup_streams());
  *out = new nve_context_s{std::move(ctx)};
  return NVE_SUCCESS;
  C_CATCH
}

nve_status_t nve_table_get_device_id(const nve_table_t table, int32_t* out) {
  if (!table || (!table->ptr && !table->host) || !out)
    return set_error(NVE_ERROR_INVALID_ARGUMENT, "table and out must not be NULL");
  *out = table->host ? -1 : table->ptr->config().device_id;
  return NVE_SUCCESS;
}

nve_status_t nve_table_get_max_row_size(const nve_table_t table, int64_t* out) {
  if (!table || (!table->ptr && !table->host) || !out)
    return set_error(NVE_ERROR_INVALID_ARGUMENT, "table and out must not be NULL");
  *out = table->host ? table->host->config().row_bytes : table->ptr->config().row_size_in_bytes;
  return NVE_SUCCESS;
}

nve_status_t nve_table_get_key_size(const nve_table_t table, int64_t* out) {
  if (!table || (!table->ptr && !table->host) || !out)
    return set_error(NVE_ERROR_INVALID_ARGUMENT, "table and out must not be NULL");
  *out = table->host ? table->host->key_bytes() : table->ptr->key_bytes();
  return NVE_SUCCESS;
}

nve_status_t nve_table_reset_lookup_counter(nve_table_t table, nve_context_t ctx) {
  NEED_TABLE_CTX
  C_TRY
  if (table->host) {
    ctx->ptr->host_lookup_counter() = 0;
    return NVE_SUCCESS;
  }
  if (table->ptr->config().count_misses) {
    ScopedDevice sd(table->ptr->config().device_id);
    ctx->ptr->reset_misses();
  }
  return NVE_SUCCESS;
  C_CATCH
}

nve_status_t nve_table_get_lookup_counter(const nve_table_t table, nve_context_t ctx,
                                          int64_t* counter) {
  NEED_TABLE_CTX
  if (!counter) return set_error(NVE_ERROR_INVALID_ARGUMENT, "counter must not be NULL");
  C_TRY
  if (table->host) {  // a host table counts the keys it resolved (host_table.hpp:363)
    *counter = ctx->ptr->host_lookup_counter();
    return NVE_SUCCESS;
  }
  if (!table->ptr->config().count_misses) {
    *counter = 0;
  } else {
    ScopedDevice sd(table->ptr->config().device_id);
    *counter = ctx->ptr->read_misses();
  }
  return NVE_SUCCESS;
  C_CATCH
}

// ---- factories: plugins are not part of this build ----
nve_status_t nve_create_table_factory(nve_table_factory_t* out, const char*, const char*) {
  if (out) *out = nullptr;
  return set_error(NVE_ERROR_NOT_IMPLEMENTED, "Table plugins are not part of this build");
}
nve_status_t nve_table_factory_destroy(nve_table_factory_t factory) {
  if (!factory) return set_error(NVE_ERROR_INVALID_ARGUMENT, "factory must not be NULL");
  delete factory;
  return NVE_SUCCESS;
}
nve_status_t nve_table_factory_produce(nve_table_factory_t, int64_t, const char*, nve_table_t* out) {
  if (out) *out = nullptr;
  return set_error(NVE_ERROR_NOT_IMPLEMENTED, "Table plugins are not part of this build");
}

// ---- layers ----
nve_status_t nve_gpu_embedding_layer_create(nve_layer_t* out, nve_key_type_t key_type,
                                            const nve_gpu_embedding_layer_config_t* config,
                                            nve_allocator_t allocator) {
  if (!out || !config) return set_error(NVE_ERROR_INVALID_ARGUMENT, "out and config must not be NULL");
  C_TRY
  NVE_CHECK_ARG(allocator == nullptr, "Custom allocators are not supported by this build");
  GPUEmbeddingLayerConfig c;
  c.layer_name = config->layer_name ? config->layer_name : "";
  c.device_id = config->device_id;
  c.embedding_table = config->embedding_table;
  c.num_embeddings = config->num_embeddings;
  c.embedding_width_in_bytes = config->embedding_width_in_bytes;
  c.value_dtype = dtype_in(config->value_dtype);
  c.default_row_index = config->default_row_index;
  *out = new nve_layer_s{std::make_shared<GPUEmbeddingLayer>(key_bytes_of(key_type), c)};
  return NVE_SUCCESS;
  C_CATCH
}

nve_status_t nve_linear_uvm_layer_create(nve_layer_t* out, nve_key_type_t key_type,
                                         const nve_linear_uvm_layer_config_t* config,
                                         nve_table_t gpu_table, nve_allocator_t allocator) {
  if (!out || !config || !gpu_table || !gpu_table->ptr)
    return set_error(NVE_ERROR_INVALID_ARGUMENT, "out, config and gpu_table must not be NULL (a GPU table)");
  C_TRY
  NVE_CHECK_ARG(allocator == nullptr, "Custom allocators are not supported by this build");
  LinearUVMLayerConfig c;
  c.layer_name = config->layer_name ? config->layer_name : "";
  if (config->insert_heuristic) c.insert_heuristic = config->insert_heuristic->ptr;
  c.min_insert_freq_gpu = config->min_insert_freq_gpu;
  c.min_insert_size_gpu = config->min_insert_size_gpu;
  c.default_row_index = config->default_row_index;
  *out = new nve_layer_s{
      std::make_shared<LinearUVMEmbeddingLayer>(key_bytes_of(key_type), c, gpu_table->ptr)};
  return NVE_SUCCESS;
  C_CATCH
}

nve_status_t nve_hierarchical_layer_create(nve_layer_t* out, nve_key_type_t,
                                           const nve_hierarchical_layer_config_t*,
                                           const nve_table_t*, int64_t, nve_allocator_t) {
  if (out) *out = nullptr;
  return set_error(NVE_ERROR_NOT_IMPLEMENTED,
                   "Hierarchical (host / remote tier) layers are not part of this build");
}

nve_status_t nve_host_embedding_layer_create(nve_layer_t* out, nve_key_type_t key_type,
                                             const nve_host_embedding_layer_config_t* config,
                                             nve_table_t host_table, nve_allocator_t allocator) {
  if (!out || !config || !host_table)
    return set_error(NVE_ERROR_INVALID_ARGUMENT, "out, config and host_table must not be NULL");
  *out = nullptr;
  // host tables come from nve_amd_linear_host_table_create (the plugin
  // factories that produce other host tables are not part of this build)
  if (!host_table->host)
    return set_error(NVE_ERROR_INVALID_ARGUMENT, "host_table must be a host table (device id < 0)");
  C_TRY
  NVE_CHECK_ARG(allocator == nullptr, "Custom allocators are not supported by this build");
  HostEmbeddingLayerConfig c;
  c.layer_name = config->layer_name ? config->layer_name : "";
  if (config->default_embedding_size > 0) {
    NVE_CHECK_ARG(config->default_embedding != nullptr, "default_embedding must not be NULL");
    const uint8_t* d = static_cast<const uint8_t*>(config->default_embedding);
    c.default_embedding.assign(d, d + config->default_embedding_size);
  }
  *out = new nve_layer_s{std::make_shared<HostEmbeddingLayer>(key_bytes_of(key_type), c, host_table->host)};
  return NVE_SUCCESS;
  C_CATCH
}

nve_status_t nve_layer_destroy(nve_layer_t layer) {
  if (!layer) return set_error(NVE_ERROR_INVALID_ARGUMENT, "layer must not be NULL");
  C_TRY
  delete layer;
  return NVE_SUCCESS;
  C_CATCH
}

#define NEED_LAYER_CTX                                                       \
  if (!layer || !layer->ptr || !ctx || !ctx->ptr)                            \
    return set_error(NVE_ERROR_INVALID_ARGUMENT, "layer and ctx must not be NULL");

nve_status_t nve_layer_lookup(nve_layer_t layer, nve_context_t ctx, int64_t num_keys,
                              const void* keys, void* output, int64_t output_stride,
                              uint64_t* hitmask, float* hitrates) {
  NEED_LAYER_CTX
  C_TRY
  NVE_TRACE("nve_layer_lookup");
  layer->ptr->lookup(*ctx->ptr, num_keys, keys, output, output_stride, hitmask, nullptr, hitrates);
  return NVE_SUCCESS;
  C_CATCH
}

nve_status_t nve_layer_lookup_pooled(nve_layer_t layer, nve_context_t ctx, int64_t num_keys,
                                     const void* keys, void* output, int64_t output_stride,
                                     uint64_t* hitmask, nve_pooling_type_t pooling_type,
                                     nve_sparse_type_t sparse_type, const void* csr_offsets,
                                     int64_t num_csr_offsets, int64_t fixed_hotness,
                                     const void* weights, nve_data_type_t weight_type,
                                     nve_data_type_t output_type, float* hitrates) {
  NEED_LAYER_CTX
  C_TRY
  NVE_TRACE("nve_layer_lookup_pooled");
  const int out_t = dtype_in(output_type);
  if (out_t == kUnknown)
    return set_error(NVE_ERROR_INVALID_ARGUMENT, "output_type must be a supported, non-UNKNOWN data type");
  PoolingParams pp;
  pp.pooling_type = (int)pooling_type;
  pp.output_type = out_t;
  if (pp.pooling_type != NVE_POOL_CONCATENATE) {
    pp.sparse_type = (int)sparse_type;
    pp.csr_offsets = csr_offsets;
    pp.num_csr_offsets = num_csr_offsets;
    pp.fixed_hotness = fixed_hotness;
    pp.weights = weights;
    pp.weight_type = dtype_in(weight_type);
  }
  layer->ptr->lookup(*ctx->ptr, num_keys, keys, output, output_stride, hitmask, &pp, hitrates);
  return NVE_SUCCESS;
  C_CATCH
}

nve_status_t nve_layer_insert(nve_layer_t layer, nve_context_t ctx, int64_t num_keys,
                              const void* keys, int64_t value_stride, int64_t value_size,
                              const void* values, int64_t table_id) {
  NEED_LAYER_CTX
  C_TRY
  NVE_TRACE("nve_layer_insert");
  layer->ptr->insert(*ctx->ptr, num_keys, keys, value_stride, value_size, values, table_id);
  return NVE_SUCCESS;
  C_CATCH
}

nve_status_t nve_layer_update(nve_layer_t layer, nve_context_t ctx, int64_t num_keys,
                              const void* keys, int64_t value_stride, int64_t value_size,
                              const void* values, int64_t table_id) {
  NEED_LAYER_CTX
  C_TRY
  NVE_TRACE("nve_layer_update");
  layer->ptr->update(*ctx->ptr, num_keys, keys, value_stride, value_size, values, table_id);
  return NVE_SUCCESS;
  C_CATCH
}

nve_status_t nve_layer_accumulate(nve_layer_t layer, nve_context_t ctx, int64_t num_keys,
                                  const void* keys, int64_t value_stride, int64_t value_size,
                                  const void* values, nve_data_type_t value_type,
                                  int64_t table_id) {
  NEED_LAYER_CTX
  C_TRY
  NVE_TRACE("nve_layer_accumulate");
  layer->ptr->accumulate(*ctx->ptr, num_keys, keys, value_stride, value_size, values,
                         dtype_in(value_type), table_id);
  return NVE_SUCCESS;
  C_CATCH
}

nve_status_t nve_layer_clear(nve_layer_t layer, nve_context_t ctx) {
  NEED_LAYER_CTX
  C_TRY
  NVE_TRACE("nve_layer_clear");
  layer->ptr->clear(*ctx->ptr);
  return NVE_SUCCESS;
  C_CATCH
}

nve_status_t nve_layer_erase(nve_layer_t layer, nve_context_t ctx, int64_t num_keys,
                             const void* keys, int64_t table_id) {
  NEED_LAYER_CTX
  C_TRY
  NVE_TRACE("nve_layer_erase");
  layer->ptr->erase(*ctx->ptr, num_keys, keys, table_id);
  return NVE_SUCCESS;
  C_CATCH
}

nve_status_t nve_layer_create_execution_context(nve_layer_t layer, nve_context_t* out,
                                                void* lookup_stream, void* modify_stream,
                                                nve_thread_pool_t thread_pool,
                                                nve_allocator_t allocator) {
  if (!layer || !layer->ptr || !out)
    return set_error(NVE_ERROR_INVALID_ARGUMENT, "layer and out must not be NULL");
  C_TRY
  NVE_CHECK_ARG(allocator == nullptr, "Custom allocators are not supported by this build");
  *out = new nve_context_s{layer->ptr->create_execution_context(
      (hipStream_t)lookup_stream, (hipStream_t)modify_stream, unwrap(thread_pool))};
  return NVE_SUCCESS;
  C_CATCH
}

nve_status_t nve_layer_get_num_tables(nve_layer_t layer, int64_t* out) {
  if (!layer || !layer->ptr || !out)
    return set_error(NVE_ERROR_INVALID_ARGUMENT, "layer and out must not be NULL");
  *out = layer->ptr->num_tables();
  return NVE_SUCCESS;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// extensions (include/nve_amd_ext.h)
// ---------------------------------------------------------------------------
extern "C" {

nve_status_t nve_amd_find_and_pool(nve_key_type_t key_type, int64_t num_keys, const void* keys,
                                   const void* table, int64_t num_rows, int64_t row_size_in_bytes,
                                   nve_data_type_t value_dtype, nve_pooling_type_t pooling_type,
                                   nve_sparse_type_t sparse_type, const void* csr_offsets,
                                   int64_t num_csr_offsets, int64_t fixed_hotness,
                                   const void* weights, nve_data_type_t weight_type,
                                   nve_data_type_t output_type, void* output,
                                   int64_t output_stride, int32_t split_hint,
                                   int32_t unroll_hint, void* stream) {
  C_TRY
  NVE_TRACE("nve_amd_find_and_pool");
  const int kb = key_bytes_of(key_type);
  const int vdt = dtype_in(value_dtype);
  const int odt = dtype_in(output_type);
  NVE_CHECK_ARG(num_keys >= 0, "Invalid num_keys");
  NVE_CHECK_ARG(table != nullptr && output != nullptr && (keys != nullptr || num_keys == 0),
                "table, keys and output must not be NULL");
  NVE_CHECK_ARG(num_rows > 0 && row_size_in_bytes > 0, "Invalid table shape");
  NVE_CHECK_ARG(vdt == kF32 || vdt == kF16 || is_rowwise(vdt), "Unsupported value type ", vdt);
  const bool ext = vdt == kXI8AF32 || vdt == kXE4M3F32;
  NVE_CHECK_ARG(ext ? (odt == kF32 || odt == kF16) : odt == native_out(vdt),
                "Unsupported find_and_pool value/output type combination");
  const int oes = dtype_size(odt);
  NVE_CHECK_ARG(output_stride > 0 && output_stride % oes == 0,
                "Pooled/dequantized output stride must be a whole number of output elements");
  const int64_t count = output_stride / oes;
  const int64_t stored = is_rowwise(vdt) ? value_elem_bytes(vdt) : oes;
  NVE_CHECK_ARG(count * stored + meta_bytes(vdt) <= row_size_in_bytes,
                "Output stride implies more value elements than the stored row holds");
  if (is_rowwise(vdt)) NVE_CHECK_ARG(row_size_in_bytes % 2 == 0, "Quantized rows must have an even width");
  RowSource src{};
  src.table = static_cast<const uint8_t*>(table);
  src.row_bytes = (uint64_t)row_size_in_bytes;
  src.load_indices = 1;
  src.num_rows = (uint64_t)num_rows;
  if (pooling_type == NVE_POOL_CONCATENATE) {
    GatherLaunch g{};
    g.keys = keys;
    g.key_bytes = kb;
    g.n = num_keys;
    g.src = src;
    g.stored_dtype = vdt;
    g.count = count;
    g.raw = 0;
    g.out = output;
    g.out_stride = output_stride;
    g.out_dtype = odt;
    NVE_HIP(launch_gather(g, (hipStream_t)stream));
    return NVE_SUCCESS;
  }
  PoolingParams pp;
  pp.pooling_type = (int)pooling_type;
  pp.sparse_type = (int)sparse_type;
  pp.csr_offsets = csr_offsets;
  pp.num_csr_offsets = num_csr_offsets;
  pp.fixed_hotness = fixed_hotness;
  pp.weights = weights;
  pp.weight_type = dtype_in(weight_type);
  pp.output_type = odt;
  validate_pool_params(pp);
  PoolLaunch p{};
  p.keys = keys;
  p.key_bytes = kb;
  p.num_keys = num_keys;
  p.num_bags = lookup_output_rows(num_keys, &pp);
  if (pp.sparse_type == NVE_SPARSE_CSR) {
    p.offsets = csr_offsets;
  } else {
    p.hotness = fixed_hotness;
  }
  p.weighted = is_weighted_pooling(pp.pooling_type);
  p.mean = is_mean_pooling(pp.pooling_type);
  if (p.weighted) {
    NVE_CHECK_ARG(pp.weight_type == kF32 || pp.weight_type == kF16,
                  "Unsupported find_and_pool weight type ", pp.weight_type);
    p.weights = weights;
    p.weight_dtype = pp.weight_type;
  }
  p.src = src;
  p.stored_dtype = vdt;
  p.count = count;
  p.out = output;
  p.out_stride = output_stride;
  p.out_dtype = odt;
  p.force_split = split_hint;
  NVE_CHECK_ARG(unroll_hint == 0 || unroll_hint == 8 || unroll_hint == 16,
                "unroll_hint must be 0, 8 or 16");
  p.force_unroll = unroll_hint;
  NVE_HIP(launch_pool(p, (hipStream_t)stream));
  return NVE_SUCCESS;
  C_CATCH
}

nve_status_t nve_amd_find_and_pool_multi(nve_key_type_t key_type, int64_t num_tables,
                                         const void* const* tables, const int64_t* table_rows,
                                         int64_t row_size_in_bytes,
                                         nve_data_type_t value_dtype, int64_t batch_size,
                                         int64_t num_keys, const void* keys, const void* offsets,
                                         const void* weights, nve_data_type_t weight_type,
                                         nve_pooling_type_t pooling_type,
                                         nve_data_type_t output_type, void* output, void* stream) {
  C_TRY
  NVE_TRACE("nve_amd_find_and_pool_multi");
  const int kb = key_bytes_of(key_type);
  const int vdt = dtype_in(value_dtype);
  const int odt = dtype_in(output_type);
  NVE_CHECK_ARG(num_tables > 0 && tables != nullptr, "tables must not be empty");
  NVE_CHECK_ARG(batch_size > 0 && num_keys >= 0, "Invalid batch_size / num_keys");
  NVE_CHECK_ARG(offsets != nullptr && output != nullptr && (keys != nullptr || num_keys == 0),
                "keys, offsets and output must not be NULL");
  NVE_CHECK_ARG(vdt == kF32 || vdt == kF16 || is_rowwise(vdt), "Unsupported value type ", vdt);
  NVE_CHECK_ARG(odt == kF32 || odt == kF16, "Output type must be Float32 or Float16");
  NVE_CHECK_ARG(pooling_type >= NVE_POOL_SUM && pooling_type <= NVE_POOL_WEIGHTED_MEAN,
                "Multi-table pooling needs a reducing pooling type");
  const bool weighted = is_weighted_pooling(pooling_type);
  if (weighted) {
    NVE_CHECK_ARG(weights != nullptr, "Sparse weights are required for weighted pooling");
    NVE_CHECK_ARG(dtype_in(weight_type) == kF32 || dtype_in(weight_type) == kF16,
                  "Unsupported weight type");
  }
  const int64_t meta = meta_bytes(vdt);
  NVE_CHECK_ARG(row_size_in_bytes > meta, "Invalid row size");
  if (is_rowwise(vdt)) NVE_CHECK_ARG(row_size_in_bytes % 2 == 0, "Quantized rows must have an even width");
  const int64_t count = (row_size_in_bytes - meta) / value_elem_bytes(vdt);
  const int64_t oes = dtype_size(odt);
  for (int64_t t = 0; t < num_tables; ++t) {
    NVE_CHECK_ARG(tables[t] != nullptr, "table ", t, " is NULL");
    if (table_rows) NVE_CHECK_ARG(table_rows[t] > 0, "table ", t, " has no rows");
  }
  for (int64_t t0 = 0; t0 < num_tables; t0 += kMaxPoolTables) {
    const int64_t nt = std::min<int64_t>(kMaxPoolTables, num_tables - t0);
    PoolLaunch p{};
    p.keys = keys;
    p.key_bytes = kb;
    p.num_keys = num_keys;
    p.offsets = static_cast<const uint8_t*>(offsets) + (size_t)t0 * batch_size * kb;
    p.num_bags = nt * batch_size;
    p.weighted = weighted;
    p.mean = is_mean_pooling(pooling_type);
    if (weighted) {
      p.weights = weights;
      p.weight_dtype = dtype_in(weight_type);
    }
    p.src.row_bytes = (uint64_t)row_size_in_bytes;
    p.src.load_indices = 1;
    p.src.table = static_cast<const uint8_t*>(tables[t0]);
    p.stored_dtype = vdt;
    p.count = count;
    p.out = static_cast<uint8_t*>(output) + t0 * count * oes;
    p.out_stride = num_tables * count * oes;
    p.out_dtype = odt;
    p.num_tables = (int)nt;
    p.keys_per_bag = std::max<int64_t>(1, num_keys / (num_tables * batch_size));
    p.bags_per_table = batch_size;
    p.out_table_stride = count * oes;
    for (int64_t t = 0; t < nt; ++t) {
      p.tables[t] = static_cast<const uint8_t*>(tables[t0 + t]);
      p.table_rows[t] = table_rows ? (uint64_t)table_rows[t0 + t] : 0;  // 0: no bound check
    }
    NVE_HIP(launch_pool(p, (hipStream_t)stream));
  }
  return NVE_SUCCESS;
  C_CATCH
}

nve_status_t nve_amd_dedup_workspace_size(int64_t num_keys, uint64_t* bytes) {
  if (!bytes) return set_error(NVE_ERROR_INVALID_ARGUMENT, "bytes must not be NULL");
  if (num_keys < 0) return set_error(NVE_ERROR_INVALID_ARGUMENT, "Invalid num_keys");
  *bytes = dedup_workspace_bytes(num_keys);
  return NVE_SUCCESS;
}

nve_status_t nve_amd_dedup(nve_key_type_t key_type, int64_t num_keys, const void* keys,
                           void* unique_out, void* counts_out, void* inverse_out, void* offsets_out,
                           int64_t* num_unique, void* workspace, uint64_t workspace_bytes,
                           void* stream) {
  C_TRY
  NVE_TRACE("nve_amd_dedup");
  NVE_CHECK_ARG(num_keys >= 0, "Invalid num_keys");
  NVE_CHECK_ARG(num_unique != nullptr, "num_unique must not be NULL");
  if (num_keys > 0)
    NVE_CHECK_ARG(keys && unique_out && counts_out && inverse_out && offsets_out,
                  "keys and output buffers must not be NULL");
  *num_unique = dedup_run(key_bytes_of(key_type), num_keys, keys, unique_out, counts_out,
                          inverse_out, offsets_out, workspace, workspace_bytes, (hipStream_t)stream);
  return NVE_SUCCESS;
  C_CATCH
}

nve_status_t nve_amd_backprop_workspace_size(int64_t num_keys, int64_t num_bags,
                                             int64_t embedding_width, uint64_t* bytes) {
  C_TRY
  NVE_CHECK_ARG(bytes != nullptr, "bytes must not be NULL");
  NVE_CHECK_ARG(num_keys >= 0 && num_bags >= 0 && embedding_width > 0, "Invalid sizes");
  *bytes = backprop_workspace_bytes(num_keys, num_bags, embedding_width);
  return NVE_SUCCESS;
  C_CATCH
}

nve_status_t nve_amd_pooling_backprop(nve_key_type_t key_type, int64_t num_keys, const void* keys,
                                      nve_pooling_type_t pooling_type, nve_sparse_type_t sparse_type,
                                      const void* csr_offsets, int64_t num_csr_offsets,
                                      int64_t fixed_hotness, const void* weights,
                                      nve_data_type_t weight_type, const void* grads_in,
                                      nve_data_type_t grad_type, int64_t embedding_width,
                                      void* unique_keys_out, void* grads_out, int64_t* num_unique_out,
                                      void* workspace, uint64_t workspace_bytes, void* stream) {
  C_TRY
  NVE_TRACE("nve_amd_pooling_backprop");
  NVE_CHECK_ARG(num_keys >= 0, "Invalid num_keys");
  NVE_CHECK_ARG(num_unique_out != nullptr, "num_unique_out must not be NULL");
  const bool concat = pooling_type == NVE_POOL_CONCATENATE;
  int64_t bags = 0;
  if (!concat) {
    if (sparse_type == NVE_SPARSE_CSR) {
      NVE_CHECK_ARG(num_csr_offsets >= 1, "CSR pooling needs num_csr_offsets >= 1");
      bags = num_csr_offsets - 1;
    } else {
      NVE_CHECK_ARG(fixed_hotness > 0 && num_keys % fixed_hotness == 0,
                    "num_keys must be a multiple of fixed_hotness");
      bags = num_keys / fixed_hotness;
    }
  }
  *num_unique_out = pooling_backprop_run(key_bytes_of(key_type), num_keys, keys, (int)pooling_type,
                                         (int)sparse_type, csr_offsets, bags, fixed_hotness, weights,
                                         dtype_in(weight_type), grads_in, dtype_in(grad_type),
                                         embedding_width, unique_keys_out, grads_out, workspace,
                                         workspace_bytes, (hipStream_t)stream);
  return NVE_SUCCESS;
  C_CATCH
}

nve_status_t nve_amd_dedup_gather(nve_key_type_t key_type, int64_t num_keys, const void* keys,
                                  const void* table, int64_t num_rows, int64_t row_size_in_bytes,
                                  void* output, int64_t output_stride, void* workspace,
                                  uint64_t workspace_bytes, void* stream) {
  C_TRY
  NVE_TRACE("nve_amd_dedup_gather");
  NVE_CHECK_ARG(num_keys >= 0, "Invalid num_keys");
  NVE_CHECK_ARG(num_rows > 0 && row_size_in_bytes > 0, "Invalid table shape");
  NVE_CHECK_ARG(output_stride >= row_size_in_bytes, "output_stride is smaller than a row");
  if (num_keys > 0) NVE_CHECK_ARG(keys && table && output, "keys, table and output must not be NULL");
  dedup_gather_run(key_bytes_of(key_type), num_keys, keys, static_cast<const uint8_t*>(table),
                   num_rows, row_size_in_bytes, output, output_stride, workspace, workspace_bytes,
                   (hipStream_t)stream);
  return NVE_SUCCESS;
  C_CATCH
}

nve_status_t nve_amd_dedup_gather_noalloc(nve_key_type_t key_type, int64_t num_keys, const void* keys,
                                          const void* table, int64_t num_rows, int64_t row_size_in_bytes,
                                          void* output, int64_t output_stride, void* stream) {
  C_TRY
  NVE_TRACE("nve_amd_dedup_gather_noalloc");
  NVE_CHECK_ARG(num_keys >= 0 && num_keys <= kNoAllocMaxKeys, "num_keys must be in [0, ", kNoAllocMaxKeys,
                "] for the allocation-free dedup gather (got ", num_keys, ")");
  NVE_CHECK_ARG(num_rows > 0 && row_size_in_bytes > 0, "Invalid table shape");
  NVE_CHECK_ARG(output_stride >= row_size_in_bytes, "output_stride is smaller than a row");
  if (num_keys == 0) return NVE_SUCCESS;
  NVE_CHECK_ARG(keys && table && output, "keys, table and output must not be NULL");
  const size_t need = dedup_workspace_bytes(num_keys);
  NVE_CHECK(need <= kNoAllocScratchBytes, "The device scratch (", kNoAllocScratchBytes,
            " bytes) is smaller than the dedup workspace of ", num_keys, " keys (", need, " bytes)");
  // the GPU's scratch array, with this call ordered after the previous one
  NoAllocSession ses;
  NVE_HIP(ses.begin((hipStream_t)stream));
  dedup_gather_run(key_bytes_of(key_type), num_keys, keys, static_cast<const uint8_t*>(table), num_rows,
                   row_size_in_bytes, output, output_stride, ses.device_scratch(), need, (hipStream_t)stream);
  NVE_HIP(ses.end());
  return NVE_SUCCESS;
  C_CATCH
}

nve_status_t nve_amd_set_log_level(int32_t level) {
  if (level < 0) return set_error(NVE_ERROR_INVALID_ARGUMENT, "log level must not be negative");
  set_log_level(level);
  return NVE_SUCCESS;
}

nve_status_t nve_amd_get_log_level(int32_t* level) {
  if (!level) return set_error(NVE_ERROR_INVALID_ARGUMENT, "level must not be NULL");
  *level = log_level();
  return NVE_SUCCESS;
}

nve_status_t nve_amd_log_message(int32_t level, const char* message) {
  if (level < 0) return set_error(NVE_ERROR_INVALID_ARGUMENT, "log level must not be negative");
  if (!message) return set_error(NVE_ERROR_INVALID_ARGUMENT, "message must not be NULL");
  if (log_enabled((LogLevel)level)) log_write((LogLevel)level, message);
  return NVE_SUCCESS;
}

nve_status_t nve_amd_read_ceiling(const void* table, int64_t row_size_in_bytes, const int64_t* idx,
                                  int64_t n, uint32_t* sink, void* stream) {
  C_TRY
  NVE_CHECK_ARG(table && idx && sink, "table, idx and sink must not be NULL");
  NVE_CHECK_ARG(row_size_in_bytes > 0 && row_size_in_bytes % 16 == 0,
                "row size must be a positive multiple of 16");
  NVE_HIP(launch_read_ceiling(static_cast<const uint8_t*>(table), (uint64_t)row_size_in_bytes, idx,
                              n, sink, (hipStream_t)stream));
  return NVE_SUCCESS;
  C_CATCH
}

nve_status_t nve_amd_gpu_table_num_sets(const nve_table_t table, int64_t* out) {
  if (!table || !table->ptr || !out)
    return set_error(NVE_ERROR_INVALID_ARGUMENT, "table and out must not be NULL");
  *out = (int64_t)table->ptr->num_sets();
  return NVE_SUCCESS;
}

nve_status_t nve_amd_gpu_table_export_state(nve_table_t table, void* tags, float* counters,
                                            int64_t* set_ts, int64_t* global_ts) {
  if (!table || !table->ptr) return set_error(NVE_ERROR_INVALID_ARGUMENT, "table must not be NULL");
  C_TRY
  table->ptr->export_state(tags, counters, set_ts, global_ts);
  return NVE_SUCCESS;
  C_CATCH
}

nve_status_t nve_amd_gpu_table_import_state(nve_table_t table, const void* tags,
                                            const float* counters, const int64_t* set_ts,
                                            int64_t global_ts) {
  if (!table || !table->ptr) return set_error(NVE_ERROR_INVALID_ARGUMENT, "table must not be NULL");
  C_TRY
  table->ptr->import_state(tags, counters, set_ts, global_ts);
  return NVE_SUCCESS;
  C_CATCH
}

nve_status_t nve_amd_table_insert_from_uvm(nve_table_t table, nve_context_t ctx, int64_t n,
                                           const void* keys) {
  NEED_TABLE_CTX
  if (!table->ptr) return set_error(NVE_ERROR_INVALID_ARGUMENT, "table must be a GPU table");
  C_TRY
  NVE_TRACE("nve_amd_table_insert_from_uvm");
  table->ptr->insert_from_uvm(*ctx->ptr, n, keys);
  return NVE_SUCCESS;
  C_CATCH
}

nve_status_t nve_amd_gpu_table_data(nve_table_t table, void** out) {
  if (!table || !table->ptr || !out)
    return set_error(NVE_ERROR_INVALID_ARGUMENT, "table and out must not be NULL");
  *out = table->ptr->data_ptr();
  return NVE_SUCCESS;
}

nve_status_t nve_amd_linear_host_table_create(nve_table_t* out, nve_key_type_t key_type,
                                              const nve_host_table_config_t* config, void* emb_table,
                                              int64_t num_rows, int64_t max_threads) {
  if (!out || !config) return set_error(NVE_ERROR_INVALID_ARGUMENT, "out and config must not be NULL");
  C_TRY
  const int kb = key_bytes_of(key_type);
  NVE_CHECK_ARG(config->key_size == kb, "config->key_size (", config->key_size,
                ") differs from the key type's size (", kb, ")");
  LinearHostTableConfig c;
  c.emb_table = emb_table;
  c.num_rows = num_rows;
  c.row_bytes = config->max_value_size;
  c.value_dtype = dtype_in(config->value_dtype);
  c.max_threads = max_threads > 0 ? max_threads : INT64_MAX;
  c.invalid_key = config->invalid_key;
  *out = new nve_table_s{nullptr, std::make_shared<LinearHostTable>(kb, c)};
  return NVE_SUCCESS;
  C_CATCH
}

}  // extern "C"
