/*
 * nve_c_api.h -- C ABI of the MI355X (gfx950, HIP) embedding-cache lookup library.
 *
 * Drop-in for the reference's C ABI: every name, enum value and struct layout
 * below is the one declared in /root/reference/include/nve_c_api.h (NVE 26.09.0),
 * so a C/C++ inference host built against the reference header links against
 * libnve_amd.so unchanged.  Streams are hipStream_t passed as void* where the
 * reference passes cudaStream_t; NVE_ERROR_CUDA reports a HIP runtime error.
 *
 * Reference interface replaced by each group (file:line in /root/reference):
 *   status codes + last error        include/nve_c_api.h:44-62, src/nve_c_api_error.cpp
 *   enums                             include/nve_c_api.h:68-134
 *   config structs + defaults         include/nve_c_api.h:150-279
 *   version                           include/nve_c_api.h:285-300
 *   thread pool                       include/nve_c_api.h:306-333
 *   insert heuristics                 include/nve_c_api.h:339-366
 *   execution context                 include/nve_c_api.h:372-400
 *   GPU table (cache)                 include/nve_c_api.h:406-572, src/nve_c_api_tables.cpp
 *   table factories (not built here)  include/nve_c_api.h:578-610
 *   layers                            include/nve_c_api.h:616-835, src/nve_c_api_layers.cpp
 *
 * Threading and ownership follow the reference: a context is used by one thread
 * at a time; contexts are waited on and destroyed before their table or layer;
 * the caller owns every table and buffer it passes in.
 */
#ifndef NVE_C_API_H
#define NVE_C_API_H

#include <stddef.h>
#include <stdint.h>

#define NVE_C_API __attribute__((visibility("default")))

#define NVE_C_ABI_VERSION_MAJOR (1)
#define NVE_C_ABI_VERSION_MINOR (0)

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes (nve_c_api.h:46-54) ---------------------------------- */
typedef int32_t nve_status_t;
enum {
  NVE_SUCCESS = 0,
  NVE_ERROR_INVALID_ARGUMENT = 1,
  NVE_ERROR_CUDA = 2, /* a HIP runtime call failed */
  NVE_ERROR_RUNTIME = 3,
  NVE_ERROR_NOT_IMPLEMENTED = 4,
  NVE_ERROR_OUT_OF_MEMORY = 5,
};

/* Message of the last failed call on this thread; valid until the next call on
 * this thread (nve_c_api.h:56-62). */
NVE_C_API nve_status_t nve_get_last_error(const char** message);

/* ---- enumerations (nve_c_api.h:68-134) --------------------------------- */
typedef int32_t nve_data_type_t;
enum {
  NVE_DTYPE_UNKNOWN = 0,
  NVE_DTYPE_FLOAT32 = 1,
  NVE_DTYPE_BFLOAT16 = 2,
  NVE_DTYPE_FLOAT16 = 3,
  NVE_DTYPE_E4M3 = 4,
  NVE_DTYPE_E5M2 = 5,
  NVE_DTYPE_FLOAT64 = 6,
  /* int8 values then one scale per row; value = q * scale. */
  NVE_DTYPE_QINT8_ROWWISE_F32 = 7,
  NVE_DTYPE_QINT8_ROWWISE_F16 = 8,
  /* uint8 values then scale and offset per row; value = q * scale + offset. */
  NVE_DTYPE_QUINT8_ROWWISE_F32 = 9,
  NVE_DTYPE_QUINT8_ROWWISE_F16 = 10,
};

typedef enum {
  NVE_SPARSE_FIXED = 0,
  NVE_SPARSE_CSR,
} nve_sparse_type_t;

typedef enum {
  NVE_POOL_CONCATENATE = 0,
  NVE_POOL_SUM,
  NVE_POOL_MEAN,
  NVE_POOL_WEIGHTED_SUM,
  NVE_POOL_WEIGHTED_MEAN,
} nve_pooling_type_t;

typedef enum {
  NVE_PART_ALWAYS_ZERO = 0,
  NVE_PART_FOWLER_NOLL_VO,
  NVE_PART_MURMUR3,
  NVE_PART_RRXMRRXMSX0,
  NVE_PART_STD_HASH,
} nve_partitioner_t;

typedef enum {
  NVE_OVERFLOW_EVICT_RANDOM = 0,
  NVE_OVERFLOW_EVICT_LRU,
  NVE_OVERFLOW_EVICT_LFU,
} nve_overflow_handler_t;

typedef enum {
  NVE_KEY_INT32 = 0,
  NVE_KEY_INT64,
} nve_key_type_t;

typedef enum {
  NVE_KERNEL_DYNAMIC = 0,
  NVE_KERNEL_LOOKUP_UVM,
  NVE_KERNEL_SORT_GATHER,
  NVE_KERNEL_PIPELINE_GATHER,
} nve_kernel_type_t;

typedef enum {
  NVE_HEURISTIC_DEFAULT = 0,
  NVE_HEURISTIC_FSM,
  NVE_HEURISTIC_STATISTICAL,
} nve_heuristic_type_t;

/* ---- opaque handles (nve_c_api.h:140-146) ------------------------------ */
typedef struct nve_context_s* nve_context_t;
typedef struct nve_table_s* nve_table_t;
typedef struct nve_layer_s* nve_layer_t;
typedef struct nve_thread_pool_s* nve_thread_pool_t;
typedef struct nve_allocator_s* nve_allocator_t;
typedef struct nve_heuristic_s* nve_heuristic_t;
typedef struct nve_table_factory_s* nve_table_factory_t;

/* ---- configuration structs (nve_c_api.h:152-228) ----------------------- */
typedef struct {
  int32_t device_id;
  uint64_t cache_size;         /* bytes of HBM for tags + rows + counters */
  int64_t row_size_in_bytes;
  void* uvm_table;             /* optional host-linear backing rows (hipHostMalloc'd), or NULL */
  int count_misses;            /* bool */
  int64_t max_modify_size;
  nve_data_type_t value_dtype;
  void* private_stream;        /* hipStream_t or NULL */
  int disable_uvm_update;      /* bool */
  int uvm_cpu_accumulate;      /* bool */
  int data_storage_on_host;    /* bool */
  int modify_on_gpu;           /* bool */
  uint64_t kernel_mode_type;
  uint64_t kernel_mode_value;
  int64_t invalid_key;         /* empty-way tag, cast to the key type; default -1 */
  int64_t uvm_num_rows;        /* rows in uvm_table; required with uvm_table */
} nve_gpu_table_config_t;

typedef struct {
  const char* layer_name;
  int32_t device_id;
  void* embedding_table;             /* linear table in device memory */
  int64_t num_embeddings;
  int64_t embedding_width_in_bytes;  /* stored bytes per row (even for quantized rows) */
  nve_data_type_t value_dtype;
  int64_t default_row_index;         /* row returned for out-of-range keys; < 0 disables */
} nve_gpu_embedding_layer_config_t;

typedef struct {
  const char* layer_name;
  nve_heuristic_t insert_heuristic;  /* NULL: default heuristic */
  int64_t min_insert_freq_gpu;
  int64_t min_insert_size_gpu;
  int64_t default_row_index;         /* UVM row returned for out-of-range keys; < 0 disables */
} nve_linear_uvm_layer_config_t;

typedef struct {
  const char* layer_name;
  nve_heuristic_t insert_heuristic;
  int64_t min_insert_freq_gpu;
  int64_t min_insert_freq_host;
  int64_t min_insert_size_gpu;
  int64_t min_insert_size_host;
  const void* default_embedding;
  int64_t default_embedding_size;
} nve_hierarchical_layer_config_t;

typedef struct {
  const char* layer_name;
  const void* default_embedding;
  int64_t default_embedding_size;
} nve_host_embedding_layer_config_t;

typedef struct {
  int64_t overflow_margin;
  nve_overflow_handler_t handler;
  double resolution_margin;
} nve_overflow_policy_config_t;

typedef struct {
  int64_t key_size;
  int64_t max_value_size;
  nve_data_type_t value_dtype;
  int64_t invalid_key;
} nve_host_table_config_t;

/* ---- config defaults (nve_c_api.h:240-279) ----------------------------- */
NVE_C_API nve_gpu_table_config_t nve_gpu_table_config_default(void);
NVE_C_API nve_gpu_embedding_layer_config_t nve_gpu_embedding_layer_config_default(void);
NVE_C_API nve_linear_uvm_layer_config_t nve_linear_uvm_layer_config_default(void);
NVE_C_API nve_hierarchical_layer_config_t nve_hierarchical_layer_config_default(void);
NVE_C_API nve_host_embedding_layer_config_t nve_host_embedding_layer_config_default(void);
NVE_C_API nve_overflow_policy_config_t nve_overflow_policy_config_default(void);
NVE_C_API nve_host_table_config_t nve_host_table_config_default(void);

/* ---- version (nve_c_api.h:285-300) ------------------------------------- */
NVE_C_API nve_status_t nve_version(int32_t* major, int32_t* minor, int32_t* patch);
NVE_C_API nve_status_t nve_abi_version(int32_t* major, int32_t* minor);

/* ---- thread pool (nve_c_api.h:306-333) --------------------------------- */
NVE_C_API nve_status_t nve_thread_pool_create(nve_thread_pool_t* out, const char* json_config);
NVE_C_API nve_status_t nve_thread_pool_destroy(nve_thread_pool_t pool);
NVE_C_API nve_status_t nve_thread_pool_num_workers(nve_thread_pool_t pool, int64_t* out);
NVE_C_API nve_status_t nve_configure_default_thread_pool(const char* json_config);

/* ---- insert heuristics (nve_c_api.h:339-366) --------------------------- */
NVE_C_API nve_status_t nve_heuristic_create_default(nve_heuristic_t* out, const float* thresholds,
                                                    int64_t num_thresholds);
NVE_C_API nve_status_t nve_heuristic_create_never(nve_heuristic_t* out);
NVE_C_API nve_status_t nve_heuristic_destroy(nve_heuristic_t heuristic);

/* ---- execution context (nve_c_api.h:372-400) --------------------------- */
NVE_C_API nve_status_t nve_context_destroy(nve_context_t ctx);
NVE_C_API nve_status_t nve_context_wait(nve_context_t ctx);
NVE_C_API nve_status_t nve_context_get_lookup_stream(nve_context_t ctx, void** out_stream);
NVE_C_API nve_status_t nve_context_get_modify_stream(nve_context_t ctx, void** out_stream);

/* ---- tables (nve_c_api.h:406-572) -------------------------------------- */
NVE_C_API nve_status_t nve_gpu_table_create(nve_table_t* out, nve_key_type_t key_type,
                                            const nve_gpu_table_config_t* config,
                                            nve_allocator_t allocator);
NVE_C_API nve_status_t nve_table_destroy(nve_table_t table);
/* hit_mask: ceil(n/64) words; bit i set on entry = already resolved (skipped);
 * on exit bit i set = resolved by this call.  values may be NULL (exists check). */
NVE_C_API nve_status_t nve_table_find(nve_table_t table, nve_context_t ctx, int64_t n,
                                      const void* keys, uint64_t* hit_mask, int64_t value_stride,
                                      void* values, int64_t* value_sizes);
NVE_C_API nve_status_t nve_table_insert(nve_table_t table, nve_context_t ctx, int64_t n,
                                        const void* keys, int64_t value_stride, int64_t value_size,
                                        const void* values);
NVE_C_API nve_status_t nve_table_update(nve_table_t table, nve_context_t ctx, int64_t n,
                                        const void* keys, int64_t value_stride, int64_t value_size,
                                        const void* values);
NVE_C_API nve_status_t nve_table_update_accumulate(nve_table_t table, nve_context_t ctx, int64_t n,
                                                   const void* keys, int64_t update_stride,
                                                   int64_t update_size, const void* updates,
                                                   nve_data_type_t update_dtype);
NVE_C_API nve_status_t nve_table_clear(nve_table_t table, nve_context_t ctx);
NVE_C_API nve_status_t nve_table_erase(nve_table_t table, nve_context_t ctx, int64_t n,
                                       const void* keys);
NVE_C_API nve_status_t nve_table_create_execution_context(nve_table_t table, nve_context_t* out,
                                                          void* lookup_stream, void* modify_stream,
                                                          nve_thread_pool_t thread_pool,
                                                          nve_allocator_t allocator);
NVE_C_API nve_status_t nve_table_get_device_id(const nve_table_t table, int32_t* out);
NVE_C_API nve_status_t nve_table_get_max_row_size(const nve_table_t table, int64_t* out);
NVE_C_API nve_status_t nve_table_get_key_size(const nve_table_t table, int64_t* out);
NVE_C_API nve_status_t nve_table_reset_lookup_counter(nve_table_t table, nve_context_t ctx);
/* GPU tables count the lookup misses of the context since the last reset
 * (nve_c_api.h:560-572, gpu_table.cu:1141-1175). */
NVE_C_API nve_status_t nve_table_get_lookup_counter(const nve_table_t table, nve_context_t ctx,
                                                    int64_t* counter);

/* ---- table factories (nve_c_api.h:578-610): plugins are not part of this
 * build; these return NVE_ERROR_NOT_IMPLEMENTED. ------------------------- */
NVE_C_API nve_status_t nve_create_table_factory(nve_table_factory_t* out, const char* plugin_path,
                                                const char* json_config);
NVE_C_API nve_status_t nve_table_factory_destroy(nve_table_factory_t factory);
NVE_C_API nve_status_t nve_table_factory_produce(nve_table_factory_t factory, int64_t table_id,
                                                 const char* json_config, nve_table_t* out);

/* ---- embedding layers (nve_c_api.h:616-835) ---------------------------- */
NVE_C_API nve_status_t nve_gpu_embedding_layer_create(nve_layer_t* out, nve_key_type_t key_type,
                                                      const nve_gpu_embedding_layer_config_t* config,
                                                      nve_allocator_t allocator);
NVE_C_API nve_status_t nve_linear_uvm_layer_create(nve_layer_t* out, nve_key_type_t key_type,
                                                   const nve_linear_uvm_layer_config_t* config,
                                                   nve_table_t gpu_table, nve_allocator_t allocator);
/* Remote / host tiers are not part of this build: NVE_ERROR_NOT_IMPLEMENTED. */
NVE_C_API nve_status_t nve_hierarchical_layer_create(nve_layer_t* out, nve_key_type_t key_type,
                                                     const nve_hierarchical_layer_config_t* config,
                                                     const nve_table_t* tables, int64_t num_tables,
                                                     nve_allocator_t allocator);
NVE_C_API nve_status_t nve_host_embedding_layer_create(nve_layer_t* out, nve_key_type_t key_type,
                                                       const nve_host_embedding_layer_config_t* config,
                                                       nve_table_t host_table,
                                                       nve_allocator_t allocator);
NVE_C_API nve_status_t nve_layer_destroy(nve_layer_t layer);
NVE_C_API nve_status_t nve_layer_lookup(nve_layer_t layer, nve_context_t ctx, int64_t num_keys,
                                        const void* keys, void* output, int64_t output_stride,
                                        uint64_t* hitmask, float* hitrates);
/* Fused find-and-pool (nve_c_api.h:697-732).  Concatenate emits one row per
 * key (raw rows when output_type is the stored type, dequantized otherwise);
 * other pooling types emit one row per bag, accumulated in fp32. */
NVE_C_API nve_status_t nve_layer_lookup_pooled(nve_layer_t layer, nve_context_t ctx,
                                               int64_t num_keys, const void* keys, void* output,
                                               int64_t output_stride, uint64_t* hitmask,
                                               nve_pooling_type_t pooling_type,
                                               nve_sparse_type_t sparse_type,
                                               const void* csr_offsets, int64_t num_csr_offsets,
                                               int64_t fixed_hotness, const void* weights,
                                               nve_data_type_t weight_type,
                                               nve_data_type_t output_type, float* hitrates);
NVE_C_API nve_status_t nve_layer_insert(nve_layer_t layer, nve_context_t ctx, int64_t num_keys,
                                        const void* keys, int64_t value_stride, int64_t value_size,
                                        const void* values, int64_t table_id);
NVE_C_API nve_status_t nve_layer_update(nve_layer_t layer, nve_context_t ctx, int64_t num_keys,
                                        const void* keys, int64_t value_stride, int64_t value_size,
                                        const void* values, int64_t table_id);
NVE_C_API nve_status_t nve_layer_accumulate(nve_layer_t layer, nve_context_t ctx, int64_t num_keys,
                                            const void* keys, int64_t value_stride,
                                            int64_t value_size, const void* values,
                                            nve_data_type_t value_type, int64_t table_id);
NVE_C_API nve_status_t nve_layer_clear(nve_layer_t layer, nve_context_t ctx);
NVE_C_API nve_status_t nve_layer_erase(nve_layer_t layer, nve_context_t ctx, int64_t num_keys,
                                       const void* keys, int64_t table_id);
NVE_C_API nve_status_t nve_layer_create_execution_context(nve_layer_t layer, nve_context_t* out,
                                                          void* lookup_stream, void* modify_stream,
                                                          nve_thread_pool_t thread_pool,
                                                          nve_allocator_t allocator);
NVE_C_API nve_status_t nve_layer_get_num_tables(nve_layer_t layer, int64_t* out);

#ifdef __cplusplus
}
#endif

#endif /* NVE_C_API_H */
