/*
 * nve_amd_ext.h -- extensions of the MI355X lookup library beyond the
 * reference's C ABI (include/nve_c_api.h).  Same conventions: every call
 * returns nve_status_t, messages go to nve_get_last_error, streams are
 * hipStream_t passed as void*.  Pointers documented as "device" must be
 * GPU-readable (device memory, or pinned host memory for a table).
 */
#ifndef NVE_AMD_EXT_H
#define NVE_AMD_EXT_H

#include "nve_c_api.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Row formats without a reference counterpart (the reference has no int8
 * affine row with fp32 offset and no fp8 row; nve_types.hpp:59-73).  Both
 * dequantize in fp32 and may be emitted as fp16 or fp32:
 *   NVE_DTYPE_X_INT8_AFFINE_F32: int8 q[count], f32 scale, f32 offset;
 *                                value = fma(q, scale, offset)
 *   NVE_DTYPE_X_E4M3_ROWWISE_F32: OCP fp8 e4m3 q[count], f32 scale;
 *                                value = e4m3(q) * scale */
enum {
  NVE_DTYPE_X_INT8_AFFINE_F32 = 32,
  NVE_DTYPE_X_E4M3_ROWWISE_F32 = 33,
};

/* Fused find-and-pool over a linear table, keys and outputs in device memory.
 * Restates the reference's kernel-level router find_and_pool
 * (cuda_ops/find_and_pool.cuh:103-132) with a linear table
 * (ECNoCache, load_indices = true): Concatenate emits one dequantized row per
 * key, every other pooling type one fp32-accumulated row per bag.  Keys
 * outside [0, num_rows) read nothing: their Concatenate output rows are left
 * as they are, and a bag counts them as zero rows.
 * output_type: the value type's float precision (either precision for the
 * extension types).  split_hint: 0 lets the library choose how many lane
 * groups share a bag; > 0 forces that many (a power of two); < 0 forces one
 * group per bag (strict key order).  unroll_hint: 0 lets the library choose how
 * many row loads each lane group keeps in flight; 8 or 16 forces it. */
NVE_C_API nve_status_t nve_amd_find_and_pool(
    nve_key_type_t key_type, int64_t num_keys, const void* keys, const void* table,
    int64_t num_rows, int64_t row_size_in_bytes, nve_data_type_t value_dtype,
    nve_pooling_type_t pooling_type, nve_sparse_type_t sparse_type, const void* csr_offsets,
    int64_t num_csr_offsets, int64_t fixed_hotness, const void* weights,
    nve_data_type_t weight_type, nve_data_type_t output_type, void* output,
    int64_t output_stride, int32_t split_hint, int32_t unroll_hint, void* stream);

/* Multi-table jagged pooling in one launch (the reference pools one table per
 * call; this fuses a batch of num_tables tables of equal row format, as a
 * TorchRec KeyedJaggedTensor lays them out).  tables: host array of
 * num_tables device table pointers; table_rows: host array of their row
 * counts (keys outside [0, table_rows[t]) read nothing), or NULL for no bound
 * check.  keys: num_keys keys of the key type,
 * table-major.  offsets: num_tables*batch_size + 1 entries of the key type;
 * bag (t, b) holds keys [offsets[t*batch_size + b], offsets[t*batch_size+b+1]).
 * weights: per key (weighted pooling), f32 or f16.  output: batch_size rows of
 * num_tables*count values of output_type, table t of sample b at
 * output[b][t][:], count = stored values per row.  Sum / Mean / WeightedSum /
 * WeightedMean, fp32 accumulation; an fp16 or fp32 output from any row format. */
NVE_C_API nve_status_t nve_amd_find_and_pool_multi(
    nve_key_type_t key_type, int64_t num_tables, const void* const* tables,
    const int64_t* table_rows, int64_t row_size_in_bytes, nve_data_type_t value_dtype,
    int64_t batch_size, int64_t num_keys,
    const void* keys, const void* offsets, const void* weights, nve_data_type_t weight_type,
    nve_pooling_type_t pooling_type, nve_data_type_t output_type, void* output, void* stream);

/* Key dedup (the reference's Deduper::dedup, cuda_ops/deduper.cuh:136-221),
 * device buffers of the key type, each sized num_keys: unique_out (ascending,
 * signed order), counts_out, inverse_out (original positions ordered by key,
 * stable: inverse_out[offsets_out[u] + j] is the j-th position of unique key
 * u) and offsets_out (exclusive scan of the counts).  *num_unique receives the
 * number of unique keys (the call synchronizes the stream).  workspace: device
 * memory of nve_amd_dedup_workspace_size(num_keys) bytes. */
NVE_C_API nve_status_t nve_amd_dedup_workspace_size(int64_t num_keys, uint64_t* bytes);
NVE_C_API nve_status_t nve_amd_dedup(nve_key_type_t key_type, int64_t num_keys, const void* keys,
                                     void* unique_out, void* counts_out, void* inverse_out,
                                     void* offsets_out, int64_t* num_unique, void* workspace,
                                     uint64_t workspace_bytes, void* stream);

/* Dedup-then-gather over a linear table in device memory: output row i =
 * table row keys[i].  The keys are deduplicated by hashing, each distinct row
 * is read from the table once into the output row of one of its positions,
 * and the other positions copy that row (UnpackDedup).  Keys outside
 * [0, num_rows) leave their output row unchanged.  Asynchronous; workspace as
 * for nve_amd_dedup. */
NVE_C_API nve_status_t nve_amd_dedup_gather(nve_key_type_t key_type, int64_t num_keys,
                                            const void* keys, const void* table, int64_t num_rows,
                                            int64_t row_size_in_bytes, void* output,
                                            int64_t output_stride, void* workspace,
                                            uint64_t workspace_bytes, void* stream);

/* nve_amd_dedup_gather without the workspace argument, for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc); it has no counterpart in the reference.  It allocates
 * nothing: its scratch is a fixed 16 MiB device array, one per GPU, held
 * until the process ends.  num_keys must not exceed 262,144 (larger batches
 * fail with NVE_ERROR_INVALID_ARGUMENT).  Every call on one GPU uses that
 * GPU's array, so the library runs the calls on one GPU one after another, in
 * the order they are issued from any thread or stream: each call's stream
 * waits for the previous call's completion event (one event per GPU, made
 * with the array's address on the GPU's first call).  Under HIP graph capture
 * that ordering is not recorded: a replayed graph must not overlap other
 * calls on its GPU.  Same results as nve_amd_dedup_gather; asynchronous on
 * `stream`. */
NVE_C_API nve_status_t nve_amd_dedup_gather_noalloc(nve_key_type_t key_type, int64_t num_keys,
                                                    const void* keys, const void* table,
                                                    int64_t num_rows, int64_t row_size_in_bytes,
                                                    void* output, int64_t output_stride, void* stream);

/* Random-row read microbenchmark: reads row idx[i] (row_size_in_bytes each, a
 * multiple of 16) of a table for i < n and folds the bytes into sink (one
 * uint32 per 256-thread workgroup, ceil(n/128) words).  The table may be
 * device memory (the HBM random-row ceiling) or pinned host memory from
 * hipHostMalloc (the host link's random-row ceiling, which bounds the reads
 * of missed rows from a LinearUVM backing table). */
NVE_C_API nve_status_t nve_amd_read_ceiling(const void* table, int64_t row_size_in_bytes,
                                            const int64_t* idx, int64_t n, uint32_t* sink,
                                            void* stream);

/* Cache state transfer of a GPU table (checkpoint-style restore, tests):
 * tags = num_sets*8 keys of the table's key type, counters = num_sets*8
 * float, set_ts = num_sets int64; host or device pointers; any may be NULL. */
NVE_C_API nve_status_t nve_amd_gpu_table_num_sets(const nve_table_t table, int64_t* out);
NVE_C_API nve_status_t nve_amd_gpu_table_export_state(nve_table_t table, void* tags,
                                                      float* counters, int64_t* set_ts,
                                                      int64_t* global_ts);
NVE_C_API nve_status_t nve_amd_gpu_table_import_state(nve_table_t table, const void* tags,
                                                      const float* counters,
                                                      const int64_t* set_ts, int64_t global_ts);
/* Device address of the cache rows ((set*8 + way) * row_size_in_bytes). */
NVE_C_API nve_status_t nve_amd_gpu_table_data(nve_table_t table, void** out);

/* GpuTable::insert_from_uvm (include/gpu_table.hpp:160-167, gpu_table.cu:494-576):
 * insert keys whose rows are read from the table's backing (UVM) table at
 * uvm_table + key * row_size_in_bytes.  The reference's C ABI reaches it only
 * through a LinearUVM layer's auto-insert; this entry exposes it directly.
 * Keys may live in host or device memory; keys outside [0, uvm_num_rows) are
 * not inserted. */
NVE_C_API nve_status_t nve_amd_table_insert_from_uvm(nve_table_t table, nve_context_t ctx,
                                                     int64_t n, const void* keys);

/* LinearHostTable (include/linear_host_table.hpp:36-183): a dense table of
 * num_rows rows of config->max_value_size bytes at emb_table (host memory the
 * caller owns and keeps alive), row k at emb_table + k * max_value_size,
 * values of config->value_dtype (FLOAT32, FLOAT16 or a rowwise-quantized
 * type); config->key_size must match key_type.  At most max_threads tasks run
 * per operation (<= 0: no limit beyond the context's thread pool).  The
 * reference builds this table inside its pynve HostEmbedding binding
 * (python/pynve/bindings/binding_layers.hpp:742-756); its C ABI has no
 * constructor for it.  The handle works with nve_table_find / update /
 * update_accumulate (FLOAT32 rows) / insert / erase / clear (the last three
 * have no effect), the getters (device id -1), the lookup counter (keys
 * found) and nve_host_embedding_layer_create.  Nothing it does enters the HIP
 * runtime while its buffers are host memory. */
NVE_C_API nve_status_t nve_amd_linear_host_table_create(nve_table_t* out, nve_key_type_t key_type,
                                                        const nve_host_table_config_t* config,
                                                        void* emb_table, int64_t num_rows,
                                                        int64_t max_threads);

/* Training backprop: the sparse gradient of a lookup with respect to the table
 * (GradientCalculator::compute_gradients, cuda_ops/gradient_calculator.cuh:238-301,
 * which the reference's pynve GPU bindings call as concat_backprop /
 * pooling_backprop, python/pynve/bindings/binding_layers.hpp:131-250).
 * pooling_type NVE_POOL_CONCATENATE: grads_in holds one row per key
 * (num_keys rows); otherwise one row per bag (fixed_hotness, or
 * num_csr_offsets - 1 bags of non-decreasing csr_offsets of the key type).
 * grads_in / grads_out rows: embedding_width values of grad_type (FLOAT32 or
 * FLOAT16); weights (WEIGHTED_*): one per key of weight_type FLOAT32 / FLOAT16.
 * Sum weighs 1, WeightedSum w, Mean 1 / (keys in the bag), WeightedMean
 * w / (the bag's weights added in order).  Outputs: the unique keys ascending
 * (reserve num_keys entries of the key type), one gradient row per unique key
 * (reserve num_keys rows) and *num_unique_out.  Sums are fp32 in a fixed order
 * and rounded once, so the result is deterministic: the positions in dedup
 * order are cut into blocks of 32, each key's positions inside one block are
 * added in position order, and a key's J block sums are added in 8
 * consecutive sub-sequences of ceil(J / 8), then the 8 sub-sums in order.
 * Device buffers and workspace; synchronizes the stream. */
NVE_C_API nve_status_t nve_amd_backprop_workspace_size(int64_t num_keys, int64_t num_bags,
                                                       int64_t embedding_width, uint64_t* bytes);
NVE_C_API nve_status_t nve_amd_pooling_backprop(
    nve_key_type_t key_type, int64_t num_keys, const void* keys, nve_pooling_type_t pooling_type,
    nve_sparse_type_t sparse_type, const void* csr_offsets, int64_t num_csr_offsets,
    int64_t fixed_hotness, const void* weights, nve_data_type_t weight_type, const void* grads_in,
    nve_data_type_t grad_type, int64_t embedding_width, void* unique_keys_out, void* grads_out,
    int64_t* num_unique_out, void* workspace, uint64_t workspace_bytes, void* stream);

/* Log level (include/logging.hpp:34-203): messages at or below the level are
 * written, errors to stderr and the rest to stdout.  Levels: 0 critical,
 * 10 error, 20 warning, 30 perf, 40 info, 100 verbose.  The initial level is
 * NVE_LOG_LEVEL's (CRITICAL, ERROR, WARNING, PERF, INFO or VERBOSE), else
 * warning.  Library calls are also marked as roctx ranges (rocprofv3
 * --marker-trace) unless NVE_ROCTX=0; the reference marks them with NVTX
 * (include/cuda_support.hpp:26-55). */
NVE_C_API nve_status_t nve_amd_set_log_level(int32_t level);
NVE_C_API nve_status_t nve_amd_get_log_level(int32_t* level);
/* Writes one message through the library's logger if `level` is enabled
 * (the bindings log hit rates at the perf level this way, as the reference's
 * binding does with NVE_LOG_PERF_, binding_layers.hpp:370-387). */
NVE_C_API nve_status_t nve_amd_log_message(int32_t level, const char* message);

#ifdef __cplusplus
}
#endif

#endif /* NVE_AMD_EXT_H */
