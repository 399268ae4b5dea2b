/*
 * nve_oracle.h -- CPU restatement of the NV Embedding Cache lookup path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the
 * MI355X build: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it, and only to check or to time the CPU
 * baseline.  Nothing in the product library links or calls it.
 *
 * Every function names the reference file:line whose behaviour it restates.
 * Where the reference's arithmetic is not fixed by its source (compiler FMA
 * contraction, CUDA __powf, cuEmbed's absent source) the choice made here is
 * stated next to the function.
 *
 * Pinning (what checks each function against something other than itself):
 *   orc_f16_to_f32 / orc_f32_to_f16      numpy float16 casts over all 65536
 *                                        codes and 10^6 random floats
 *   orc_e4m3_to_f32                      torch.float8_e4m3fn over all 256 codes
 *   orc_sanitize_keys                    closed form + reference test cases
 *   orc_gather                           brute force memcmp (row i == table[key i])
 *   orc_dequant_row                      closed form float(q)*s(+o), numpy
 *   orc_pool (GPU order)                 dyadic-fraction table => exact Sum;
 *                                        torch.nn.EmbeddingBag in float64
 *   orc_pool_host (CPU HostLayer order)  torch.nn.EmbeddingBag, 1e-6; dyadic
 *                                        tables exact; the element values of
 *                                        every format by numpy closed forms
 *   orc_convert_host                     numpy casts (f32 <-> f16) and the
 *                                        float64 closed form of q*s+o, exact
 *                                        in float64, rounded once
 *   orc_cache_*                          closed-form set/tag math, brute force
 *                                        residency invariants, hand-built cases
 *   orc_histogram                        brute force (collections.Counter)
 *   orc_cache_insert                     hand-derived cases of the 8-lane
 *                                        bitonic networks, invariants
 *   orc_histogram_host                   brute force (stable sort of
 *                                        collections.Counter by count)
 *   orc_cache_insert_host                hand-derived cases (fill order,
 *                                        >= replacement, one record per way,
 *                                        decay closed form, stale counters
 *                                        after erase, truncation)
 *   orc_dedup                            sorted/unique/inverse round trip
 *   orc_pooling_backprop                 torch autograd of embedding_bag /
 *                                        embedding in float64; dyadic Sum exact;
 *                                        run-length invariance
 * Parity unpinned: orc_cache_insert's decay factor is defined here as
 * (float)pow((double)rate, (double)delta); the reference uses CUDA __powf,
 * whose bits are not published.
 */
#ifndef NVE_ORACLE_H
#define NVE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype ids follow nve_c_api.h (values 1..10) plus the two extension row
 * formats of the MI355X build (see include/nve_amd_ext.h). */
enum {
  ORC_F32 = 1,
  ORC_F16 = 3,
  ORC_QI8_F32 = 7,   /* int8 + f32 scale           */
  ORC_QI8_F16 = 8,   /* int8 + f16 scale           */
  ORC_QU8_F32 = 9,   /* uint8 + f32 scale + offset */
  ORC_QU8_F16 = 10,  /* uint8 + f16 scale + offset */
  ORC_XI8A_F32 = 32, /* int8 + f32 scale + offset (extension)   */
  ORC_XE4M3_F32 = 33 /* fp8 e4m3 + f32 scale (extension)        */
};

enum { ORC_CONCAT = 0, ORC_SUM = 1, ORC_MEAN = 2, ORC_WSUM = 3, ORC_WMEAN = 4 };
enum { ORC_FIXED = 0, ORC_CSR = 1 };

/* ---- scalar conversions ---- */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);
float orc_e4m3_to_f32(uint8_t v);
void orc_f16_to_f32_n(const uint16_t* in, float* out, int64_t n);
void orc_f32_to_f16_n(const float* in, uint16_t* out, int64_t n);

/* ---- row layout ---- */
int64_t orc_meta_bytes(int dtype);
int64_t orc_value_bytes(int dtype); /* bytes per stored value element */
int orc_out_dtype_native(int dtype);  /* float precision of the metadata */

/* ---- keys ---- */
int orc_key_in_range(int64_t key, uint64_t num_rows);
void orc_sanitize_keys(const void* keys, void* out, int64_t n, int key_bytes, uint64_t num_rows,
                       int64_t default_row);

/* ---- linear-table gather (cpu_gather.hpp:28-80) ----
 * Returns the number of keys resolved; keys already marked in hit_mask or out of
 * range are skipped (their output rows are left untouched). */
int64_t orc_gather(const void* keys, int key_bytes, int64_t n, uint64_t* hit_mask,
                   const uint8_t* table, uint64_t num_rows, int64_t row_bytes, uint8_t* out,
                   int64_t out_stride);

/* ---- dequant: one stored row -> `count` output elements ---- */
void orc_dequant_row(const uint8_t* row, int dtype, int64_t count, int out_dtype, void* out);

/* ---- pooling over already-resolved rows ----
 * rows[k] points at the stored row of key k (k in [0, num_keys)).
 * offsets: CSR (num_bags+1 entries, int32 or int64 per key_bytes) or NULL for Fixed.
 * GPU order: find_and_combine_kernel.cuh:40-154 (FMA weighted accumulate,
 * Mean = acc / denom).  */
void orc_pool(const uint8_t* const* rows, int dtype, int64_t count, int sparse, int pooling,
              int64_t num_keys, const void* offsets, int key_bytes, int64_t num_bags,
              int64_t hotness, const void* weights, int weight_dtype, int out_dtype, void* out,
              int64_t out_stride);

/* CPU HostLayer order: cpu_pooling.hpp:68-150 (v *= w; acc += v; Mean = acc * (1/denom)). */
void orc_pool_host(const uint8_t* const* rows, int dtype, int64_t count, int sparse, int pooling,
                   int64_t num_keys, const void* offsets, int key_bytes, int64_t num_bags,
                   int64_t hotness, const void* weights, int weight_dtype, int out_dtype,
                   void* out, int64_t out_stride);

/* CPU HostLayer Concatenate to another type: cpu_pooling.hpp:272-341, one row
 * (count values of dtype) converted / dequantized to out_dtype. */
void orc_convert_host(const uint8_t* row, int dtype, int64_t count, int out_dtype, void* out);

/* Resolve linear-table row pointers (table + key*row_bytes). */
void orc_linear_rows(const void* keys, int key_bytes, int64_t n, const uint8_t* table,
                     int64_t row_bytes, const uint8_t** rows);

/* ---- threaded HostLayer lookup (host_embedding_layer.cpp:55-247) ----
 * CPU baseline: gather then pool, `threads` workers.  pooling == ORC_CONCAT
 * means plain gather into out.  gather_buf must hold n*row_bytes. */
void orc_host_layer_lookup(const void* keys, int key_bytes, int64_t n, const uint8_t* table,
                           uint64_t num_rows, int64_t row_bytes, int dtype, int pooling,
                           int sparse, const void* offsets, int64_t num_bags, int64_t hotness,
                           const void* weights, int weight_dtype, int out_dtype, uint8_t* gather_buf,
                           void* out, int64_t out_stride, int threads);

/* ---- set-associative cache model (ecache) ---- */
typedef struct orc_cache {
  uint64_t num_sets;
  int64_t row_bytes;
  int key_bytes;     /* 4 or 8; tag type == key type */
  int64_t sentinel;  /* invalid key / empty-way tag */
  float decay_rate;
  int64_t global_ts;
  uint8_t* data;     /* num_sets*8 rows */
  int64_t* tags;     /* num_sets*8, value of the TagT (sign-extended for int32) */
  float* counters;   /* num_sets*8 */
  int64_t* set_ts;   /* num_sets */
  int host_modify;   /* 1: CacheSAHostModify (modify_on_gpu = false), 0: device modify */
} orc_cache;

uint64_t orc_cache_num_sets(uint64_t cache_bytes, int64_t row_bytes, int key_bytes);
/* host-metadata variant: the way counters live in host memory, so a set costs
 * only its tags and rows (ec_set_associative.h:677-683, no counter term) */
uint64_t orc_cache_num_sets_host(uint64_t cache_bytes, int64_t row_bytes, int key_bytes);
int orc_cache_init(orc_cache* c, uint64_t cache_bytes, int64_t row_bytes, int key_bytes,
                   int64_t sentinel);
int orc_cache_init_ex(orc_cache* c, uint64_t cache_bytes, int64_t row_bytes, int key_bytes,
                      int64_t sentinel, int host_modify);
void orc_cache_free(orc_cache* c);
uint32_t orc_cache_set(const orc_cache* c, int64_t key);
int64_t orc_cache_tag(const orc_cache* c, int64_t key);
int64_t orc_cache_key_of(const orc_cache* c, int64_t tag, uint32_t set);
/* returns way (0..7) or -1 on miss */
int orc_cache_find_way(const orc_cache* c, int64_t key);
/* Resolve rows: hit -> cache row, miss -> uvm + key*row (or NULL when uvm==NULL).
 * Returns the number of misses. hit_bits (optional) gets bit i set for hits. */
int64_t orc_cache_resolve(const orc_cache* c, const void* keys, int64_t n, const uint8_t* uvm,
                          const uint8_t** rows, uint64_t* hit_bits);

/* histogram (gather_keys_data_ptrs.cuh:121-191): unique keys ordered by count
 * descending, ties by ascending (signed) key; priority = float(count)*(1/float(n));
 * first_idx = first position of the key in the input.  Returns #unique. */
int64_t orc_histogram(const void* keys, int key_bytes, int64_t n, int64_t* ukeys,
                      float* priority, int64_t* first_idx);

/* Insert (ec_set_associative_device_modify.cuh:225-288 + ec_set_associative_modify.cuh:139-513).
 * src_rows[i] is the row to copy for histogram entry i (already ordered).  Writes the
 * replace records (set, way) to out_set/out_way if non-NULL and returns their count. */
int64_t orc_cache_insert_hist(orc_cache* c, const int64_t* ukeys, const float* priority,
                              const uint8_t* const* src_rows, int64_t m, int64_t* out_set,
                              int64_t* out_way);

/* Convenience: histogram + insert, rows from a dense table of uvm_rows rows
 * (insert_from_uvm) when uvm != NULL, else from values + first_idx*stride
 * (GpuTable::insert).  A key outside [0, uvm_rows) has no source row and is not
 * a candidate (resident, it still gains its priority); the reference would
 * read past the table.  In orc_cache_insert_hist and orc_cache_insert_host,
 * likewise, a NULL entry of a non-NULL src_rows is no candidate. */
int64_t orc_cache_insert_keys(orc_cache* c, const void* keys, int64_t n, const uint8_t* uvm,
                              uint64_t uvm_rows, const uint8_t* values, int64_t value_stride,
                              int64_t max_modify_size);

/* Invalidate (erase) keys: every way whose key matches gets the sentinel tag. */
int64_t orc_cache_erase(orc_cache* c, const void* keys, int64_t n);

/* clear_cache: every tag empty, set timestamps and the insert clock back to 0
 * (ec_set_associative_device_modify.cuh:205-222); the host-metadata cache also
 * zeroes its counters (ec_set_associative_host_modify.h:192-211). */
void orc_cache_clear(orc_cache* c);

/* CPU DefaultHistogram (embed_cache.h:188-229): unique keys in order of first
 * occurrence, then sorted by count descending; priority = float(count) /
 * float(n) (a division); first_idx = first position of the key.  The reference
 * sorts with std::sort, which leaves the order of equal counts unspecified;
 * here equal counts keep first-occurrence order (a stable sort).  Returns
 * #unique. */
int64_t orc_histogram_host(const void* keys, int key_bytes, int64_t n, int64_t* ukeys,
                           float* priority, int64_t* first_idx);

/* CacheSAHostModify::insert (ec_set_associative_host_modify.h:218-296): the
 * sequential policy of modify_on_gpu = false.  Candidates in histogram order;
 * a set is decayed by (float)pow((double)rate, (double)delta) on its first
 * touch of the call; a resident key adds its priority to its way; otherwise the
 * first way with the smallest counter is replaced when priority >= that
 * counter and that way was not already replaced in this call.  Stops once
 * max_update records exist.  Writes (set, way) records if out_set/out_way are
 * non-NULL; returns their count. */
int64_t orc_cache_insert_host(orc_cache* c, const int64_t* ukeys, const float* priority,
                              const uint8_t* const* src_rows, int64_t m, int64_t max_update,
                              int64_t* out_set, int64_t* out_way);

/* Convenience for the host-metadata cache: orc_histogram_host + insert, rows
 * from a dense table of uvm_rows rows when uvm != NULL (keys outside it are no
 * candidates), else values + first_idx*stride. */
int64_t orc_cache_insert_keys_host(orc_cache* c, const void* keys, int64_t n, const uint8_t* uvm,
                                   uint64_t uvm_rows, const uint8_t* values, int64_t value_stride,
                                   int64_t max_modify_size);

/* ---- training backprop (GradientCalculator::compute_gradients,
 * gradient_calculator.cuh:238-301; GradientDedup, dedup_grads_kernel.cuh:57-107) ----
 * Sparse gradient of a lookup: unique keys ascending (unique_out, key type) and
 * one gradient row per unique key (grads_out, dim values of grad_dtype F32/F16).
 *   pooled (pooling Sum/Mean/WSum/WMean): grads_in has one row per bag;
 *     grad(u) = sum over the positions p of key u of nw(p) * grads_in[bag(p)],
 *     nw = 1 (Sum), w[p] (WSum), 1/count(bag) (Mean), w[p] / (the bag's weights
 *     added in position order) (WMean); bag(p) = p / hotness (Fixed) or the bag
 *     whose [offsets[b], offsets[b+1]) holds p (CSR); a position in no bag adds
 *     nothing;
 *   Concatenate: grads_in has one row per key position; grad(u) = sum of the
 *     rows of u's positions.
 * Order (defined here; the reference cuts runs at 1024 positions and adds the
 * pieces with atomics, so its order is not fixed): the positions of all keys,
 * stably sorted by key (the dedup order), are cut at every multiple of `block`;
 * a piece is one key's positions inside one block.  A piece is accumulated in
 * fp32 in position order from 0 (fmaf(g, nw, acc), or acc + g when unweighted:
 * Sum, Concatenate).  A key's J pieces are split into 8 consecutive
 * sub-sequences of ceil(J / 8) pieces (the last ones may be short or empty);
 * each adds its pieces' rows in order from 0, the key's row adds the 8 sums in
 * order from 0, and the sum is rounded once to grad_dtype.  Returns the number
 * of unique keys. */
int64_t orc_pooling_backprop(const void* keys, int key_bytes, int64_t n, int pooling, int sparse,
                             const void* offsets, int64_t num_bags, int64_t hotness,
                             const void* weights, int weight_dtype, const void* grads_in,
                             int grad_dtype, int64_t dim, int64_t block, void* unique_out,
                             void* grads_out);

/* ---- dedup (deduper.cuh:136-221) ----
 * unique: ascending unique keys; counts; inverse: positions sorted stably by key
 * (inverse[offsets[u] + j] = j-th position of unique key u); offsets: exclusive
 * scan of counts.  Returns #unique. */
int64_t orc_dedup(const void* keys, int key_bytes, int64_t n, int64_t* unique, int64_t* counts,
                  int64_t* inverse, int64_t* offsets);

/* ---- key generator (pytorch_samples_common.py:21-47 restated) ----
 * x[i] uniform doubles in [0,1); writes y = trunc((x*(max^g - min^g) + min^g)^(1/g)),
 * g = 1 - alpha, clamped to max-1. */
void orc_power_law(const double* x, int64_t n, double min_v, double max_v, double alpha,
                   int64_t* out);

#ifdef __cplusplus
}
#endif
#endif
