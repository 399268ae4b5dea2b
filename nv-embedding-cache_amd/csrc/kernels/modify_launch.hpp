// modify_launch.hpp -- host launchers of the cache insert kernels (modify.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nve_amd {

// Arguments of the per-set replacement kernel.
struct ReplaceLaunch {
  const uint32_t* rset;   // represented sets
  const uint32_t* roff;   // num_rsets + 1 offsets into order
  int64_t num_rsets;
  const uint32_t* order;  // histogram indices grouped by set (ascending within a set)
  const int64_t* hkeys;   // histogram keys
  const float* hprio;     // histogram priorities
  const uint64_t* hsrc;   // histogram source rows
  const void* tags;       // num_sets*8 tags of the key type
  float* counters;        // num_sets*8
  int64_t* set_ts;        // num_sets
  int64_t global_ts;
  float decay_rate;
  const float* decay_table;  // decay_table[d] = (float)pow(rate, d), d < decay_len
  int64_t decay_len;
  uint64_t num_sets;
  int64_t sentinel;
  // insert_from_uvm: rows of the backing table; a key outside [0, src_rows)
  // has no source row and is no candidate (a resident one still gains its
  // priority).  0: every key is a candidate (rows come with the keys).
  uint64_t src_rows;
  // Records, one per position of the candidate order: position roff[r] + x
  // holds set r's x-th replacement, and every position without one holds
  // kNoRecord as its slot (a set replaces at most min(its candidates, 8) ways,
  // so its records fit its own range of the order).
  uint32_t max_records;      // positions (the length of order)
  uint64_t* rec_slot;        // set*8 + way, or kNoRecord
  int64_t* rec_tag;          // new tag
  uint64_t* rec_src;         // source row address
};

// rec_slot of a record position that holds no record
constexpr uint64_t kNoRecord = ~0ull;

// Hashed histogram of an insert into a large cache (modify.hip): the batch's
// unique keys, counts and first positions from a hash table of 2^bits slots
// (+1 for the key word ~0), each unique key chained into its set through the
// table's per-set words, then the per-set replacement over the candidates
// sorted into histogram order.  A set with more than kHashSetMax candidates
// makes the call a no-op (counts[2] = 1) for the sorted histogram to redo.
constexpr int kHashSetMax = 32;
constexpr uint64_t kSetClean = 0x00000000ffffffffull;  // per-set word: no candidate, no chain
struct HashInsertLaunch {
  const void* keys;
  int key_bytes;
  int64_t n;
  int bits;            // 2^bits >= 2n slots
  uint64_t* tkey;      // 2^bits + 1 key words
  uint32_t* tcount;    // 2^bits + 1 counts
  uint32_t* tfirst;    // 2^bits + 1 first positions
  uint32_t* ulist;     // n: the unique keys' slots, [0, counts[0])
  uint32_t* unext;     // n: a unique key's successor in its set's chain
  uint32_t* rsets;     // n: the touched sets, [0, counts[1])
  uint32_t* counts;    // 4 words: unique keys, touched sets, overflow
  uint64_t* set_word;  // num_sets words (candidates << 32 | chain head), kSetClean between inserts
  uint64_t num_sets;
  float norm;          // priority = float(count) * norm, norm = 1 / float(n)
  const uint8_t* rows_base;
  int64_t row_stride;
  int by_key;          // source row: rows_base + key * stride (1) or + first position * stride (0)
};
// clear, count, chain, replace; the records (r.rec_*) are indexed by unique
// key, [0, counts[0]), for the record kernels with num = counts
hipError_t launch_hash_insert(const HashInsertLaunch& h, const ReplaceLaunch& r, hipStream_t stream);

hipError_t launch_hist_prep(const void* keys, int key_bytes, int64_t n, uint64_t* k64, uint32_t* v,
                            hipStream_t stream);
// heads[i] = 1 where a run of equal sorted keys starts; with span_part
// (nparts words, e.g. a raw sort pass's tile spans) also *span_out = their OR.
hipError_t launch_run_heads(const uint64_t* ks, int64_t n, uint32_t* heads, hipStream_t stream,
                            const uint64_t* span_part = nullptr, int64_t nparts = 0,
                            unsigned long long* span_out = nullptr);
hipError_t launch_run_gather(const uint64_t* ks, const uint32_t* vs, const uint32_t* scan, int64_t n,
                             uint32_t* start, uint64_t* ukey, uint32_t* first, hipStream_t stream);
hipError_t launch_count_key(const uint32_t* start, uint32_t u_n, uint64_t* k2, uint32_t* v2,
                            hipStream_t stream);
hipError_t launch_hist_gather(const uint32_t* order, const uint32_t* start, const uint64_t* ukey,
                              const uint32_t* first, uint32_t m, int key_bytes, float norm,
                              const uint8_t* rows_base, int64_t row_stride, int by_key,
                              uint64_t num_sets, int64_t* hkeys, float* hprio, uint64_t* hsrc,
                              uint64_t* k3, uint32_t* v3, hipStream_t stream);
hipError_t launch_set_gather(const uint64_t* ks, const uint32_t* scan, int64_t m, uint32_t* rset,
                             uint32_t* roff, hipStream_t stream);
hipError_t launch_set_replace(const ReplaceLaunch& a, int key_bytes, hipStream_t stream);
// The record kernels take records [0, min(*num, max_records)), or with num
// null [0, max_records); records whose slot is kNoRecord are skipped.
hipError_t launch_invalidate(const uint32_t* num, uint32_t max_records, const uint64_t* slot,
                             void* tags, int key_bytes, int64_t sentinel, hipStream_t stream);
hipError_t launch_commit(const uint32_t* num, uint32_t max_records, const uint64_t* slot,
                         const int64_t* tag, void* tags, int key_bytes, hipStream_t stream);
hipError_t launch_copy_rows(const uint32_t* num, uint32_t max_records, const uint64_t* slot,
                            const uint64_t* src, int src_align, uint8_t* data, uint64_t row_bytes,
                            hipStream_t stream);

}  // namespace nve_amd
