// launch.hpp -- host-side launchers of the lookup kernels.
//
// Plain pointers and sizes only; every pointer handed to a launcher must be
// readable (or writable) by the GPU: device memory, or pinned host memory for
// a backing table.  Shapes are validated by the caller (the layers) before a
// launch; the launchers check the launch geometry they derive.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nve_amd {

constexpr int kMaxPoolTables = 64;  // tables one multi-table pooling launch can address

// Where rows come from (see resolve_row in device_common.cuh).
struct RowSource {
  const uint8_t* table;      // linear table / backing table (may be null with a cache)
  uint64_t row_bytes;        // stored bytes per row (also the cache slot size)
  int load_indices;          // 1: index = key; 0: index = key position (pre-gathered buffer)
  const uint8_t* cache_data; // null: no cache
  const void* cache_tags;    // num_sets*8 tags of the key type
  uint64_t num_sets;
  uint64_t num_rows;         // rows of `table`: keys >= num_rows read nothing (0 = no bound)
};

// One output row per key: the raw stored row (raw != 0) or its dequantized
// values (count elements of out_dtype).  hitmask (optional, ceil(n/64) words):
// bit set on entry = skip the key; on exit bit set = resolved.
struct GatherLaunch {
  const void* keys;
  int key_bytes;
  int64_t n;
  RowSource src;
  int stored_dtype;
  int64_t count;
  int raw;
  void* out;
  int64_t out_stride;
  int out_dtype;
  uint64_t* hitmask;
  unsigned long long* miss_counter;  // optional: += number of cache misses
  const uint32_t* out_index;         // optional: key i is written to output row out_index[i]
};

// One output row per bag (Fixed hotness or CSR offsets of the key type),
// accumulated in fp32; Mean / WeightedMean divide by the key count / weight
// sum, a zero denominator giving a zero row.
struct PoolLaunch {
  const void* keys;
  int key_bytes;
  int64_t num_keys;
  const void* offsets;  // null: fixed hotness
  int64_t num_bags;
  int64_t hotness;
  const void* weights;  // per key (global position), f32 or f16
  int weight_dtype;
  int weighted;
  int mean;
  RowSource src;
  int stored_dtype;
  int64_t count;
  void* out;
  int64_t out_stride;
  int out_dtype;
  unsigned long long* miss_counter;
  int force_split;   // 0: heuristic; > 0: groups per bag (power of two); < 0: one group per bag
  int force_unroll;  // 0: heuristic; 8 or 16: row loads in flight per lane group
  // Several tables in one launch (num_tables > 0): bag g belongs to table
  // g / bags_per_table, reads rows of tables[table] (linear, no cache) and writes
  // output row (g % bags_per_table) * out_stride + table * out_table_stride.
  int num_tables;
  int64_t keys_per_bag;  // mean bag length for the geometry choice (0: num_keys / num_bags)
  int64_t bags_per_table;
  int64_t out_table_stride;
  const uint8_t* tables[kMaxPoolTables];
  uint64_t table_rows[kMaxPoolTables];  // rows of each table (0: no bound check)
};

hipError_t launch_gather(const GatherLaunch& a, hipStream_t stream);
hipError_t launch_pool(const PoolLaunch& a, hipStream_t stream);
// keys outside [0, num_rows) -> default_row (in place allowed)
hipError_t launch_sanitize(const void* keys, void* out, int64_t n, int key_bytes,
                           uint64_t num_rows, int64_t default_row, hipStream_t stream);
// Random-row read ceiling: reads rows idx[i] (row_bytes each, a multiple of 16)
// of `table`, folding them into `sink` (one word per workgroup).
hipError_t launch_read_ceiling(const uint8_t* table, uint64_t row_bytes, const int64_t* idx,
                               int64_t n, uint32_t* sink, hipStream_t stream);

// Geometry the pool launcher picks (exposed for tests and the bench).
struct PoolGeometry {
  int vb, g, passes, gpb, threads, bags_per_wg, unroll;
  int64_t grid;
  int lds_bytes;
};
bool pool_geometry(const PoolLaunch& a, PoolGeometry* g);

}  // namespace nve_amd
