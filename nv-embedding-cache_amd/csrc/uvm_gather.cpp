// uvm_gather.cpp -- the SortGather and PipelineGather modes of
// GpuTable::find over a host-resident backing table.
//
// Reference behaviour restated:
//   mode choice      get_kernel_mode (gpu_table.cu:271-287): type 0 picks the
//                    direct lookup below kernel_mode_value keys (default 2^20)
//                    and SortGather from there on; 1, 2, 3 force LookupUVM,
//                    SortGather, PipelineGather
//   SortGather       call_sort_gather (ec_set_associative.cuh:966-1057)
//   PipelineGather   gather_flow_pipeline / executeCpuGatherPhase
//                    (pipeline_gather.cuh:203-412)
//
// Both write exactly what the direct lookup writes.  SortGather keeps every
// wave's loads on one side of the host link: lookups are sorted (misses
// first, hits after, each by key) and gathered in that order with the output
// permutation.  PipelineGather copies the hits on the GPU while host threads
// copy the missed rows from the backing table into a pinned staging buffer in
// tasks of task_size rows; each finished task's rows are scattered to the
// output by a kernel that reads the staging buffer over the host link in
// order (sequential transfers instead of random 256-byte reads).
#include <algorithm>
#include <cstring>
#include <future>
#include <vector>

#include "kernels/cache_launch.hpp"
#include "kernels/sort_launch.hpp"
#include "kernels/uvm_gather_launch.hpp"
#include "layers.hpp"

namespace nve_amd {

namespace {

int bits_for(uint64_t v) {
  int b = 0;
  while (b < 64 && (v >> b) != 0) ++b;
  return b;
}

template <typename T>
T* carve(uint8_t*& p, size_t count) {
  T* r = reinterpret_cast<T*>(p);
  p += (count * sizeof(T) + 255) / 256 * 256;
  return r;
}

struct SortedLookups {
  const uint32_t* pos;  // original positions in sort order
  const void* keys;     // keys in sort order (the key type)
  uint32_t misses;      // lookups [0, misses) of the order are misses
};

// Resolves and sorts the lookups: misses first, then hits, each by key.
SortedLookups sort_lookups(ExecutionContext& ctx, const GatherLaunch& g, int key_bytes,
                           uint64_t uvm_rows, bool want_misses, hipStream_t s) {
  const int64_t n = g.n;
  const int bits = std::max(1, std::min(62, bits_for(uvm_rows)));
  const int end_bit = bits + 1;
  const size_t bytes = 256 * 8 + (size_t)n * (8 * 2 + 4 * 2 + 8) + radix_sort_temp_bytes(n);
  uint8_t* p = static_cast<uint8_t*>(ctx.buffer("sort_gather", bytes));
  unsigned long long* nmiss = carve<unsigned long long>(p, kMissCounterWords);
  uint64_t* ka = carve<uint64_t>(p, (size_t)n);
  uint64_t* kb = carve<uint64_t>(p, (size_t)n);
  uint32_t* va = carve<uint32_t>(p, (size_t)n);
  uint32_t* vb = carve<uint32_t>(p, (size_t)n);
  uint8_t* sorted_keys = carve<uint8_t>(p, (size_t)n * 8);
  void* tmp = p;
  if (want_misses) NVE_HIP(launch_fill_u64(reinterpret_cast<uint64_t*>(nmiss), kMissCounterWords, 0, s));
  NVE_HIP(launch_sortgather_keys(g.keys, n, key_bytes, g.src, bits, ka, va, g.miss_counter,
                                 want_misses ? nmiss : nullptr, s));
  int alt = 0;
  NVE_HIP(radix_sort_pairs(ka, va, kb, vb, n, 0, end_bit, tmp, &alt, s));
  const uint32_t* pos = alt ? vb : va;
  NVE_HIP(launch_permute_keys(g.keys, key_bytes, pos, n, sorted_keys, s));
  SortedLookups r{pos, sorted_keys, 0};
  if (want_misses) {
    r.misses = (uint32_t)read_miss_words(nmiss, s);
  }
  return r;
}

}  // namespace

GpuTable::UvmMode GpuTable::uvm_mode(int64_t n) const {
  switch (cfg_.kernel_mode_type) {
    case 0: {
      // Automatic.  The reference switches to SortGather from 2^20 keys
      // (gpu_table.cu:271-287); here the direct lookup reads missed rows over
      // the host link at its random-row ceiling while the hits stream from
      // HBM, and measured faster at every size tried (262,144 / 1,048,576 /
      // 4,194,304 keys of the C3 table: 187 / 513 / 1,506 us per batch against
      // 277 / 702 / 2,050 sorted), so it stays direct unless kernel_mode_value
      // names a threshold.
      if (cfg_.kernel_mode_value == 0) return UvmMode::Lookup;
      return n < (int64_t)cfg_.kernel_mode_value ? UvmMode::Lookup : UvmMode::SortGather;
    }
    case 1: return UvmMode::Lookup;
    case 2: return UvmMode::SortGather;
    case 3: return UvmMode::PipelineGather;
    default: NVE_NOT_IMPLEMENTED("Unsupported kernel_mode_type ", cfg_.kernel_mode_type);
  }
}

void GpuTable::find_sort_gather(ExecutionContext& ctx, const GatherLaunch& g, hipStream_t s) {
  NVE_CHECK(g.n <= (int64_t)UINT32_MAX, "Too many keys for one sorted lookup");
  const SortedLookups sl = sort_lookups(ctx, g, key_bytes_, (uint64_t)cfg_.uvm_num_rows, false, s);
  GatherLaunch h = g;
  h.keys = sl.keys;
  h.out_index = sl.pos;
  h.miss_counter = nullptr;  // counted while sorting
  NVE_HIP(launch_gather(h, s));
}

void GpuTable::find_pipeline_gather(ExecutionContext& ctx, const GatherLaunch& g, hipStream_t s) {
  NVE_CHECK(g.n <= (int64_t)UINT32_MAX, "Too many keys for one pipelined lookup");
  const int64_t n = g.n;
  const SortedLookups sl = sort_lookups(ctx, g, key_bytes_, (uint64_t)cfg_.uvm_num_rows, true, s);
  const int64_t m = sl.misses;
  // hits: the GPU copies them from the cache (keys [m, n) of the order)
  if (n > m) {
    GatherLaunch h = g;
    h.keys = static_cast<const uint8_t*>(sl.keys) + (size_t)m * key_bytes_;
    h.n = n - m;
    h.out_index = sl.pos + m;
    h.miss_counter = nullptr;
    NVE_HIP(launch_gather(h, s));
  }
  if (m == 0) return;
  // misses: host threads copy the backing rows into pinned staging rows
  const uint64_t row = (uint64_t)cfg_.row_size_in_bytes;
  uint8_t* hp = static_cast<uint8_t*>(
      ctx.buffer("pipeline_host", (size_t)m * (key_bytes_ + 4) + 1024, true));
  uint8_t* h_keys = carve<uint8_t>(hp, (size_t)m * key_bytes_);
  uint32_t* h_pos = carve<uint32_t>(hp, (size_t)m);
  NVE_HIP(hipMemcpyAsync(h_keys, sl.keys, (size_t)m * key_bytes_, hipMemcpyDeviceToHost, s));
  NVE_HIP(hipMemcpyAsync(h_pos, sl.pos, (size_t)m * 4, hipMemcpyDeviceToHost, s));
  NVE_HIP(hipStreamSynchronize(s));
  uint8_t* staging = static_cast<uint8_t*>(ctx.buffer("pipeline_rows", (size_t)m * row, true));
  uint32_t* staged_pos = static_cast<uint32_t*>(ctx.buffer("pipeline_pos", (size_t)m * 4, true));
  const uint8_t* uvm = static_cast<const uint8_t*>(cfg_.uvm_table);
  const uint64_t rows = (uint64_t)cfg_.uvm_num_rows;
  const int kb = key_bytes_;
  const int64_t task = (int64_t)std::max<uint64_t>(1, pipeline_task_size_);
  const int64_t ntasks = (m + task - 1) / task;
  // each task compacts its keys inside the table into staging rows [b, b + kept)
  std::vector<std::future<int64_t>> done;
  done.reserve((size_t)ntasks);
  for (int64_t t = 0; t < ntasks; ++t) {
    const int64_t b = t * task, e = std::min(m, b + task);
    auto job = std::make_shared<std::packaged_task<int64_t()>>([=] {
      int64_t kept = 0;
      for (int64_t i = b; i < e; ++i) {
        int64_t key;
        if (kb == 4) {
          int32_t k32;
          std::memcpy(&k32, h_keys + (size_t)i * 4, 4);
          key = k32;
        } else {
          std::memcpy(&key, h_keys + (size_t)i * 8, 8);
        }
        if ((uint64_t)key >= rows) continue;  // outside the table: its row stays as it was
        std::memcpy(staging + (uint64_t)(b + kept) * row, uvm + (uint64_t)key * row, row);
        staged_pos[b + kept] = h_pos[i];
        ++kept;
      }
      return kept;
    });
    done.push_back(job->get_future());
    ctx.pool().submit([job] { (*job)(); });
  }
  // scatter each task's rows as soon as it is done (in task order)
  for (int64_t t = 0; t < ntasks; ++t) {
    const int64_t kept = done[(size_t)t].get();
    const int64_t b = t * task;
    NVE_HIP(launch_scatter_rows(staging + (uint64_t)b * row, staged_pos + b, kept, row,
                                static_cast<uint8_t*>(g.out), g.out_stride, s));
  }
  // the staging buffers are reused by the next call
  NVE_HIP(hipStreamSynchronize(s));
}

}  // namespace nve_amd
