// host_modify.cpp -- GpuTable with modify_on_gpu = false: the reference's
// CacheSAHostModify policy (ec_set_associative_host_modify.h:218-296).
//
// The replacement decision is sequential over the histogram, so it runs on
// the host, over a host copy of the tags and the host-resident counters and
// set timestamps.  Only the outcome touches the GPU: the chosen ways are
// uploaded as records and go through the same invalidate -> drain -> copy ->
// commit kernels as the device policy (modify(), :428-480).
//
//   histogram   DefaultHistogram (embed_cache.h:188-229): bins in order of
//               first occurrence, count as a float, sorted by count
//               descending; priority = count / n.  std::sort there leaves the
//               order of equal counts unspecified; here it is first
//               occurrence (std::stable_sort).
//   per bin     decay its set on the first touch of this call by
//               (float)pow((double)rate, (double)(now - set_ts)); a resident
//               key adds its priority to its way; else the first way with the
//               smallest counter (empty ways included, with whatever counter
//               they kept) is replaced when priority >= that counter and no
//               earlier bin of this call took that way.  Stops at
//               max_modify_size records.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <unordered_map>
#include <unordered_set>

#include "kernels/cache_launch.hpp"
#include "kernels/modify_launch.hpp"
#include "layers.hpp"

namespace nve_amd {

// ec_hash.h:36-60 on the host: unsigned arithmetic in the key type's width.
int64_t GpuTable::load_key(const uint8_t* keys, int64_t i) const {
  if (key_bytes_ == 4) {
    int32_t k;
    std::memcpy(&k, keys + (size_t)i * 4, 4);
    return k;
  }
  int64_t k;
  std::memcpy(&k, keys + (size_t)i * 8, 8);
  return k;
}

uint64_t GpuTable::set_of(int64_t key) const {
  if (key_bytes_ == 4) return (uint32_t)(int32_t)key % (uint32_t)num_sets_;
  return (uint64_t)key % num_sets_;
}

int64_t GpuTable::tag_of(int64_t key) const {
  if (key_bytes_ == 4) return (int32_t)((uint32_t)(int32_t)key / (uint32_t)num_sets_);
  return (int64_t)((uint64_t)key / num_sets_);
}

int64_t GpuTable::key_of(int64_t tag, uint64_t set) const {
  if (key_bytes_ == 4) return (int32_t)((uint32_t)(int32_t)tag * (uint32_t)num_sets_ + (uint32_t)set);
  return (int64_t)((uint64_t)tag * num_sets_ + set);
}

int64_t GpuTable::h_tag(uint64_t slot) const { return load_key(h_tags_.data(), (int64_t)slot); }

void GpuTable::set_h_tag(uint64_t slot, int64_t tag) {
  uint8_t* p = h_tags_.data() + (size_t)slot * key_bytes_;
  if (key_bytes_ == 4) {
    const int32_t t = (int32_t)tag;
    std::memcpy(p, &t, 4);
  } else {
    std::memcpy(p, &tag, 8);
  }
}

void GpuTable::apply_records(ExecutionContext& ctx, hipStream_t s, const std::vector<uint64_t>& slot,
                             const std::vector<int64_t>& tag, const std::vector<uint64_t>& src,
                             bool invalidate_only) {
  const size_t n = slot.size();
  if (n == 0) return;
  NVE_CHECK(n <= (size_t)UINT32_MAX, "Too many cache records");
  auto pad = [](size_t b) { return (b + 255) / 256 * 256; };
  const size_t bytes = 256 + 2 * pad(n * 8) + pad(n * 8);
  // one host block (count, slots, tags, sources) and one copy of it
  uint8_t* h = static_cast<uint8_t*>(ctx.buffer("host_modify_records_h", bytes, true));
  uint8_t* d = static_cast<uint8_t*>(ctx.buffer("host_modify_records", bytes));
  const uint32_t cnt = (uint32_t)n;
  std::memcpy(h, &cnt, 4);
  std::memcpy(h + 256, slot.data(), n * 8);
  std::memcpy(h + 256 + pad(n * 8), tag.data(), n * 8);
  std::memcpy(h + 256 + 2 * pad(n * 8), src.data(), n * 8);
  NVE_HIP(hipMemcpyAsync(d, h, bytes, hipMemcpyHostToDevice, s));
  const uint32_t* d_num = reinterpret_cast<const uint32_t*>(d);
  const uint64_t* d_slot = reinterpret_cast<const uint64_t*>(d + 256);
  const int64_t* d_tag = reinterpret_cast<const int64_t*>(d + 256 + pad(n * 8));
  const uint64_t* d_src = reinterpret_cast<const uint64_t*>(d + 256 + 2 * pad(n * 8));
  NVE_HIP(launch_invalidate(d_num, cnt, d_slot, tags_, key_bytes_, cfg_.invalid_key, s));
  NVE_HIP(hipStreamSynchronize(s));
  if (!invalidate_only) {
    // lookups queued before the invalidation finish before a row is overwritten
    lookups_->order_before(s);
    uintptr_t align = 0;
    for (uint64_t p : src) align |= (uintptr_t)p;
    const int src_align = (align % 16 == 0) ? 16 : (align % 4 == 0) ? 4 : 1;
    NVE_HIP(launch_copy_rows(d_num, cnt, d_slot, d_src, src_align, data_,
                             (uint64_t)cfg_.row_size_in_bytes, s));
    NVE_HIP(launch_commit(d_num, cnt, d_slot, d_tag, tags_, key_bytes_, s));
  }
  NVE_HIP(hipStreamSynchronize(s));
}

void GpuTable::host_modify_insert(ExecutionContext& ctx, hipStream_t s, int64_t n, const void* keys,
                                  const uint8_t* rows, int64_t row_stride, bool from_uvm) {
  std::lock_guard<std::mutex> mk(modify_mu_);
  const uint8_t* hk =
      static_cast<const uint8_t*>(host_input(ctx, "modify_keys_host", keys, (size_t)n * key_bytes_, s));

  struct Bin {
    int64_t key;
    int64_t first;
    float count;
  };
  std::vector<Bin> bins;
  bins.reserve((size_t)std::min<int64_t>(n, 1 << 22));
  std::unordered_map<int64_t, uint32_t> bin_of;
  bin_of.reserve((size_t)std::min<int64_t>(n, 1 << 22));
  for (int64_t i = 0; i < n; ++i) {
    const int64_t k = load_key(hk, i);
    auto it = bin_of.find(k);
    if (it == bin_of.end()) {
      bin_of.emplace(k, (uint32_t)bins.size());
      bins.push_back({k, i, 1.0f});
    } else {
      bins[it->second].count += 1.0f;
    }
  }
  std::stable_sort(bins.begin(), bins.end(), [](const Bin& a, const Bin& b) { return a.count > b.count; });

  const float total = (float)n;
  const int64_t now = ++global_ts_;
  const uint64_t backing_rows = (uint64_t)cfg_.uvm_num_rows;
  std::unordered_set<uint64_t> taken;  // ways replaced in this call (the reference's insertMap)
  std::vector<uint64_t> slot;
  std::vector<int64_t> tag;
  std::vector<uint64_t> src;
  for (size_t b = 0; b < bins.size() && (int64_t)slot.size() < cfg_.max_modify_size; ++b) {
    const int64_t key = bins[b].key;
    const float prio = bins[b].count / total;
    const uint64_t set = set_of(key);
    float* sc = h_counters_.data() + set * kWays;
    if (h_set_ts_[set] != now) {
      const float f = (float)std::pow((double)decay_rate_, (double)(now - h_set_ts_[set]));
      for (int w = 0; w < kWays; ++w) sc[w] *= f;
      h_set_ts_[set] = now;
    }
    bool hit = false;
    for (int w = 0; w < kWays; ++w) {
      if (key_of(h_tag(set * kWays + w), set) == key) {
        sc[w] += prio;
        hit = true;
        break;
      }
    }
    if (hit) continue;
    // a key outside the backing table has no row to insert from (the
    // reference would read past the table): it is not a candidate
    if (from_uvm && (uint64_t)key >= backing_rows) continue;
    const int wmin = (int)(std::min_element(sc, sc + kWays) - sc);
    if (sc[wmin] > prio) continue;
    const uint64_t sl = set * kWays + (uint64_t)wmin;
    if (!taken.insert(sl).second) continue;
    sc[wmin] = prio;
    const int64_t t = tag_of(key);
    set_h_tag(sl, t);
    slot.push_back(sl);
    tag.push_back(t);
    const int64_t idx = from_uvm ? key : bins[b].first;
    src.push_back((uint64_t)(uintptr_t)(rows + (uint64_t)idx * (uint64_t)row_stride));
  }
  apply_records(ctx, s, slot, tag, src, false);
}

}  // namespace nve_amd
