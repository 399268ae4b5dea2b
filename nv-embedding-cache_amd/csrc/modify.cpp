// modify.cpp -- GpuTable::insert / insert_from_uvm: the cache insert pipeline
// on the modify stream.
//
//   keys -> (1) histogram: stable radix sort of the keys, run-length encode,
//                stable sort of the runs by count descending, truncate to
//                max_modify_size (gather_keys_data_ptrs.cuh:121-191,
//                gpu_table.cu:416-576)
//        -> (2) group by set: stable radix sort of (set, histogram index)
//                (ec_set_associative_modify.cuh:364-513)
//        -> (3) per-set replacement kernel -> records (slot, tag, source row)
//        -> (4) invalidate the records' tags, order the copy after the lookups
//                queued on the table's registered lookup streams, copy the
//                rows, commit the tags (ec_set_associative_device_modify.cuh:
//                225-288, :428-451)
// The host reads two counts back (unique keys, represented sets) and waits
// once for the invalidation, where the reference also synchronizes
// (gather_keys_data_ptrs.cuh:168, ec_set_associative_modify.cuh:489,
// ec_set_associative_device_modify.cuh:443).  The key sort first assumes that
// the keys differ only below bit kInsertSpecBits (rows of tables up to 2^32:
// four 8-bit passes, as many as 25 to 32 exact bits take) and learns whether
// they did with the unique count; a batch whose keys differ higher up is
// sorted again on its exact bits.
//
// Caches with at least as many sets as keys take the hashed histogram instead
// of (1) and (2) (GpuTable::hashed_insert, modify.hip): hash counts, per-set
// candidate chains and each set's candidates sorted into histogram order in
// its replacement group; no readback, one wait.
#include <algorithm>
#include <cmath>
#include <cstring>

#include "kernels/cache_launch.hpp"
#include "kernels/modify_launch.hpp"
#include "kernels/sort_launch.hpp"
#include "layers.hpp"

namespace nve_amd {

namespace {

constexpr int kInsertSpecBits = 32;

// Read back after the histogram's first sort: unique keys, and the OR over
// the keys of key ^ key[0] (the bits where they differ).
struct InsertHead {
  uint32_t uniq;
  uint32_t pad;
  unsigned long long span;
};

int bits_for(uint64_t max_value) {
  int b = 0;
  while (b < 64 && (max_value >> b) != 0) ++b;
  return b;
}


template <typename T>
T* carve(uint8_t*& p, size_t count) {
  T* r = reinterpret_cast<T*>(p);
  p += (count * sizeof(T) + 255) / 256 * 256;
  return r;
}

uint32_t read_u32(const uint32_t* d, hipStream_t s) {
  return read_back(d, s);
}

}  // namespace

// Decay factors (float)pow((double)rate, (double)d) for d < len; the table
// ends where the factor has become 0 in float (every larger d is 0 too) or at
// 1M entries, beyond which the kernel evaluates pow itself.
void GpuTable::build_decay_table() {
  std::vector<float> t;
  t.push_back(1.0f);
  if (decay_rate_ < 1.0f) {
    for (int64_t d = 1; d < (1 << 20); ++d) {
      const float f = (float)std::pow((double)decay_rate_, (double)d);
      t.push_back(f);
      if (f == 0.0f) break;
    }
  }
  decay_len_ = (int64_t)t.size();
  NVE_HIP(hipMalloc((void**)&decay_table_, t.size() * sizeof(float)));
  NVE_HIP(hipMemcpy(decay_table_, t.data(), t.size() * sizeof(float), hipMemcpyHostToDevice));
}

void GpuTable::insert(ExecutionContext& ctx, int64_t n, const void* keys, int64_t value_stride,
                      int64_t value_size, const void* values) {
  ScopedDevice sd(cfg_.device_id);
  if (n <= 0) return;
  NVE_CHECK_ARG(keys != nullptr, "keys must not be null");
  NVE_CHECK(values != nullptr, "Invalid cache insert params");
  NVE_CHECK(value_size == cfg_.row_size_in_bytes, "Unsupported value_size");
  NVE_CHECK_ARG(value_stride >= value_size, "value_stride is smaller than value_size");
  StreamQueue q(ctx.modify_stream(), cfg_.private_stream);
  const void* d_vals = device_input(ctx, "insert_values", values,
                                    (size_t)(n - 1) * value_stride + value_size, q.stream);
  if (cfg_.modify_on_gpu)
    modify_insert(ctx, q.stream, n, keys, static_cast<const uint8_t*>(d_vals), value_stride, false);
  else
    host_modify_insert(ctx, q.stream, n, keys, static_cast<const uint8_t*>(d_vals), value_stride, false);
}

void GpuTable::insert_from_uvm(ExecutionContext& ctx, int64_t n, const void* keys) {
  ScopedDevice sd(cfg_.device_id);
  NVE_CHECK(cfg_.uvm_table != nullptr, "insert_from_uvm requires a UVM table");
  if (n <= 0) return;
  NVE_CHECK_ARG(keys != nullptr, "keys must not be null");
  StreamQueue q(ctx.modify_stream(), cfg_.private_stream);
  const uint8_t* rows = static_cast<const uint8_t*>(cfg_.uvm_table);
  if (cfg_.modify_on_gpu)
    modify_insert(ctx, q.stream, n, keys, rows, cfg_.row_size_in_bytes, true);
  else
    host_modify_insert(ctx, q.stream, n, keys, rows, cfg_.row_size_in_bytes, true);
}

// The hashed histogram (large caches): hash counts -> per-set chains -> per-set
// replacement with the candidates sorted in their set -> invalidate; one
// synchronization (where the sorted path also waits), which also reads the
// overflow word; then the rows and tags.  Six launches before the wait and
// two after, against about forty and two readbacks for the sorted histogram.
bool GpuTable::hashed_insert(ExecutionContext& ctx, hipStream_t s, int64_t n, const void* d_keys,
                             const uint8_t* rows, int64_t row_stride, bool from_uvm) {
  if (set_words_dirty_) {  // an earlier insert stopped part way
    NVE_HIP(launch_fill_u64(set_word_, (int64_t)num_sets_, kSetClean, s));
    set_words_dirty_ = false;
  }
  int bits = 10;
  while ((1ll << bits) < 2 * n) ++bits;
  const size_t slots = ((size_t)1 << bits) + 1;
  const size_t un = (size_t)n;
  const size_t bytes = 12 * 256 + slots * (8 + 4 + 4) + un * (4 * 3 + 8 * 3) + 64 * 256;
  uint8_t* p = static_cast<uint8_t*>(ctx.buffer("insert_hashed", bytes));
  HashInsertLaunch h{};
  h.keys = d_keys;
  h.key_bytes = key_bytes_;
  h.n = n;
  h.bits = bits;
  h.tkey = carve<uint64_t>(p, slots);
  h.tcount = carve<uint32_t>(p, slots);
  h.tfirst = carve<uint32_t>(p, slots);
  h.ulist = carve<uint32_t>(p, un);
  h.unext = carve<uint32_t>(p, un);
  h.rsets = carve<uint32_t>(p, un);
  h.counts = carve<uint32_t>(p, 4);
  h.set_word = set_word_;
  h.num_sets = num_sets_;
  h.norm = 1.0f / (float)n;
  h.rows_base = rows;
  h.row_stride = row_stride;
  h.by_key = from_uvm ? 1 : 0;
  uint64_t* rec_slot = carve<uint64_t>(p, un);
  int64_t* rec_tag = carve<int64_t>(p, un);
  uint64_t* rec_src = carve<uint64_t>(p, un);
  ReplaceLaunch r{};
  r.tags = tags_;
  r.counters = counters_;
  r.set_ts = set_ts_;
  r.global_ts = global_ts_;
  r.decay_rate = decay_rate_;
  r.decay_table = decay_table_;
  r.decay_len = decay_len_;
  r.num_sets = num_sets_;
  r.sentinel = cfg_.invalid_key;
  r.src_rows = from_uvm ? (uint64_t)cfg_.uvm_num_rows : 0;
  r.max_records = (uint32_t)n;
  r.rec_slot = rec_slot;
  r.rec_tag = rec_tag;
  r.rec_src = rec_src;
  // the words are dirty from here until the replacement has run to its end
  set_words_dirty_ = true;
  NVE_HIP(launch_hash_insert(h, r, s));
  set_words_dirty_ = false;  // stream order: the next insert's kernels follow these
  const uint32_t* num = h.counts;  // records: one position per unique key
  NVE_HIP(launch_invalidate(num, (uint32_t)n, rec_slot, tags_, key_bytes_, cfg_.invalid_key, s));
  uint32_t* flags = static_cast<uint32_t*>(ctx.buffer("insert_hashed_flags", 64, true));
  NVE_HIP(launch_small_read(flags, h.counts, 16, s));
  // Lookups queued from here on see the invalidated tags; earlier ones may
  // still read the replaced rows, so the copy waits for them
  NVE_HIP(hipStreamSynchronize(s));
  if (flags[2] != 0u) return false;  // a set past kHashSetMax candidates: nothing changed
  lookups_->order_before(s);
  uintptr_t align = (uintptr_t)rows | (uintptr_t)row_stride;
  const int src_align = (align % 16 == 0) ? 16 : (align % 4 == 0) ? 4 : 1;
  NVE_HIP(launch_copy_rows(num, (uint32_t)n, rec_slot, rec_src, src_align, data_,
                           (uint64_t)cfg_.row_size_in_bytes, s));
  NVE_HIP(launch_commit(num, (uint32_t)n, rec_slot, rec_tag, tags_, key_bytes_, s));
  NVE_HIP(hipStreamSynchronize(s));
  return true;
}

void GpuTable::modify_insert(ExecutionContext& ctx, hipStream_t s, int64_t n, const void* keys,
                             const uint8_t* rows, int64_t row_stride, bool from_uvm) {
  NVE_CHECK(n <= (int64_t)UINT32_MAX, "Too many keys for one insert");
  std::lock_guard<std::mutex> mk(modify_mu_);
  const void* d_keys = device_input(ctx, "modify_keys", keys, (size_t)n * key_bytes_, s);
  ++global_ts_;  // once per insert (ec_set_associative_device_modify.cuh:262)
  // The hashed histogram where a set's candidates are few (fewer sets than
  // keys would crowd them), none is cut (n <= max_modify_size) and the
  // reference's histogram positions, which MergeBlock passes through a float,
  // are exact (n <= 2^24), so that places within a set give the same result
  if (n >= 2 && n <= cfg_.max_modify_size && n <= (1ll << 24) && num_sets_ >= (uint64_t)n &&
      hashed_insert(ctx, s, n, d_keys, rows, row_stride, from_uvm))
    return;

  // ---- scratch (grow-only, per context) ----
  const size_t un = (size_t)n;
  const size_t bytes = 18 * 256 + un * (8 * 2 + 4 * 2) * 3 + un * (4 * 4 + 8 * 4) +
                       (size_t)radix_tiles(n) * 8 + radix_sort_temp_bytes(n) + 64 * 256;
  uint8_t* p = static_cast<uint8_t*>(ctx.buffer("insert_scratch", bytes));
  unsigned long long* d_span = carve<unsigned long long>(p, 1);
  InsertHead* head = carve<InsertHead>(p, 1);
  uint64_t* span_part = carve<uint64_t>(p, (size_t)radix_tiles(n));
  uint32_t* d_count = carve<uint32_t>(p, 4);
  uint64_t* ka = carve<uint64_t>(p, un);
  uint32_t* va = carve<uint32_t>(p, un);
  uint64_t* kb = carve<uint64_t>(p, un);
  uint32_t* vb = carve<uint32_t>(p, un);
  uint32_t* heads = carve<uint32_t>(p, un);
  uint32_t* start = carve<uint32_t>(p, un + 1);
  uint64_t* ukey = carve<uint64_t>(p, un);
  uint32_t* first = carve<uint32_t>(p, un);
  int64_t* hkeys = carve<int64_t>(p, un);
  float* hprio = carve<float>(p, un);
  uint64_t* hsrc = carve<uint64_t>(p, un);
  uint32_t* rset = carve<uint32_t>(p, un);
  uint32_t* roff = carve<uint32_t>(p, un + 1);
  uint64_t* rec_slot = carve<uint64_t>(p, un);
  int64_t* rec_tag = carve<int64_t>(p, un);
  uint64_t* rec_src = carve<uint64_t>(p, un);
  void* sort_tmp = carve<uint8_t>(p, radix_sort_temp_bytes(n));

  // ---- (1) histogram ----
  int alt = 0;
  uint32_t uniq = 0;
  bool exact = n < 2;  // one key: nothing to sort, the exact path sorts nothing
  if (!exact) {
    // the first pass reads the caller's keys and writes each tile's span part
    const RadixSource src{d_keys, key_bytes_, 1, span_part};
    NVE_HIP(radix_sort_pairs(ka, va, kb, vb, n, 0, kInsertSpecBits, sort_tmp, &alt, s, &src));
    NVE_HIP(launch_run_heads(alt ? kb : ka, n, heads, s, span_part, radix_tiles(n), &head->span));
    NVE_HIP(exclusive_scan_u32(heads, n, &head->uniq, sort_tmp, s));
    const InsertHead h = read_back(head, s);
    exact = (h.span >> kInsertSpecBits) != 0;
    uniq = h.uniq;
  }
  if (exact) {
    NVE_HIP(launch_hist_prep(d_keys, key_bytes_, n, ka, va, s));
    NVE_HIP(launch_fill_u64(reinterpret_cast<uint64_t*>(d_span), 1, 0, s));
    NVE_HIP(key_span(ka, n, d_span, s));
    const unsigned long long span = read_back(d_span, s);
    NVE_HIP(radix_sort_pairs(ka, va, kb, vb, n, 0, bits_for(span), sort_tmp, &alt, s));
    NVE_HIP(launch_run_heads(alt ? kb : ka, n, heads, s));
    NVE_HIP(exclusive_scan_u32(heads, n, d_count, sort_tmp, s));
    uniq = read_u32(d_count, s);
  }
  uint64_t* ks = alt ? kb : ka;
  uint32_t* vs = alt ? vb : va;
  NVE_HIP(launch_run_gather(ks, vs, heads, n, start, ukey, first, s));
  // sort the runs by count descending (stable: ties keep ascending key order)
  uint64_t* k2 = alt ? ka : kb;  // the buffers not holding ks / vs
  uint32_t* v2 = alt ? va : vb;
  uint64_t* k2b = reinterpret_cast<uint64_t*>(rec_slot);
  uint32_t* v2b = reinterpret_cast<uint32_t*>(rset);
  NVE_HIP(launch_count_key(start, uniq, k2, v2, s));
  int alt2 = 0;
  NVE_HIP(radix_sort_pairs(k2, v2, k2b, v2b, uniq, 0, bits_for((uint64_t)n), sort_tmp, &alt2, s));
  const uint32_t* order = alt2 ? v2b : v2;
  const uint32_t m = (uint32_t)std::min<int64_t>(uniq, cfg_.max_modify_size);
  // hist entries and their sets (k3 / v3 reuse the first sort's free buffers)
  uint64_t* k3 = alt ? kb : ka;
  uint32_t* v3 = alt ? vb : va;
  NVE_HIP(launch_hist_gather(order, start, ukey, first, m, key_bytes_, 1.0f / (float)n, rows,
                             row_stride, from_uvm ? 1 : 0, num_sets_, hkeys, hprio, hsrc, k3, v3, s));

  // ---- (2) group by set ----
  uint64_t* k3b = reinterpret_cast<uint64_t*>(ukey);  // runs' keys are consumed by now
  uint32_t* v3b = heads;
  int alt3 = 0;
  NVE_HIP(radix_sort_pairs(k3, v3, k3b, v3b, m, 0, bits_for(num_sets_ - 1), sort_tmp, &alt3, s));
  const uint64_t* sk = alt3 ? k3b : k3;
  const uint32_t* sv = alt3 ? v3b : v3;
  NVE_HIP(launch_run_heads(sk, m, start, s));  // start reused as head flags
  NVE_HIP(exclusive_scan_u32(start, m, d_count, sort_tmp, s));
  const uint32_t nrs = read_u32(d_count, s);
  NVE_HIP(launch_set_gather(sk, start, m, rset, roff, s));

  // ---- (3) replacement ----
  ReplaceLaunch r{};
  r.rset = rset;
  r.roff = roff;
  r.num_rsets = nrs;
  r.order = sv;
  r.hkeys = hkeys;
  r.hprio = hprio;
  r.hsrc = hsrc;
  r.tags = tags_;
  r.counters = counters_;
  r.set_ts = set_ts_;
  r.global_ts = global_ts_;
  r.decay_rate = decay_rate_;
  r.decay_table = decay_table_;
  r.decay_len = decay_len_;
  r.num_sets = num_sets_;
  r.sentinel = cfg_.invalid_key;
  r.src_rows = from_uvm ? (uint64_t)cfg_.uvm_num_rows : 0;  // keys past the backing table: no candidates
  r.max_records = m;
  r.rec_slot = rec_slot;
  r.rec_tag = rec_tag;
  r.rec_src = rec_src;
  NVE_HIP(launch_set_replace(r, key_bytes_, s));

  // ---- (4) invalidate -> drain -> copy -> commit ----
  NVE_HIP(launch_invalidate(nullptr, m, rec_slot, tags_, key_bytes_, cfg_.invalid_key, s));
  // Lookups queued from here on see the invalidated tags (the invalidation is
  // complete before the host goes on); lookups queued earlier may still read
  // the old rows of those ways, so the copy waits for them
  NVE_HIP(hipStreamSynchronize(s));
  lookups_->order_before(s);
  uintptr_t align = (uintptr_t)rows | (uintptr_t)row_stride;
  const int src_align = (align % 16 == 0) ? 16 : (align % 4 == 0) ? 4 : 1;
  NVE_HIP(launch_copy_rows(nullptr, m, rec_slot, rec_src, src_align, data_,
                           (uint64_t)cfg_.row_size_in_bytes, s));
  NVE_HIP(launch_commit(nullptr, m, rec_slot, rec_tag, tags_, key_bytes_, s));
  NVE_HIP(hipStreamSynchronize(s));
}

}  // namespace nve_amd
