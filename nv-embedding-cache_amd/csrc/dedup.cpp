// dedup.cpp -- host orchestration of key dedup (Deduper::dedup,
// deduper.cuh:136-221) and of the dedup-then-gather (a hash dedup, one table
// read per distinct key, then UnpackDedup, cuda_utils.cuh:24-79; batches past
// 2^30 keys sort instead and gather in key order).
#include "dedup.hpp"

#include "kernels/backprop_launch.hpp"
#include "kernels/cache_launch.hpp"
#include "kernels/dedup_launch.hpp"
#include "kernels/launch.hpp"
#include "kernels/modify_launch.hpp"
#include "kernels/sort_launch.hpp"
#include "runtime.hpp"

namespace nve_amd {

namespace {

int bits_for(uint64_t max_value) {
  int b = 0;
  while (b < 64 && (max_value >> b) != 0) ++b;
  return b;
}

struct DedupBufs {
  DedupHead* head;
  uint64_t* span_part;
  uint64_t *ka, *kb;
  uint32_t *va, *vb, *heads, *start;
  void* sort_tmp;
};

size_t pad(size_t b) { return (b + 255) / 256 * 256; }

DedupBufs carve(void* ws, int64_t n) {
  uint8_t* p = static_cast<uint8_t*>(ws);
  DedupBufs d;
  d.head = reinterpret_cast<DedupHead*>(p);
  p += 256;
  d.span_part = reinterpret_cast<uint64_t*>(p);
  p += pad(8 * (size_t)dedup_span_parts(n));
  d.ka = reinterpret_cast<uint64_t*>(p);
  p += pad(8 * n);
  d.kb = reinterpret_cast<uint64_t*>(p);
  p += pad(8 * n);
  d.va = reinterpret_cast<uint32_t*>(p);
  p += pad(4 * n);
  d.vb = reinterpret_cast<uint32_t*>(p);
  p += pad(4 * n);
  d.heads = reinterpret_cast<uint32_t*>(p);
  p += pad(4 * n);
  d.start = reinterpret_cast<uint32_t*>(p);
  p += pad(4 * (n + 1));
  d.sort_tmp = p;
  return d;
}

}  // namespace

// Scratch of the hash dedup-then-gather: table keys, owner per slot, slot per key.
size_t hash_gather_bytes(int64_t n) {
  const size_t slots = hash_dedup_slots(n);
  return pad(8 * slots) + pad(4 * slots) + pad(4 * (size_t)n);
}

// Batches up to this size take the hash path (slot numbers fit 32 bits).
constexpr int64_t kHashGatherMaxKeys = int64_t(1) << 30;

size_t dedup_workspace_bytes(int64_t n) {
  if (n < 1) n = 1;
  const size_t sort = 256 + pad(8 * (size_t)dedup_span_parts(n)) + 2 * pad(8 * n) + 4 * pad(4 * n) +
                      pad(4 * (n + 1)) + radix_sort_temp_bytes(n);
  const size_t hash = n <= kHashGatherMaxKeys ? hash_gather_bytes(n) : 0;
  return sort > hash ? sort : hash;
}

int64_t dedup_run(int key_bytes, int64_t n, const void* keys, void* unique, void* counts,
                  void* inverse, void* offsets, void* ws, size_t ws_bytes, hipStream_t s,
                  uint32_t* pos_key, const DedupHead** head_dev, bool exact, const PositionGrad* pg) {
  if (n <= 0) return 0;
  NVE_CHECK_ARG(n <= (int64_t)UINT32_MAX, "Too many keys for one dedup");
  NVE_CHECK_ARG(ws != nullptr && ws_bytes >= dedup_workspace_bytes(n), "Workspace too small");
  DedupBufs b = carve(ws, n);
  // a single key needs no sort: it takes the exact path, which sorts nothing
  if (n < 2) exact = true;
  int alt = 0;
  if (exact) {
    NVE_HIP(launch_dedup_prep(keys, key_bytes, n, 1, b.ka, b.va, s));
    NVE_HIP(launch_fill_u64(reinterpret_cast<uint64_t*>(&b.head->span), 1, 0, s));
    NVE_HIP(key_span(b.ka, n, &b.head->span, s));
    const int bits = bits_for(read_back(&b.head->span, s));
    NVE_HIP(radix_sort_pairs(b.ka, b.va, b.kb, b.vb, n, 0, bits, b.sort_tmp, &alt, s));
  } else {
    // the first pass reads the caller's keys and writes each tile's span part;
    // the outputs' workgroup 0 reduces them and whoever reads the head checks
    const RadixSource src{keys, key_bytes, 1, b.span_part};
    NVE_HIP(radix_sort_pairs(b.ka, b.va, b.kb, b.vb, n, 0, kSpecSortBits, b.sort_tmp, &alt, s, &src));
  }
  const uint64_t* ks = alt ? b.kb : b.ka;
  const uint32_t* vs = alt ? b.vb : b.va;
  if (run_blocks(n) <= kRunMaxBlocks) {
    // every output in two launches (block scratch in the heads / start arrays)
    NVE_HIP(launch_dedup_runs(ks, vs, n, key_bytes, unique, counts, inverse, offsets, pos_key, &b.head->total,
                              b.heads, reinterpret_cast<int64_t*>(b.start), exact ? nullptr : b.span_part,
                              exact ? nullptr : &b.head->span, pg, s));
    if (head_dev != nullptr) {
      *head_dev = b.head;
      return -1;
    }
    const DedupHead h = read_back(b.head, s);
    if (!exact && dedup_spec_failed(h))
      return dedup_run(key_bytes, n, keys, unique, counts, inverse, offsets, ws, ws_bytes, s, pos_key, nullptr,
                       true, pg);
    return (int64_t)h.total;
  }
  NVE_HIP(launch_run_heads(ks, n, b.heads, s));
  NVE_HIP(exclusive_scan_u32(b.heads, n, &b.head->total, b.sort_tmp, s));
  NVE_HIP(launch_dedup_outputs(ks, vs, b.heads, n, key_bytes, unique, inverse, offsets, b.start, pos_key,
                               exact ? nullptr : b.span_part, exact ? nullptr : &b.head->span, s));
  if (pg != nullptr) NVE_HIP(launch_backprop_prep(inverse, key_bytes, n, *pg, s));
  if (head_dev != nullptr) {  // the caller reads the head when it needs it
    NVE_HIP(launch_dedup_counts(b.start, (uint32_t)n, &b.head->total, key_bytes, counts, s));
    *head_dev = b.head;
    return -1;
  }
  const DedupHead h = read_back(b.head, s);
  if (!exact && dedup_spec_failed(h))
    return dedup_run(key_bytes, n, keys, unique, counts, inverse, offsets, ws, ws_bytes, s, pos_key, nullptr,
                     true, pg);
  NVE_HIP(launch_dedup_counts(b.start, h.total, nullptr, key_bytes, counts, s));
  return (int64_t)h.total;
}

void dedup_gather_run(int key_bytes, int64_t n, const void* keys, const uint8_t* table,
                      int64_t num_rows, int64_t row_bytes, void* out, int64_t out_stride, void* ws,
                      size_t ws_bytes, hipStream_t s) {
  if (n <= 0) return;
  NVE_CHECK_ARG(n <= (int64_t)UINT32_MAX, "Too many keys for one dedup");
  NVE_CHECK_ARG(ws != nullptr && ws_bytes >= dedup_workspace_bytes(n), "Workspace too small");
  if (n <= kHashGatherMaxKeys) {
    // hash dedup: no order is needed, only one read of each distinct row
    uint8_t* p = static_cast<uint8_t*>(ws);
    const size_t slots = hash_dedup_slots(n);
    void* tab = p;  // keys of 4 or 8 bytes (room for 8)
    p += pad(8 * slots);
    uint32_t* owner = reinterpret_cast<uint32_t*>(p);
    p += pad(4 * slots);
    uint32_t* slot_of = reinterpret_cast<uint32_t*>(p);
    NVE_HIP(launch_hash_dedup_gather(keys, key_bytes, n, table, num_rows, row_bytes, out, out_stride, tab,
                                     owner, slot_of, s));
    return;
  }
  DedupBufs b = carve(ws, n);
  // rows of [0, num_rows): sort on the row-index bits only (keys outside the
  // table stay unresolved and their output rows untouched)
  NVE_HIP(launch_dedup_prep(keys, key_bytes, n, 0, b.ka, b.va, s));
  int alt = 0;
  NVE_HIP(radix_sort_pairs(b.ka, b.va, b.kb, b.vb, n, 0,
                           bits_for((uint64_t)(num_rows > 1 ? num_rows - 1 : 1)),
                           b.sort_tmp, &alt, s));
  GatherLaunch g{};
  g.keys = alt ? b.kb : b.ka;  // sorted keys as int64
  g.key_bytes = 8;
  g.n = n;
  g.src.table = table;
  g.src.row_bytes = (uint64_t)row_bytes;
  g.src.load_indices = 1;
  g.src.num_rows = (uint64_t)num_rows;
  g.raw = 1;
  g.out = out;
  g.out_stride = out_stride;
  g.out_index = alt ? b.vb : b.va;  // original positions in key order
  NVE_HIP(launch_gather(g, s));
}

}  // namespace nve_amd
