// modify.hip -- cache insert on the GPU: key histogram, per-set replacement
// policy and the invalidate -> copy rows -> commit tags protocol.
//
// Reference behaviour restated (file:line in /root/reference):
//   histogram   DefaultGPUHistogram::compute_histogram (gather_keys_data_ptrs.cuh:121-191):
//               unique keys ordered by count descending, ties by ascending key
//               (stable sorts), priority = float(count) * (1 / float(n)), row =
//               backing table + key*row (insert_from_uvm) or values + first
//               position*stride (insert)
//   replacement SetReplaceDataKernel + SortBlock + MergeBlock
//               (ec_set_associative_modify.cuh:36-309): per touched set, lazy
//               decay of the 8 way counters by rate^(ts - set_ts), hits add
//               their priority, misses compete 8 at a time through the bitonic
//               networks, the best <= min(8, candidates) replace the ways of
//               lowest counter (an empty way counts 0) when priority > counter
//   protocol    CacheSADeviceModify::insert (ec_set_associative_device_modify.cuh:225-288):
//               invalidate the replaced ways' tags, synchronize, copy the rows,
//               write the new tags
//
// The replacement runs one 8-lane group per set (8 sets per wave); the way
// counters live in the lanes' registers and the two bitonic networks are
// shuffles inside the group, lane for lane the reference's networks (their tie
// rules included), so the resulting residency is the same.  The decay factor
// comes from a table of (float)pow((double)rate, (double)delta) built on the
// host; the reference computes it with CUDA's __powf, whose bits are not
// published.
#include <algorithm>

#include "device_common.cuh"
#include "modify_launch.hpp"
#include "sort_launch.hpp"

namespace nve_amd {

__global__ __launch_bounds__(256) void hist_prep_kernel(const void* keys, int key_bytes, int64_t n,
                                                        uint64_t* k64, uint32_t* v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    k64[i] = flip_key(load_key(keys, key_bytes, i), key_bytes);
    v[i] = (uint32_t)i;
  }
}

// heads[i] = 1 where a run of equal sorted keys starts
// span_part (optional, nparts words): workgroup 0 also ORs the sort's span
// parts into *span_out.
__global__ __launch_bounds__(256) void run_heads_kernel(const uint64_t* ks, int64_t n,
                                                        uint32_t* heads, const uint64_t* span_part,
                                                        int64_t nparts, unsigned long long* span_out) {
  if (span_part != nullptr && blockIdx.x == 0) {  // uniform over the workgroup
    uint64_t x = 0;
    for (int64_t j = threadIdx.x; j < nparts; j += blockDim.x) x |= span_part[j];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x |= __shfl_xor(x, o);
    __shared__ uint64_t red[4];
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
    __syncthreads();
    if (threadIdx.x == 0) *span_out = red[0] | red[1] | red[2] | red[3];
  }
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) heads[i] = (i == 0 || ks[i] != ks[i - 1]) ? 1u : 0u;
}

// For each run u (start i): start[u] = i, key[u], first position[u]; start[U] = n.
// heads was scanned in place (exclusive), flags recomputed from the keys.
__global__ __launch_bounds__(256) void run_gather_kernel(const uint64_t* ks, const uint32_t* vs,
                                                         const uint32_t* scan, int64_t n,
                                                         uint32_t* start, uint64_t* ukey,
                                                         uint32_t* first) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const bool head = (i == 0 || ks[i] != ks[i - 1]);
  if (head) {
    const uint32_t u = scan[i];
    start[u] = (uint32_t)i;
    ukey[u] = ks[i];
    first[u] = vs[i];
  }
  if (i == n - 1) start[scan[i] + (head ? 1u : 0u)] = (uint32_t)n;
}

// count sort key: ascending order of (max_count - count) = count descending
__global__ __launch_bounds__(256) void count_key_kernel(const uint32_t* start, uint32_t u_n,
                                                        uint64_t* k2, uint32_t* v2) {
  const uint32_t u = blockIdx.x * blockDim.x + threadIdx.x;
  if (u < u_n) {
    const uint32_t c = start[u + 1] - start[u];
    k2[u] = (uint64_t)(0xffffffffu - c);
    v2[u] = u;
  }
}

// Histogram entry h (hist order): key, priority, source row, and its set.
__global__ __launch_bounds__(256) void hist_gather_kernel(
    const uint32_t* order, const uint32_t* start, const uint64_t* ukey, const uint32_t* first,
    uint32_t m, int key_bytes, float norm, const uint8_t* rows_base, int64_t row_stride,
    int by_key, uint64_t num_sets, int64_t* hkeys, float* hprio, uint64_t* hsrc, uint64_t* k3,
    uint32_t* v3) {
  const uint32_t h = blockIdx.x * blockDim.x + threadIdx.x;
  if (h >= m) return;
  const uint32_t u = order[h];
  const int64_t key = unflip_key(ukey[u], key_bytes);
  const uint32_t c = start[u + 1] - start[u];
  hkeys[h] = key;
  hprio[h] = (float)(int32_t)c * norm;
  const int64_t idx = by_key ? key : (int64_t)first[u];
  hsrc[h] = (uint64_t)rows_base + (uint64_t)idx * (uint64_t)row_stride;
  const uint64_t set = key_bytes == 4 ? (uint64_t)((uint32_t)(int32_t)key % (uint32_t)num_sets)
                                      : (uint64_t)key % num_sets;
  k3[h] = set;
  v3[h] = h;
}

// represented sets: rset[r], roff[r] (start in the set-sorted order), roff[R] = m
__global__ __launch_bounds__(256) void set_gather_kernel(const uint64_t* ks, const uint32_t* scan,
                                                         int64_t m, uint32_t* rset, uint32_t* roff) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= m) return;
  const bool head = (i == 0 || ks[i] != ks[i - 1]);
  if (head) {
    rset[scan[i]] = (uint32_t)ks[i];
    roff[scan[i]] = (uint32_t)i;
  }
  if (i == m - 1) roff[scan[i] + (head ? 1u : 0u)] = (uint32_t)m;
}

// ---------------------------------------------------------------------------
// replacement: one 8-lane group per represented set
// ---------------------------------------------------------------------------
__device__ __forceinline__ float g8f(float v, int src) { return __shfl(v, src, 8); }
__device__ __forceinline__ uint32_t g8u(uint32_t v, int src) {
  return (uint32_t)__shfl((int)v, src, 8);
}

// SortBlock (ec_set_associative_modify.cuh:36-71): bitonic network over the 8
// lanes, a lane swapping with its partner only when the values differ.
__device__ __forceinline__ void sort_block8(float& v, uint32_t& pos, int x) {
  for (int k = 2; k <= 8; k *= 2) {
    for (int j = k / 2; j > 0; j /= 2) {
      const int p = x ^ j;
      const uint32_t pp = g8u(pos, p);
      const float pv = g8f(v, p);
      if (v != pv) {
        const bool in_order_pos = x > p;
        const bool in_order_val = v > pv;
        const bool swap = (x & k) ? (in_order_pos != in_order_val) : (in_order_pos == in_order_val);
        if (swap) {
          pos = pp;
          v = pv;
        }
      }
    }
  }
}

// MergeBlock (ec_set_associative_modify.cuh:73-103): take the partner-reversed
// second list where strictly larger (its position passing through a float, as
// in the reference), then a bitonic clean-up with no equality guard.
__device__ __forceinline__ void merge_block8(float& p1, uint32_t& pos1, float p2, uint32_t pos2,
                                             int x) {
  const float rp = g8f(p2, 7 - x);
  const float rpos = (float)g8u(pos2, 7 - x);
  if (rp > p1) {
    p1 = rp;
    pos1 = (uint32_t)rpos;
  }
  for (int j = 4; j > 0; j /= 2) {
    const int pr = x ^ j;
    const uint32_t ppos = g8u(pos1, pr);
    const float pp = g8f(p1, pr);
    const bool in_order_pos = x < pr;
    const bool in_order_p = p1 > pp;
    if (in_order_pos != in_order_p) {
      pos1 = ppos;
      p1 = pp;
    }
  }
}

// The replacement of one set by its 8-lane group (this lane: x).  The set's
// cnt candidates come in histogram order: cand(t, &key, &prio) fetches
// candidate t, id(t) names it; the id travels through the networks (as a
// float through MergeBlock, as in the reference) and key_of(id) gives the
// winner's key back.  record(x, write, slot, tag, id) stores lane x's outcome
// (x < min(cnt, 8)); no_record(j) marks the set's record position j >= 8 empty.
template <typename K, typename UK, typename Cand, typename Id, typename KeyOf, typename Record,
          typename NoRecord>
__device__ __forceinline__ void replace_set(const ReplaceLaunch& a, uint32_t set, uint32_t cnt, int x,
                                            Cand cand, Id id, KeyOf key_of, Record record,
                                            NoRecord no_record) {
  const K* tags = static_cast<const K*>(a.tags) + (uint64_t)set * 8;
  float* ctr = a.counters + (uint64_t)set * 8;
  const UK ns = (UK)a.num_sets;
  const K sentinel = (K)a.sentinel;

  // lazy decay of this lane's way counter, then stamp the set current
  float c = ctr[x];
  const int64_t delta = a.global_ts - a.set_ts[set];
  if (delta > 0 && a.decay_rate != 1.0f) {
    const float f = delta < a.decay_len ? a.decay_table[delta]
                                        : (float)pow((double)a.decay_rate, (double)delta);
    c *= f;
  }
  const K my_tag = tags[x];

  float best = 0.0f;
  uint32_t best_pos = 0;
  for (uint32_t done = 0; done == 0 || done < cnt; done += 8) {
    float hp = 0.0f;
    uint32_t hpos = 0;
    uint32_t hit_ways = 0;  // every way holding this candidate's key
    float prio = 0.0f;
    if (done + x < cnt) {
      const uint32_t t = done + (uint32_t)x;
      const uint32_t loc = id(t);
      int64_t k64;
      cand(t, &k64, &prio);
      const K key = (K)k64;
      for (int w = 0; w < 8; ++w) {
        const K tw = tags[w];
        if ((K)((UK)tw * ns + (UK)set) == key) hit_ways |= 1u << w;
      }
      if (hit_ways == 0 && (a.src_rows == 0 || (uint64_t)(int64_t)key < a.src_rows)) {
        hpos = loc;
        hp = prio;
      }
    }
    // a way holds one key, so at most one candidate of the chunk adds to it
    for (int sl = 0; sl < 8; ++sl) {
      const uint32_t hw = g8u(hit_ways, sl);
      const float hpr = g8f(prio, sl);
      if ((hw >> x) & 1u) c += hpr;
    }
    sort_block8(hp, hpos, x);
    if (done == 0) {
      best = hp;
      best_pos = hpos;
    } else {
      merge_block8(best, best_pos, hp, hpos, x);
    }
  }

  // order the ways by counter (an empty way counts 0), reverse to ascending
  float cv = (my_tag == sentinel) ? 0.0f : c;
  uint32_t dpos = (uint32_t)x;
  sort_block8(cv, dpos, x);
  const uint32_t rd = g8u(dpos, 7 - x);
  const float rc = g8f(cv, 7 - x);
  const uint32_t num_repl = cnt < 8 ? cnt : 8;
  const bool write = ((uint32_t)x < num_repl) && (best > rc);
  if ((uint32_t)x < cnt) {
    const int64_t key = write ? key_of(best_pos) : 0;
    record(x, write, (uint64_t)set * 8 + rd, (int64_t)(K)((UK)(K)key / ns), best_pos);  // embed_cache_construct_tag
  }
  for (uint32_t j = 8 + x; j < cnt; j += 8) no_record(j);
  // the replaced way's counter becomes the winner's priority
  for (int sl = 0; sl < 8; ++sl) {
    const int wr = __shfl((int)write, sl, 8);
    const uint32_t wd = g8u(rd, sl);
    const float wb = g8f(best, sl);
    if (wr && wd == (uint32_t)x) c = wb;
  }
  ctr[x] = c;
  if (x == 0) a.set_ts[set] = a.global_ts;
}

// Sorted histogram: set r's candidates are a.order[roff[r] .. roff[r+1]).
// Records at the set's own positions of the order: lane x's at base + x
// (x < num_repl <= cnt), every other position of the set marked empty (a
// counter of records bumped by each replacing wave serialized thousands of
// same-address atomics at the memory side: 70 us per 262,144-key insert).
template <typename K, typename UK>
__global__ __launch_bounds__(256) void set_replace_kernel(ReplaceLaunch a) {
  const int x = threadIdx.x & 7;
  const int64_t r = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 3;
  if (r >= a.num_rsets) return;  // whole 8-lane groups leave together
  const uint32_t set = a.rset[r];
  const uint32_t base = a.roff[r];
  const uint32_t cnt = a.roff[r + 1] - base;
  // a candidate's id is its histogram index
  auto id = [&](uint32_t t) { return a.order[base + t]; };
  auto cand = [&](uint32_t t, int64_t* key, float* prio) {
    const uint32_t loc = a.order[base + t];
    *key = a.hkeys[loc];
    *prio = a.hprio[loc];
  };
  auto key_of = [&](uint32_t loc) { return a.hkeys[loc]; };
  auto record = [&](int lx, bool write, uint64_t slot, int64_t tag, uint32_t loc) {
    const uint32_t pos = base + (uint32_t)lx;
    if (write) {
      a.rec_slot[pos] = slot;
      a.rec_tag[pos] = tag;
      a.rec_src[pos] = a.hsrc[loc];
    } else {
      a.rec_slot[pos] = kNoRecord;
    }
  };
  auto no_record = [&](uint32_t j) { a.rec_slot[base + j] = kNoRecord; };
  replace_set<K, UK>(a, set, cnt, x, cand, id, key_of, record, no_record);
}

// ---------------------------------------------------------------------------
// hashed histogram (large caches: num_sets >= batch size)
//
// The sorted histogram above takes ten radix passes and two readbacks for a
// 262,144-key batch.  Here the batch's unique keys, their counts and first
// positions come from a hash table (a workgroup dedups its 1,024 keys in LDS
// first, so a key is claimed once per workgroup); each unique key is chained
// into its set through a per-set word (candidate count << 32 | chain head),
// which the table keeps clean between inserts; and the replacement of a set
// sorts its few candidates into the histogram's order -- count descending,
// then key ascending in the key's signed order, which is the order the stable
// sorts give -- before running the same per-set replacement.  Positions
// passing through the networks are then the candidates' places in their set,
// so they are exact.  A set with more than kHashSetMax candidates sets the
// overflow word; the replacement then only cleans up and the host falls back
// to the sorted histogram (nothing of the cache has changed).
// ---------------------------------------------------------------------------
namespace {

constexpr uint64_t kHashEmpty = ~0ull;
constexpr int kHashLocalBits = 11;  // 2,048 LDS slots for a workgroup's 1,024 keys

// Fibonacci hash to `bits` bits
__device__ __forceinline__ uint32_t hins_hash(uint64_t k, int bits) {
  return (uint32_t)((k * 0x9E3779B97F4A7C15ull) >> (64 - bits));
}

// Claims k's slot of a linear-probing table of 2^bits 64-bit slots (k is never
// kHashEmpty; the caller guarantees a free slot).  *won: this call put k there.
__device__ __forceinline__ uint32_t hins_claim(uint64_t* tab, uint64_t k, int bits, bool* won) {
  const uint32_t mask = (1u << bits) - 1u;
  uint32_t h = hins_hash(k, bits);
  for (;;) {
    const uint64_t cur = (uint64_t)atomicCAS(reinterpret_cast<unsigned long long*>(tab + h),
                                             (unsigned long long)kHashEmpty, (unsigned long long)k);
    if (cur == kHashEmpty || cur == k) {
      *won = cur == kHashEmpty;
      return h;
    }
    h = (h + 1) & mask;
  }
}

// Appends v to list[base + i] for every thread with app set, one global
// atomic per workgroup (all threads of the workgroup call it).
__device__ __forceinline__ void wg_append(bool app, uint32_t v, uint32_t* counter, uint32_t* list,
                                          uint32_t* s_wave, uint32_t* s_base) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nwaves = (int)(blockDim.x + 63) >> 6;
  const uint64_t bal = __ballot(app);
  const uint32_t below = (uint32_t)__popcll(bal & (lane == 0 ? 0ull : (~0ull >> (64 - lane))));
  if (lane == 0) s_wave[wave] = (uint32_t)__popcll(bal);
  __syncthreads();
  if (tid == 0) {
    uint32_t run = 0;
    for (int w = 0; w < nwaves; ++w) {
      const uint32_t c = s_wave[w];
      s_wave[w] = run;
      run += c;
    }
    *s_base = run ? atomicAdd(counter, run) : 0u;
  }
  __syncthreads();
  if (app) list[*s_base + s_wave[wave] + below] = v;
}

}  // namespace

// The hash table emptied, the counts zeroed and every record position marked
// empty (2^bits + 1 > n threads).
__global__ __launch_bounds__(256) void hins_clear_kernel(HashInsertLaunch a, uint64_t* rec_slot) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t slots = (1ll << a.bits) + 1;
  if (i < slots) {
    a.tkey[i] = kHashEmpty;
    a.tcount[i] = 0u;
    a.tfirst[i] = 0xffffffffu;
  }
  if (i < a.n) rec_slot[i] = kNoRecord;
  if (i < 4) a.counts[i] = 0u;
}

// Counts and first positions of the batch's unique keys; the slots of the
// unique keys listed in ulist[0 .. counts[0]).  Keys are held as 64-bit words
// (32-bit keys zero-extended); the word kHashEmpty (a 64-bit key of -1) uses
// the extra slot 2^bits.
__global__ __launch_bounds__(1024) void hins_count_kernel(HashInsertLaunch a) {
  __shared__ uint64_t lkey[1 << kHashLocalBits];
  __shared__ uint32_t lcnt[1 << kHashLocalBits];
  __shared__ uint32_t lfirst[1 << kHashLocalBits];
  __shared__ uint32_t s_wave[16];
  __shared__ uint32_t s_base;
  const int tid = threadIdx.x;
  const int64_t i = (int64_t)blockIdx.x * 1024 + tid;
  const uint32_t special = 1u << a.bits;
  const bool in = i < a.n;
  uint64_t k = 0;
  if (in)
    k = a.key_bytes == 4 ? (uint64_t)(uint32_t) reinterpret_cast<const int32_t*>(a.keys)[i]
                         : (uint64_t) reinterpret_cast<const int64_t*>(a.keys)[i];
  for (int j = tid; j < (1 << kHashLocalBits); j += 1024) {
    lkey[j] = kHashEmpty;
    lcnt[j] = 0u;
    lfirst[j] = 0xffffffffu;
  }
  __syncthreads();
  uint32_t ls = 0;
  bool first = false, won = false;
  if (in && k != kHashEmpty) {
    // the workgroup's own table: one entry per distinct key, its count and first position
    const uint32_t mask = (1u << kHashLocalBits) - 1u;
    uint32_t h = hins_hash(k, kHashLocalBits);
    for (;;) {
      const uint64_t cur = (uint64_t)atomicCAS(reinterpret_cast<unsigned long long*>(lkey + h),
                                               (unsigned long long)kHashEmpty, (unsigned long long)k);
      if (cur == kHashEmpty || cur == k) {
        first = cur == kHashEmpty;
        break;
      }
      h = (h + 1) & mask;
    }
    ls = h;
    atomicAdd(&lcnt[ls], 1u);
    atomicMin(&lfirst[ls], (uint32_t)i);
  } else if (in) {  // the key word kHashEmpty: its own slot
    atomicAdd(&a.tcount[special], 1u);
    if (!a.by_key) atomicMin(&a.tfirst[special], (uint32_t)i);
    won = atomicCAS(reinterpret_cast<unsigned long long*>(a.tkey + special), (unsigned long long)kHashEmpty,
                    0ull) == (unsigned long long)kHashEmpty;
  }
  __syncthreads();
  uint32_t gs = special;
  if (first) {
    gs = hins_claim(a.tkey, k, a.bits, &won);
    atomicAdd(&a.tcount[gs], lcnt[ls]);
    // the first position names the source row only for rows given with the keys
    if (!a.by_key) atomicMin(&a.tfirst[gs], lfirst[ls]);
  }
  wg_append(won, gs, &a.counts[0], a.ulist, s_wave, &s_base);
}

// The signed histogram key of a unique key's slot (the extra slot: key -1).
__device__ __forceinline__ int64_t hins_key(const HashInsertLaunch& a, uint32_t gs) {
  if (gs == (1u << a.bits)) return -1;
  const uint64_t w = a.tkey[gs];
  return a.key_bytes == 4 ? (int64_t)(int32_t)(uint32_t)w : (int64_t)w;
}

// Chains each unique key u < counts[0] into its set; the first key of a set
// lists the set in rsets[0 .. counts[1]); a set past kHashSetMax candidates
// sets counts[2].
__global__ __launch_bounds__(256) void hins_chain_kernel(HashInsertLaunch a) {
  __shared__ uint32_t s_wave[4];
  __shared__ uint32_t s_base;
  const int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint32_t nu = a.counts[0];
  bool first_of_set = false;
  uint32_t set = 0;
  if (u < nu) {
    const int64_t key = hins_key(a, a.ulist[u]);
    set = a.key_bytes == 4 ? (uint32_t)((uint32_t)(int32_t)key % (uint32_t)a.num_sets)
                           : (uint32_t)((uint64_t)key % a.num_sets);
    unsigned long long* w = reinterpret_cast<unsigned long long*>(a.set_word + set);
    unsigned long long old = *w;
    for (;;) {
      const unsigned long long nw = ((unsigned long long)((uint32_t)(old >> 32) + 1u) << 32) | (uint32_t)u;
      const unsigned long long seen = atomicCAS(w, old, nw);
      if (seen == old) break;
      old = seen;
    }
    a.unext[u] = (uint32_t)old;  // the previous head (0xffffffff: none)
    const uint32_t before = (uint32_t)(old >> 32);
    first_of_set = before == 0;
    if (before + 1 > (uint32_t)kHashSetMax) a.counts[2] = 1u;
  }
  wg_append(first_of_set, set, &a.counts[1], a.rsets, s_wave, &s_base);
}

// One 8-lane group per touched set (grid-stride): the set's candidates from
// its chain into LDS, sorted into histogram order, then replace_set.  Records
// go to the candidates' unique indices (rec_* [0, counts[0])).  Every set's
// word is cleaned.  On overflow nothing is replaced: every record is marked
// empty and the words are cleaned.
template <typename K, typename UK>
__global__ __launch_bounds__(256) void hins_replace_kernel(HashInsertLaunch h, ReplaceLaunch a) {
  constexpr int kGroups = 256 / 8;
  __shared__ int64_t s_key[kGroups][kHashSetMax];
  __shared__ uint32_t s_cnt[kGroups][kHashSetMax];
  __shared__ uint32_t s_first[kGroups][kHashSetMax];
  __shared__ uint32_t s_u[kGroups][kHashSetMax];
  __shared__ uint32_t s_ord[kGroups][kHashSetMax];
  __shared__ uint32_t s_n[kGroups];
  const int x = threadIdx.x & 7;
  const int g = threadIdx.x >> 3;
  const int64_t group = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 3;
  const int64_t groups = ((int64_t)gridDim.x * blockDim.x) >> 3;
  const uint32_t nu = h.counts[0];
  const uint32_t nrs = h.counts[1];
  if (h.counts[2] != 0u) {  // overflow: clean up only (uniform)
    for (int64_t u = group * 8 + x; u < nu; u += groups * 8) a.rec_slot[u] = kNoRecord;
    for (int64_t r = group * 8 + x; r < nrs; r += groups * 8) h.set_word[h.rsets[r]] = kSetClean;
    return;
  }
  const float norm = h.norm;
  for (int64_t r = group; r < nrs; r += groups) {  // uniform over the 8-lane group
    const uint32_t set = h.rsets[r];
    const uint64_t word = h.set_word[set];
    if (x == 0) {
      // the chain, at most kHashSetMax long (no overflow) and inside [0, nu)
      const uint32_t want = (uint32_t)(word >> 32);
      uint32_t u = (uint32_t)word, j = 0;
      while (j < want && j < (uint32_t)kHashSetMax && u < nu) {
        s_u[g][j++] = u;
        u = h.unext[u];
      }
      s_n[g] = j;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const uint32_t cnt = s_n[g];
    for (uint32_t j = (uint32_t)x; j < cnt; j += 8) {
      const uint32_t gs = h.ulist[s_u[g][j]];
      s_key[g][j] = hins_key(h, gs);
      s_cnt[g][j] = h.tcount[gs];
      s_first[g][j] = h.tfirst[gs];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // histogram order: count descending, then key ascending (the key's signed order)
    for (uint32_t j = (uint32_t)x; j < cnt; j += 8) {
      const uint32_t cj = s_cnt[g][j];
      const int64_t kj = s_key[g][j];
      uint32_t rank = 0;
      for (uint32_t i = 0; i < cnt; ++i) {
        const uint32_t ci = s_cnt[g][i];
        rank += (ci > cj || (ci == cj && s_key[g][i] < kj)) ? 1u : 0u;
      }
      s_ord[g][rank] = j;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    auto id = [&](uint32_t t) { return t; };
    auto cand = [&](uint32_t t, int64_t* key, float* prio) {
      const uint32_t j = s_ord[g][t];
      *key = s_key[g][j];
      *prio = (float)(int32_t)s_cnt[g][j] * norm;
    };
    auto key_of = [&](uint32_t t) { return s_key[g][s_ord[g][t]]; };
    auto record = [&](int lx, bool write, uint64_t slot, int64_t tag, uint32_t t) {
      const uint32_t pos = s_u[g][lx];
      if (write) {
        const uint32_t j = s_ord[g][t];
        const int64_t idx = h.by_key ? s_key[g][j] : (int64_t)s_first[g][j];
        a.rec_slot[pos] = slot;
        a.rec_tag[pos] = tag;
        a.rec_src[pos] = (uint64_t)h.rows_base + (uint64_t)idx * (uint64_t)h.row_stride;
      } else {
        a.rec_slot[pos] = kNoRecord;
      }
    };
    auto no_record = [&](uint32_t j) { a.rec_slot[s_u[g][j]] = kNoRecord; };
    replace_set<K, UK>(a, set, cnt, x, cand, id, key_of, record, no_record);
    if (x == 0) h.set_word[set] = kSetClean;
    // the group's LDS is rewritten for its next set
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
}

// ---------------------------------------------------------------------------
// protocol kernels over the replacement records
// ---------------------------------------------------------------------------
template <typename K>
__global__ __launch_bounds__(256) void invalidate_kernel(const uint32_t* num, uint32_t max_records,
                                                         const uint64_t* slot, K* tags, K sentinel) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  const uint32_t n = num != nullptr && *num < max_records ? *num : max_records;
  if (i < n && slot[i] != kNoRecord) tags[slot[i]] = sentinel;
}

template <typename K>
__global__ __launch_bounds__(256) void commit_kernel(const uint32_t* num, uint32_t max_records,
                                                     const uint64_t* slot, const int64_t* tag,
                                                     K* tags) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  const uint32_t n = num != nullptr && *num < max_records ? *num : max_records;
  if (i < n && slot[i] != kNoRecord) tags[slot[i]] = (K)tag[i];
}

// one wave per record: 16-byte (or 4 / 1 byte) chunks of the row
template <int VB>
__global__ __launch_bounds__(256) void copy_rows_kernel(const uint32_t* num, uint32_t max_records,
                                                        const uint64_t* slot, const uint64_t* src,
                                                        uint8_t* data, uint64_t row_bytes) {
  const int lane = threadIdx.x & 63;
  const uint32_t n = num != nullptr && *num < max_records ? *num : max_records;
  const int64_t waves = ((int64_t)gridDim.x * blockDim.x) >> 6;
  for (int64_t rec = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6; rec < n; rec += waves) {
    if (slot[rec] == kNoRecord) continue;
    const uint8_t* s = reinterpret_cast<const uint8_t*>(src[rec]);
    uint8_t* d = data + slot[rec] * row_bytes;
    for (uint64_t o = (uint64_t)lane * VB; o < row_bytes; o += 64 * VB)
      store_vec<VB>(d + o, load_vec<VB>(s + o));
  }
}

// ---------------------------------------------------------------------------
hipError_t launch_hist_prep(const void* keys, int key_bytes, int64_t n, uint64_t* k64, uint32_t* v,
                            hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(hist_prep_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, keys, key_bytes,
                     n, k64, v);
  return hipGetLastError();
}

hipError_t launch_run_heads(const uint64_t* ks, int64_t n, uint32_t* heads, hipStream_t stream,
                            const uint64_t* span_part, int64_t nparts, unsigned long long* span_out) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(run_heads_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, ks, n, heads,
                     span_part, nparts, span_out);
  return hipGetLastError();
}

hipError_t launch_run_gather(const uint64_t* ks, const uint32_t* vs, const uint32_t* scan, int64_t n,
                             uint32_t* start, uint64_t* ukey, uint32_t* first, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(run_gather_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, ks, vs, scan, n,
                     start, ukey, first);
  return hipGetLastError();
}

hipError_t launch_count_key(const uint32_t* start, uint32_t u_n, uint64_t* k2, uint32_t* v2,
                            hipStream_t stream) {
  if (u_n == 0) return hipSuccess;
  hipLaunchKernelGGL(count_key_kernel, dim3((u_n + 255) / 256), dim3(256), 0, stream, start, u_n, k2,
                     v2);
  return hipGetLastError();
}

hipError_t launch_hist_gather(const uint32_t* order, const uint32_t* start, const uint64_t* ukey,
                              const uint32_t* first, uint32_t m, int key_bytes, float norm,
                              const uint8_t* rows_base, int64_t row_stride, int by_key,
                              uint64_t num_sets, int64_t* hkeys, float* hprio, uint64_t* hsrc,
                              uint64_t* k3, uint32_t* v3, hipStream_t stream) {
  if (m == 0) return hipSuccess;
  hipLaunchKernelGGL(hist_gather_kernel, dim3((m + 255) / 256), dim3(256), 0, stream, order, start,
                     ukey, first, m, key_bytes, norm, rows_base, row_stride, by_key, num_sets, hkeys,
                     hprio, hsrc, k3, v3);
  return hipGetLastError();
}

hipError_t launch_set_gather(const uint64_t* ks, const uint32_t* scan, int64_t m, uint32_t* rset,
                             uint32_t* roff, hipStream_t stream) {
  if (m <= 0) return hipSuccess;
  hipLaunchKernelGGL(set_gather_kernel, dim3((m + 255) / 256), dim3(256), 0, stream, ks, scan, m, rset,
                     roff);
  return hipGetLastError();
}

hipError_t launch_set_replace(const ReplaceLaunch& a, int key_bytes, hipStream_t stream) {
  if (a.num_rsets <= 0) return hipSuccess;
  const int64_t threads = a.num_rsets * 8;
  const int64_t grid = (threads + 255) / 256;
  if (key_bytes == 4)
    hipLaunchKernelGGL((set_replace_kernel<int32_t, uint32_t>), dim3(grid), dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL((set_replace_kernel<int64_t, uint64_t>), dim3(grid), dim3(256), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_invalidate(const uint32_t* num, uint32_t max_records, const uint64_t* slot,
                             void* tags, int key_bytes, int64_t sentinel, hipStream_t stream) {
  if (max_records == 0) return hipSuccess;
  const dim3 grid((max_records + 255) / 256);
  if (key_bytes == 4)
    hipLaunchKernelGGL(invalidate_kernel<int32_t>, grid, dim3(256), 0, stream, num, max_records, slot,
                       (int32_t*)tags, (int32_t)sentinel);
  else
    hipLaunchKernelGGL(invalidate_kernel<int64_t>, grid, dim3(256), 0, stream, num, max_records, slot,
                       (int64_t*)tags, (int64_t)sentinel);
  return hipGetLastError();
}

hipError_t launch_commit(const uint32_t* num, uint32_t max_records, const uint64_t* slot,
                         const int64_t* tag, void* tags, int key_bytes, hipStream_t stream) {
  if (max_records == 0) return hipSuccess;
  const dim3 grid((max_records + 255) / 256);
  if (key_bytes == 4)
    hipLaunchKernelGGL(commit_kernel<int32_t>, grid, dim3(256), 0, stream, num, max_records, slot, tag,
                       (int32_t*)tags);
  else
    hipLaunchKernelGGL(commit_kernel<int64_t>, grid, dim3(256), 0, stream, num, max_records, slot, tag,
                       (int64_t*)tags);
  return hipGetLastError();
}

hipError_t launch_copy_rows(const uint32_t* num, uint32_t max_records, const uint64_t* slot,
                            const uint64_t* src, int src_align, uint8_t* data, uint64_t row_bytes,
                            hipStream_t stream) {
  if (max_records == 0) return hipSuccess;
  // one wave per record, at most 8,192 workgroups (a record count known only
  // on the device leaves most of an upper-bound grid idle)
  const dim3 grid((unsigned)std::min<uint64_t>(((uint64_t)max_records * 64 + 255) / 256, 8192));
  const bool d16 = ((uintptr_t)data % 16 == 0) && row_bytes % 16 == 0;
  if (d16 && src_align % 16 == 0)
    hipLaunchKernelGGL(copy_rows_kernel<16>, grid, dim3(256), 0, stream, num, max_records, slot, src,
                       data, row_bytes);
  else if (row_bytes % 4 == 0 && (uintptr_t)data % 4 == 0 && src_align % 4 == 0)
    hipLaunchKernelGGL(copy_rows_kernel<4>, grid, dim3(256), 0, stream, num, max_records, slot, src,
                       data, row_bytes);
  else
    hipLaunchKernelGGL(copy_rows_kernel<1>, grid, dim3(256), 0, stream, num, max_records, slot, src,
                       data, row_bytes);
  return hipGetLastError();
}

hipError_t launch_hash_insert(const HashInsertLaunch& h, const ReplaceLaunch& r, hipStream_t stream) {
  if (h.n <= 0) return hipSuccess;
  if (h.bits < 10 || h.bits > 30 || (1ll << h.bits) < 2 * h.n || h.n > 0xffffffffll) return hipErrorInvalidValue;
  const int64_t slots = (1ll << h.bits) + 1;
  hipLaunchKernelGGL(hins_clear_kernel, dim3((unsigned)((slots + 255) / 256)), dim3(256), 0, stream, h,
                     r.rec_slot);
  hipLaunchKernelGGL(hins_count_kernel, dim3((unsigned)((h.n + 1023) / 1024)), dim3(1024), 0, stream, h);
  hipLaunchKernelGGL(hins_chain_kernel, dim3((unsigned)((h.n + 255) / 256)), dim3(256), 0, stream, h);
  const unsigned rgrid = (unsigned)std::min<int64_t>((h.n * 8 + 255) / 256, 2048);
  if (h.key_bytes == 4)
    hipLaunchKernelGGL((hins_replace_kernel<int32_t, uint32_t>), dim3(rgrid), dim3(256), 0, stream, h, r);
  else
    hipLaunchKernelGGL((hins_replace_kernel<int64_t, uint64_t>), dim3(rgrid), dim3(256), 0, stream, h, r);
  return hipGetLastError();
}

}  // namespace nve_amd
