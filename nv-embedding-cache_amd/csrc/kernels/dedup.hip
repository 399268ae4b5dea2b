// dedup.hip -- key deduplication on the GPU (Deduper::dedup, deduper.cuh:136-221)
// and the dedup-then-gather.
//
// dedup: stable radix sort of (key, position) -> runs of equal keys -> per
// run: unique key, start offset, count; per position: inverse = original
// position in key order.  The runs take two launches (per-block head counts,
// then every output with the blocks before as carry-in) up to kRunMaxBlocks
// blocks, else run heads -> exclusive scan -> outputs -> counts.  Outputs
// match the reference's: unique keys ascending (signed order), counts, the
// stable inverse map and exclusive offsets.
//
// dedup-then-gather needs no order, so it dedups by hashing instead of
// sorting (three launches instead of eleven): every distinct key of a
// workgroup claims a slot of an open-addressed table (linear probing, at most
// half full) with one compare-and-swap, the winner becoming the key's owner
// and its workgroup copying the key's table row to the owner's output row at
// once (each distinct row read once); with 32-bit keys a slot holds key and
// owner, so every claimant learns the owner at once; then every other
// position copies its owner's output row (UnpackDedup, cuda_utils.cuh:24-79).
#include "device_common.cuh"
#include "dedup_launch.hpp"
#include "position_grad.cuh"
#include "sort_launch.hpp"

namespace nve_amd {

// OR of x over the 256 threads of the workgroup, in every thread (all threads call it)
__device__ __forceinline__ uint64_t block_or(uint64_t x) {
  __shared__ uint64_t red[4];
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x |= __shfl_xor(x, o);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
  __syncthreads();
  return red[0] | red[1] | red[2] | red[3];
}

__global__ __launch_bounds__(256) void dedup_prep_kernel(const void* keys, int key_bytes, int64_t n,
                                                         int flip, uint64_t* k64, uint32_t* v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    const int64_t k = load_key(keys, key_bytes, i);
    k64[i] = flip ? flip_key(k, key_bytes) : (uint64_t)k;
    v[i] = (uint32_t)i;
  }
}

// inverse[i] = position of the i-th key in key order; at a run head:
// unique[u] = key, offsets[u] = i (= start[u]); start[U] = n.
// span_part (optional, nparts words): workgroup 0 also ORs the prep's span
// parts into *span_out.
__global__ __launch_bounds__(256) void dedup_outputs_kernel(const uint64_t* ks, const uint32_t* vs,
                                                            const uint32_t* scan, int64_t n,
                                                            int key_bytes, void* unique,
                                                            void* inverse, void* offsets,
                                                            uint32_t* start, uint32_t* pos_key,
                                                            const uint64_t* span_part, int64_t nparts,
                                                            unsigned long long* span_out) {
  if (span_part != nullptr && blockIdx.x == 0) {  // uniform over the workgroup
    uint64_t a = 0;
    for (int64_t j = threadIdx.x; j < nparts; j += blockDim.x) a |= span_part[j];
    a = block_or(a);
    if (threadIdx.x == 0) *span_out = a;
  }
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  store_key(inverse, key_bytes, i, (int64_t)vs[i]);
  const bool head = (i == 0 || ks[i] != ks[i - 1]);
  if (pos_key != nullptr) pos_key[i] = head ? scan[i] : scan[i] - 1u;  // unique index of position i
  if (head) {
    const uint32_t u = scan[i];
    store_key(unique, key_bytes, u, unflip_key(ks[i], key_bytes));
    store_key(offsets, key_bytes, u, i);
    start[u] = (uint32_t)i;
  }
  if (i == n - 1) start[scan[i] + (head ? 1u : 0u)] = (uint32_t)n;
}

// u_dev (optional): the unique count in device memory, for a grid sized by an
// upper bound without reading the count back first.
__global__ __launch_bounds__(256) void dedup_counts_kernel(const uint32_t* start, uint32_t u_n,
                                                           const uint32_t* u_dev, int key_bytes,
                                                           void* counts) {
  const uint32_t u = blockIdx.x * blockDim.x + threadIdx.x;
  const uint32_t m = u_dev != nullptr ? *u_dev : u_n;
  if (u < m) store_key(counts, key_bytes, u, (int64_t)(start[u + 1] - start[u]));
}

// ---------------------------------------------------------------------------
// runs of the sorted keys in two launches (batches of up to kRunMaxBlocks
// blocks of kRunBlock keys): run_block_kernel counts each block's run heads
// and notes its last head; run_outputs_kernel takes the sums and maxima of
// the blocks before its own as carry-in (so no scan launch sits between), and
// writes every output of the dedup: per position its inverse entry and unique
// index, per run its key and offset at the head and its count at the tail.
// ---------------------------------------------------------------------------
constexpr int kRunThreads = 256;
constexpr int kRunItems = 4;
constexpr int kRunBlock = kRunThreads * kRunItems;

// Block-wide exclusive sum of c and exclusive maximum of l over thread order
// (every thread calls it); *sum = the block's total of c.
__device__ __forceinline__ void block_scan_sum_max(uint32_t c, int64_t l, uint32_t* ex_c, int64_t* ex_l,
                                                   uint32_t* sum) {
  __shared__ uint32_t wc[kRunThreads / 64];
  __shared__ int64_t wl[kRunThreads / 64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  uint32_t ic = c;  // inclusive within the wave
  int64_t il = l;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t pc = __shfl_up(ic, o);
    const int64_t pl = __shfl_up(il, o);
    if (lane >= o) {
      ic += pc;
      il = pl > il ? pl : il;
    }
  }
  if (lane == 63) {
    wc[wave] = ic;
    wl[wave] = il;
  }
  __syncthreads();
  uint32_t bc = 0;
  int64_t bl = -1;
  for (int w = 0; w < wave; ++w) {
    bc += wc[w];
    bl = wl[w] > bl ? wl[w] : bl;
  }
  uint32_t tot = 0;
  for (int w = 0; w < kRunThreads / 64; ++w) tot += wc[w];
  // exclusive: inclusive minus own, maximum of the lanes before
  const int64_t prev_l = __shfl_up(il, 1);
  *ex_c = bc + ic - c;
  const int64_t lane_l = lane > 0 ? prev_l : -1;
  *ex_l = lane_l > bl ? lane_l : bl;
  *sum = tot;
}

// blk_count[b] = run heads in block b, blk_last[b] = its last head position (-1: none)
__global__ __launch_bounds__(kRunThreads) void run_block_kernel(const uint64_t* ks, int64_t n,
                                                                uint32_t* blk_count, int64_t* blk_last) {
  const int64_t base = (int64_t)blockIdx.x * kRunBlock;
  uint32_t c = 0;
  int64_t l = -1;
#pragma unroll 4
  for (int j = 0; j < kRunItems; ++j) {
    const int64_t i = base + (int64_t)j * kRunThreads + threadIdx.x;  // coalesced
    if (i < n && (i == 0 || ks[i] != ks[i - 1])) {
      ++c;
      l = i;
    }
  }
  uint32_t ex_c, sum;
  int64_t ex_l;
  block_scan_sum_max(c, l, &ex_c, &ex_l, &sum);
  // the block's last head: the maximum over all threads
  __shared__ int64_t last;
  if (threadIdx.x == kRunThreads - 1) last = l > ex_l ? l : ex_l;
  __syncthreads();
  if (threadIdx.x == 0) {
    blk_count[blockIdx.x] = sum;
    blk_last[blockIdx.x] = last;
  }
}

struct RunOutputs {
  const uint64_t* ks;
  const uint32_t* vs;
  int64_t n;
  const uint32_t* blk_count;
  const int64_t* blk_last;
  int key_bytes;
  void* unique;
  void* counts;
  void* inverse;
  void* offsets;
  uint32_t* pos_key;   // optional
  uint32_t* total;     // the unique count, written by the last block
  const uint64_t* span_part;  // optional: block 0 ORs these into *span_out
  int64_t nparts;
  unsigned long long* span_out;
  PositionGrad pg;            // pg.rows non-null: each position's gradient row and weight too
};

__global__ __launch_bounds__(kRunThreads) void run_outputs_kernel(RunOutputs a) {
  if (a.span_part != nullptr && blockIdx.x == 0) {  // uniform over the workgroup
    uint64_t x = 0;
    for (int64_t j = threadIdx.x; j < a.nparts; j += blockDim.x) x |= a.span_part[j];
    x = block_or(x);
    if (threadIdx.x == 0) *a.span_out = x;
  }
  // carry-in: heads before this block, and the last head before it
  uint32_t u0;
  int64_t h0;
  {
    __shared__ uint32_t in_c[kRunThreads / 64];
    __shared__ int64_t in_l[kRunThreads / 64];
    uint32_t c = 0;
    int64_t l = -1;
    for (uint32_t b = threadIdx.x; b < blockIdx.x; b += blockDim.x) {
      c += a.blk_count[b];
      l = a.blk_last[b] > l ? a.blk_last[b] : l;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      c += __shfl_xor(c, o);
      const int64_t p = __shfl_xor(l, o);
      l = p > l ? p : l;
    }
    if ((threadIdx.x & 63) == 0) {
      in_c[threadIdx.x >> 6] = c;
      in_l[threadIdx.x >> 6] = l;
    }
    __syncthreads();
    u0 = 0;
    h0 = -1;
#pragma unroll
    for (int w = 0; w < kRunThreads / 64; ++w) {
      u0 += in_c[w];
      h0 = in_l[w] > h0 ? in_l[w] : h0;
    }
  }

  // this thread's kRunItems consecutive positions
  const int64_t first = (int64_t)blockIdx.x * kRunBlock + (int64_t)threadIdx.x * kRunItems;
  uint64_t k[kRunItems];
#pragma unroll
  for (int j = 0; j < kRunItems; ++j) k[j] = first + j < a.n ? a.ks[first + j] : 0;
  const uint64_t before = first > 0 && first - 1 < a.n ? a.ks[first - 1] : 0;
  const uint64_t after = first + kRunItems < a.n ? a.ks[first + kRunItems] : 0;
  uint32_t c = 0;
  int64_t l = -1;
#pragma unroll
  for (int j = 0; j < kRunItems; ++j) {
    const int64_t i = first + j;
    const bool head = i < a.n && (i == 0 || k[j] != (j ? k[j - 1] : before));
    if (head) {
      ++c;
      l = i;
    }
  }
  uint32_t ex_c, sum;
  int64_t ex_l;
  block_scan_sum_max(c, l, &ex_c, &ex_l, &sum);
  if (blockIdx.x == gridDim.x - 1 && threadIdx.x == 0) *a.total = u0 + sum;

  // the run in progress at this thread's first position
  uint32_t u = u0 + ex_c - 1u;  // wraps for position 0, which is a head
  int64_t start = ex_l > h0 ? ex_l : h0;
#pragma unroll
  for (int j = 0; j < kRunItems; ++j) {
    const int64_t i = first + j;
    if (i >= a.n) break;
    const bool head = i == 0 || k[j] != (j ? k[j - 1] : before);
    if (head) {
      ++u;
      start = i;
      store_key(a.unique, a.key_bytes, u, unflip_key(k[j], a.key_bytes));
      store_key(a.offsets, a.key_bytes, u, i);
    }
    const uint32_t pos = a.vs[i];
    store_key(a.inverse, a.key_bytes, i, (int64_t)pos);
    if (a.pos_key != nullptr) a.pos_key[i] = u;
    if (a.pg.rows != nullptr) position_grad(a.pg, i, (int64_t)pos);
    const bool tail = i == a.n - 1 || k[j] != (j + 1 < kRunItems ? k[j + 1] : after);
    if (tail) store_key(a.counts, a.key_bytes, u, i + 1 - start);
  }
}

// ---------------------------------------------------------------------------
// hash dedup for the gather
// ---------------------------------------------------------------------------
constexpr uint32_t kNoSlot = 0xffffffffu;

// Table keys are 32-bit when every row index fits (num_rows < 2^32), else
// 64-bit; all ones marks an empty slot (no row index has that value).
template <typename KT>
constexpr KT empty_slot() {
  return (KT)~(KT)0;
}

// the table's keys to empty
template <typename KT>
__global__ __launch_bounds__(256) void hash_clear_kernel(KT* tab, int64_t slots) {
  constexpr int64_t per = 16 / sizeof(KT);  // slots per 16-byte store
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if ((i + 1) * per <= slots) {
    u32x4 e{0xffffffffu, 0xffffffffu, 0xffffffffu, 0xffffffffu};
    reinterpret_cast<u32x4*>(tab)[i] = e;
  } else {
    for (int64_t j = i * per; j < slots; ++j) tab[j] = empty_slot<KT>();
  }
}

// Multiplicative (Fibonacci) hash to `bits` bits.
__device__ __forceinline__ uint32_t slot_hash(uint64_t k, int bits) {
  return (uint32_t)((k * 0x9E3779B97F4A7C15ull) >> (64 - bits));
}

__device__ __forceinline__ uint32_t cas(uint32_t* p, uint32_t expect, uint32_t v) {
  return atomicCAS(p, expect, v);
}
__device__ __forceinline__ uint64_t cas(uint64_t* p, uint64_t expect, uint64_t v) {
  return (uint64_t)atomicCAS(reinterpret_cast<unsigned long long*>(p), (unsigned long long)expect,
                             (unsigned long long)v);
}

// Claim key k's slot of a table of 2^bits slots (linear probing; the caller
// guarantees a free slot).  Returns the slot; *won: this call put k there.
// A slot only changes from empty to a key, so the compare-and-swap's answer
// is final.
template <typename KT>
__device__ __forceinline__ uint32_t claim(KT* tab, KT k, int bits, bool* won) {
  const uint32_t mask = (1u << bits) - 1u;
  uint32_t h = slot_hash(k, bits);
  for (;;) {
    const KT cur = cas(tab + h, empty_slot<KT>(), k);
    if (cur == empty_slot<KT>() || cur == k) {
      *won = cur == empty_slot<KT>();
      return h;
    }
    h = (h + 1) & mask;
  }
}

struct HashClaim {
  const void* keys;
  int key_bytes;
  int64_t n;
  uint64_t num_rows;
  void* tab;
  int bits;
  uint32_t* owner;    // owner[slot]: position that owns the slot's key
  uint32_t* slot_of;  // slot_of[i]: slot of position i's key (kNoSlot: out of range)
  const uint8_t* table;
  uint64_t row_bytes;
  uint8_t* out;
  int64_t out_stride;
  int g_shift;  // 2^g_shift lanes move one row
  int passes;   // row pieces of 2^g_shift * VB bytes
};

// Claim 32-bit key k for position pos in a table of 2^bits 64-bit slots
// holding key << 32 | owner position (all ones: empty), so that a loser of
// the compare-and-swap learns the owner from its answer.  Returns the owner;
// *won: pos became it.
__device__ __forceinline__ uint32_t claim_owner(uint64_t* tab, uint32_t k, uint32_t pos, int bits,
                                                bool* won) {
  const uint32_t mask = (1u << bits) - 1u;
  const uint64_t mine = ((uint64_t)k << 32) | pos;
  uint32_t h = slot_hash(k, bits);
  for (;;) {
    const uint64_t cur = cas(tab + h, ~0ull, mine);
    if (cur == ~0ull) {
      *won = true;
      return pos;
    }
    if ((uint32_t)(cur >> 32) == k) {
      *won = false;
      return (uint32_t)cur;
    }
    h = (h + 1) & mask;
  }
}

constexpr int kClaimThreads = 1024;  // one key per thread
constexpr int kLocalBits = 11;       // 2048 LDS slots per workgroup, at most half full

// The claims and the owners' copies in one launch.  Each workgroup first
// dedups its 1024 keys in an LDS table, so a key claims its global slot once
// per workgroup rather than once per occurrence (device-scope
// compare-and-swaps on one hot key's slot serialize at the memory side).  The
// global winner of a slot owns the key: it records itself in owner[slot], and
// its workgroup then copies the key's table row to the owner's output row --
// each distinct row is read once.  Rows move as in the plain gather:
// 2^g_shift lanes per row, U rows in flight per lane group, every load of a
// round issued before any store.  Measured on 262,144 Zipf(1.05) keys, this
// launch and the repeats' take 39 us where separate claim, owner-list and
// owner-copy launches took 48; chunks of 512 or 2048 keys per workgroup were
// slower (41 and 42 us), and so was reading a slot before its
// compare-and-swap (43 us: the workgroups reach the hot keys' slots together).
// Packing key and owner into one slot (32-bit keys) then let the repeats read
// each position's owner directly (39.6 -> 37.5 us), and copying each wave's
// wins without waiting for the other waves' claims gave 36.1 us.
// PACKED (32-bit keys): the table holds key and owner together and slot_of
// receives each position's owner; otherwise the table holds keys, owner[]
// the owner of each slot and slot_of each position's slot.
template <typename KT, int VB, int U, bool PACKED>
__global__ __launch_bounds__(kClaimThreads) void hash_claim_copy_kernel(HashClaim a) {
  static_assert(!PACKED || sizeof(KT) == 4, "packed slots hold 32-bit keys");
  __shared__ KT lkey[1 << kLocalBits];
  __shared__ uint32_t lslot[1 << kLocalBits];  // global slot (PACKED: owner) of the local entry
  __shared__ uint64_t win_row[kClaimThreads];  // each wave's wins (64 entries a wave): table row
  __shared__ uint32_t win_pos[kClaimThreads];  // ... and output row
  const int tid = threadIdx.x;
  // the key load is issued before the LDS table is cleared
  const int64_t i = (int64_t)blockIdx.x * kClaimThreads + tid;
  bool in = false;
  KT k = 0;
  if (i < a.n) {
    const uint64_t k64 = (uint64_t)load_key(a.keys, a.key_bytes, i);
    in = k64 < a.num_rows;  // keys outside the table get no slot and no output row
    k = (KT)k64;
  }
  for (int j = tid; j < (1 << kLocalBits); j += kClaimThreads) lkey[j] = empty_slot<KT>();
  __syncthreads();
  uint32_t ls = 0;
  bool first = false;
  if (in) ls = claim<KT>(lkey, k, kLocalBits, &first);
  __syncthreads();
  bool won = false;
  if (first) {
    if constexpr (PACKED) {
      lslot[ls] = claim_owner(static_cast<uint64_t*>(a.tab), (uint32_t)k, (uint32_t)i, a.bits, &won);
    } else {
      const uint32_t gs = claim<KT>(static_cast<KT*>(a.tab), k, a.bits, &won);
      lslot[ls] = gs;
      if (won) a.owner[gs] = (uint32_t)i;
    }
  }
  // each wave lists the keys it won in its own LDS region and copies their
  // rows at once, without waiting for the other waves' claims
  const uint64_t ballot = __ballot(won);
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const uint32_t below = (uint32_t)__popcll(ballot & (lane == 0 ? 0ull : (~0ull >> (64 - lane))));
  const int nw = (int)__popcll(ballot);
  uint64_t* wrow = win_row + wave * 64;
  uint32_t* wpos = win_pos + wave * 64;
  if (won) {
    wrow[below] = (uint64_t)k;
    wpos[below] = (uint32_t)i;
  }
  // lanes read what other lanes of the wave wrote: LDS keeps a wave's
  // accesses in order; the fences keep the compiler from moving them
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const int G = 1 << a.g_shift;
  const int gl = lane & (G - 1);
  const int grp = lane >> a.g_shift;
  const int groups = 64 >> a.g_shift;
  const uint64_t zero_row = (uint64_t)g_zero_row;
  for (int p = 0; p < a.passes; ++p) {
    const int64_t off = ((int64_t)p * G + gl) * VB;
    const bool in_row = off < (int64_t)a.row_bytes;
    for (int q0 = 0; q0 < nw; q0 += groups * U) {
      uint64_t src[U];
      uint32_t dst[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int q = q0 + u * groups + grp;
        const bool real = q < nw && in_row;
        src[u] = real ? (uint64_t)a.table + wrow[q] * a.row_bytes + off : zero_row + (off & kZeroRowMask);
        dst[u] = real ? wpos[q] : kNoSlot;
      }
      Vec<VB> v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) v[u] = load_vec<VB>(src[u]);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (dst[u] == kNoSlot) continue;
        store_vec<VB, false>(a.out + (int64_t)dst[u] * a.out_stride + off, v[u]);
      }
    }
  }
  __syncthreads();  // every local entry's owner (or slot) is in LDS
  if (i < a.n) a.slot_of[i] = in ? lslot[ls] : kNoSlot;
}

// Every position that does not own its key copies its owner's output row
// (written by the claims' launch).  A wave resolves T positions (one per
// lane), then groups of G lanes move one row each, U rows in flight, VB
// bytes per lane and load.
struct HashRepeat {
  int64_t n;
  uint64_t row_bytes;
  const uint32_t* slot_of;
  const uint32_t* owner;
  uint8_t* out;
  int64_t out_stride;
};

template <int VB, int U, bool PACKED>
__global__ __launch_bounds__(256) void hash_repeat_kernel(HashRepeat a, int g_shift, int t_shift, int passes) {
  const int T = 1 << t_shift;
  const int lane = threadIdx.x & 63;
  const int64_t tile = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int64_t base = tile << t_shift;
  if (base >= a.n) return;  // whole wave past the end
  const int64_t j = base + lane;
  uint64_t src = 0;  // row to copy from, 0: nothing to do for this lane's position
  if (lane < T && j < a.n) {
    const uint32_t sl = a.slot_of[j];
    if (sl != kNoSlot) {
      const uint32_t own = PACKED ? sl : a.owner[sl];
      if (own != (uint32_t)j) src = (uint64_t)a.out + (uint64_t)own * (uint64_t)a.out_stride;
    }
  }
  const uint32_t dst = (uint32_t)j;
  const int G = 1 << g_shift;
  const int gl = lane & (G - 1);
  const int grp = lane >> g_shift;
  const int groups = 64 >> g_shift;
  const int per_group = T >> (6 - g_shift) > 0 ? T >> (6 - g_shift) : 1;
  const uint64_t zero_row = (uint64_t)g_zero_row;
  for (int p = 0; p < passes; ++p) {
    const int64_t off = ((int64_t)p * G + gl) * VB;
    const bool in_row = off < (int64_t)a.row_bytes;
    for (int q0 = 0; q0 < per_group; q0 += U) {
      uint64_t ra[U];
      uint32_t rd[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int q = q0 + u;
        const int from = grp + (q < per_group ? q : 0) * groups;
        ra[u] = shfl64(src, from);
        rd[u] = shfl32(dst, from);
        if (q >= per_group) ra[u] = 0;
      }
      Vec<VB> v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool real = ra[u] != 0;
        v[u] = load_vec<VB>((real ? ra[u] : zero_row) + ((real && in_row) ? off : (off & kZeroRowMask)));
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (ra[u] == 0 || !in_row) continue;
        store_vec<VB>(a.out + (int64_t)rd[u] * a.out_stride + off, v[u]);
      }
    }
  }
}

size_t hash_dedup_slots(int64_t n) {
  size_t s = 1024;
  while (s < 2 * (size_t)n) s <<= 1;
  return s;
}

size_t hash_dedup_key_bytes(int64_t num_rows) { return (uint64_t)num_rows <= 0xffffffffull ? 4 : 8; }

hipError_t launch_hash_dedup_gather(const void* keys, int key_bytes, int64_t n, const uint8_t* table,
                                    int64_t num_rows, int64_t row_bytes, void* out, int64_t out_stride,
                                    void* tab, uint32_t* owner, uint32_t* slot_of, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  const int64_t slots = (int64_t)hash_dedup_slots(n);
  int bits = 0;
  while ((1ll << bits) < slots) ++bits;
  const bool k32 = hash_dedup_key_bytes(num_rows) == 4;
  // widest vector every row, output row and base is aligned to
  int vb = 16;
  while (vb > 1 && (row_bytes % vb || out_stride % vb || (uintptr_t)table % vb || (uintptr_t)out % vb))
    vb >>= 1;
  const int64_t nv = row_bytes / vb;
  int g = 1;
  while (g < nv && g < 64) g <<= 1;
  const int passes = (int)((nv + g - 1) / g);
  int gs = 0;
  while ((1 << gs) < g) ++gs;
  constexpr int U = 8;
  const int tkeys = (64 / g) * U < 64 ? (64 / g) * U : 64;
  int ts = 0;
  while ((1 << ts) < tkeys) ++ts;
  const int64_t waves = (n + tkeys - 1) / tkeys;
  const int64_t grid = (waves * 64 + 255) / 256;
  if (grid > 0x7fffffffLL) return hipErrorInvalidValue;
  const dim3 claim_grid((unsigned)((n + kClaimThreads - 1) / kClaimThreads));
  HashClaim c{keys, key_bytes, n, (uint64_t)num_rows, tab, bits, owner, slot_of, table, (uint64_t)row_bytes,
              static_cast<uint8_t*>(out), out_stride, gs, passes};
  HashRepeat r{n, (uint64_t)row_bytes, slot_of, owner, static_cast<uint8_t*>(out), out_stride};
  // 64-bit slots either way: 32-bit keys packed with their owner, or 64-bit keys
  hipLaunchKernelGGL(hash_clear_kernel<uint64_t>, dim3((slots / 2 + 255) / 256), dim3(256), 0, stream,
                     static_cast<uint64_t*>(tab), slots);
#define HC(V)                                                                                           \
  do {                                                                                                  \
    if (k32) {                                                                                          \
      hipLaunchKernelGGL((hash_claim_copy_kernel<uint32_t, V, U, true>), claim_grid,                    \
                         dim3(kClaimThreads), 0, stream, c);                                            \
      hipLaunchKernelGGL((hash_repeat_kernel<V, U, true>), dim3(grid), dim3(256), 0, stream, r, gs, ts, \
                         passes);                                                                       \
    } else {                                                                                            \
      hipLaunchKernelGGL((hash_claim_copy_kernel<uint64_t, V, U, false>), claim_grid,                   \
                         dim3(kClaimThreads), 0, stream, c);                                            \
      hipLaunchKernelGGL((hash_repeat_kernel<V, U, false>), dim3(grid), dim3(256), 0, stream, r, gs,    \
                         ts, passes);                                                                   \
    }                                                                                                   \
  } while (0)
  switch (vb) {
    case 16: HC(16); break;
    case 8: HC(8); break;
    case 4: HC(4); break;
    case 2: HC(2); break;
    default: HC(1); break;
  }
#undef HC
  return hipGetLastError();
}

int64_t dedup_span_parts(int64_t n) { return radix_tiles(n); }

hipError_t launch_dedup_prep(const void* keys, int key_bytes, int64_t n, int flip, uint64_t* k64,
                             uint32_t* v, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(dedup_prep_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, keys, key_bytes,
                     n, flip, k64, v);
  return hipGetLastError();
}

hipError_t launch_dedup_outputs(const uint64_t* ks, const uint32_t* vs, const uint32_t* scan,
                                int64_t n, int key_bytes, void* unique, void* inverse,
                                void* offsets, uint32_t* start, uint32_t* pos_key,
                                const uint64_t* span_part, unsigned long long* span_out,
                                hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(dedup_outputs_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, ks, vs, scan,
                     n, key_bytes, unique, inverse, offsets, start, pos_key, span_part,
                     dedup_span_parts(n), span_out);
  return hipGetLastError();
}

int64_t run_blocks(int64_t n) { return (n + kRunBlock - 1) / kRunBlock; }

hipError_t launch_dedup_runs(const uint64_t* ks, const uint32_t* vs, int64_t n, int key_bytes, void* unique,
                             void* counts, void* inverse, void* offsets, uint32_t* pos_key, uint32_t* total,
                             uint32_t* blk_count, int64_t* blk_last, const uint64_t* span_part,
                             unsigned long long* span_out, const PositionGrad* pg, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  const int64_t nb = run_blocks(n);
  if (nb > kRunMaxBlocks) return hipErrorInvalidValue;
  hipLaunchKernelGGL(run_block_kernel, dim3(nb), dim3(kRunThreads), 0, stream, ks, n, blk_count, blk_last);
  RunOutputs a{ks, vs, n, blk_count, blk_last, key_bytes, unique, counts, inverse, offsets, pos_key, total,
               span_part, dedup_span_parts(n), span_out, pg != nullptr ? *pg : PositionGrad{}};
  hipLaunchKernelGGL(run_outputs_kernel, dim3(nb), dim3(kRunThreads), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_dedup_counts(const uint32_t* start, uint32_t u_n, const uint32_t* u_dev,
                               int key_bytes, void* counts, hipStream_t stream) {
  if (u_n == 0) return hipSuccess;
  hipLaunchKernelGGL(dedup_counts_kernel, dim3((u_n + 255) / 256), dim3(256), 0, stream, start, u_n,
                     u_dev, key_bytes, counts);
  return hipGetLastError();
}

}  // namespace nve_amd
