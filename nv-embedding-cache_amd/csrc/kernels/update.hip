// update.hip -- row updates of the cache and of linear tables.
//
// Reference behaviour restated:
//   cache update / update_accumulate  SetUpdateDataKernel (ec_set_associative_modify.cuh:516-561),
//       mem_update_kernel / mem_update_accumulate_kernel (ec_set_associative.cuh:157-185),
//       driven by CacheSADeviceModify::update / update_accumulate
//       (ec_set_associative_device_modify.cuh:290-388)
//   linear table  UpdateTableKernel / UpdateAccumulateTableKernel (cuda_ops/update_accumulate.cuh)
//
// The records kernel finds every way holding a key (one lane per key, the
// set's 8 tags compared); the caller invalidates those ways, drains running
// lookups, then copies (launch_copy_rows) or accumulates the rows and
// restores the tags -- the same protocol as an insert.  Accumulation is
// atomic per element: fp32 adds are native atomics, fp16 elements are
// updated by a 32-bit compare-and-swap of the word that holds them, the sum
// computed in fp32 and rounded to nearest even (the exact fp16 sum rounded
// once: two fp16 values add exactly in fp32 unless their exponents differ by
// more than 13, and then the smaller is below a quarter ulp of the larger).
#include "device_common.cuh"
#include "modify_launch.hpp"
#include "update_launch.hpp"

namespace nve_amd {

// The ways whose rebuilt key (tag * num_sets + set, empty ways included, as
// the reference's SetUpdateDataKernel compares them) equals key: bit w.
template <typename K, typename UK>
__device__ __forceinline__ uint32_t matching_ways(const K* tags, UK num_sets, K key, UK* set_out) {
  const UK set = (UK)key % num_sets;
  const K* t = tags + (uint64_t)set * 8;
  uint32_t mask = 0;
#pragma unroll
  for (int w = 0; w < 8; ++w)
    if ((K)((UK)t[w] * num_sets + set) == key) mask |= 1u << w;
  *set_out = set;
  return mask;
}

// The tag a record commits: the key's own tag, key / num_sets in unsigned
// arithmetic (the device policy, SetUpdateDataKernel
// ec_set_associative_modify.cuh:557), or the way's current tag (the host
// policy, ec_set_associative_host_modify.h:503-506).  The two differ only for
// a key equal to the rebuilt key of empty ways: the device policy turns those
// ways into ordinary tags.
template <typename K, typename UK>
__device__ __forceinline__ int64_t record_tag(K key, UK num_sets, K way_tag, bool own_tag) {
  return own_tag ? (int64_t)(K)((UK)key / num_sets) : (int64_t)way_tag;
}

// Record i for key i: its first matching way, or kNoRecord.  A key matching
// more than one way (only one equal to the rebuilt key of empty ways, which
// needs num_sets to divide 2^64 or 2^32) sets *multi, a pinned host word, and
// its further ways are recorded by update_more_records_kernel.  (A counter of
// records bumped by every wave, as all records once took their slots,
// serialized the waves' atomics at the memory side.)
template <typename K, typename UK>
__global__ __launch_bounds__(256) void update_records_kernel(
    const K* keys, int64_t n, const K* tags, UK num_sets, const uint8_t* values,
    int64_t value_stride, uint64_t* rec_slot, int64_t* rec_tag, uint64_t* rec_src, uint32_t* multi,
    bool own_tag) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  UK set;
  const K key = keys[i];
  const uint32_t mask = matching_ways<K, UK>(tags, num_sets, key, &set);
  if (mask == 0) {
    rec_slot[i] = kNoRecord;
    return;
  }
  const int w = __ffs(mask) - 1;
  rec_slot[i] = (uint64_t)set * 8 + (uint64_t)w;
  rec_tag[i] = record_tag<K, UK>(key, num_sets, tags[(uint64_t)set * 8 + w], own_tag);
  rec_src[i] = (uint64_t)values + (uint64_t)i * (uint64_t)value_stride;
  if (mask & (mask - 1)) *multi = 1u;
}

// The further matching ways of every key: records [0, *count) (count zeroed
// by the caller), at most cap.  Device policy only (the host policy records
// the first matching way of a key and stops).
template <typename K, typename UK>
__global__ __launch_bounds__(256) void update_more_records_kernel(
    const K* keys, int64_t n, const K* tags, UK num_sets, const uint8_t* values,
    int64_t value_stride, uint64_t* rec_slot, int64_t* rec_tag, uint64_t* rec_src, uint32_t* count,
    uint32_t cap) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  UK set;
  const K key = keys[i];
  uint32_t mask = matching_ways<K, UK>(tags, num_sets, key, &set);
  mask &= mask - 1;  // the first way has record i
  while (mask) {
    const int w = __ffs(mask) - 1;
    mask &= mask - 1;
    const uint32_t r = atomicAdd(count, 1u);
    if (r >= cap) return;
    rec_slot[r] = (uint64_t)set * 8 + (uint64_t)w;
    rec_tag[r] = record_tag<K, UK>(key, num_sets, tags[(uint64_t)set * 8 + w], true);
    rec_src[r] = (uint64_t)values + (uint64_t)i * (uint64_t)value_stride;
  }
}

// *p (a 32-bit word holding fp16 element `half` at bits 16*half) += v.
__device__ __forceinline__ void atomic_add_f16(uint32_t* word, int half, uint16_t v) {
  uint32_t old = __hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  while (true) {
    const uint16_t cur = (uint16_t)(old >> (16 * half));
    const uint16_t sum = f2h(h2f(cur) + h2f(v));
    const uint32_t nw = half ? ((old & 0x0000ffffu) | ((uint32_t)sum << 16))
                             : ((old & 0xffff0000u) | sum);
    const uint32_t seen = atomicCAS(word, old, nw);
    if (seen == old) return;
    old = seen;
  }
}

// The 32-bit word at *word += the two fp16 elements of v (low half to low
// half), each sum computed in fp32 and rounded to nearest even once.
__device__ __forceinline__ void atomic_add_f16x2(uint32_t* word, uint32_t v) {
  uint32_t old = __hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  while (true) {
    const uint16_t lo = f2h(h2f((uint16_t)old) + h2f((uint16_t)v));
    const uint16_t hi = f2h(h2f((uint16_t)(old >> 16)) + h2f((uint16_t)(v >> 16)));
    const uint32_t nw = ((uint32_t)hi << 16) | lo;
    const uint32_t seen = atomicCAS(word, old, nw);
    if (seen == old) return;
    old = seen;
  }
}

// dst[0..elems) += src[0..elems) in the float type T (fp32 or fp16 bits).
// fp16 rows whose destination and length are 4-byte aligned are added a word
// (two elements) per lane: lanes updating the two halves of one word would
// otherwise retry each other's compare-and-swaps.
template <bool F16>
__device__ __forceinline__ void add_row(uint8_t* dst, const uint8_t* src, uint64_t row_bytes,
                                        int lane, int lanes) {
  if constexpr (F16) {
    if ((((uint64_t)dst | row_bytes) & 3u) == 0) {
      const uint64_t words = row_bytes / 4;
      for (uint64_t e = lane; e < words; e += lanes) {
        const uint64_t sa = (uint64_t)src + 4 * e;
        const uint32_t v = (sa & 3u) == 0 ? gload<uint32_t>(sa)
                                          : (uint32_t)gload<uint16_t>(sa) |
                                                ((uint32_t)gload<uint16_t>(sa + 2) << 16);
        atomic_add_f16x2(reinterpret_cast<uint32_t*>(dst) + e, v);
      }
      return;
    }
    const uint64_t elems = row_bytes / 2;
    for (uint64_t e = lane; e < elems; e += lanes) {
      const uint64_t a = (uint64_t)dst + 2 * e;
      const uint16_t v = gload<uint16_t>((uint64_t)src + 2 * e);
      atomic_add_f16(reinterpret_cast<uint32_t*>(a & ~(uint64_t)3), (int)((a >> 1) & 1), v);
    }
  } else {
    const uint64_t elems = row_bytes / 4;
    for (uint64_t e = lane; e < elems; e += lanes) {
      const float v = __uint_as_float(gload<uint32_t>((uint64_t)src + 4 * e));
      atomicAdd(reinterpret_cast<float*>(dst) + e, v);
    }
  }
}

// one wave per record
template <bool F16>
__global__ __launch_bounds__(256) void accumulate_rows_kernel(const uint32_t* num,
                                                              uint32_t max_records,
                                                              const uint64_t* slot,
                                                              const uint64_t* src, uint8_t* data,
                                                              uint64_t row_bytes) {
  const int64_t rec = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const uint32_t n = num != nullptr && *num < max_records ? *num : max_records;
  if (rec >= n || slot[rec] == kNoRecord) return;
  add_row<F16>(data + slot[rec] * row_bytes, reinterpret_cast<const uint8_t*>(src[rec]), row_bytes,
               threadIdx.x & 63, 64);
}

// one wave per key: whole-row copy in VB-byte chunks
template <typename K, int VB>
__global__ __launch_bounds__(256) void table_update_kernel(const K* keys, int64_t n,
                                                           const uint8_t* values,
                                                           int64_t value_stride, uint8_t* table,
                                                           uint64_t row_bytes, uint64_t num_rows) {
  const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (i >= n) return;
  const uint64_t key = (uint64_t)(int64_t)keys[i];
  if (key >= num_rows) return;  // outside the table (negative keys wrap above it)
  const uint8_t* s = values + (uint64_t)i * (uint64_t)value_stride;
  uint8_t* d = table + key * row_bytes;
  for (uint64_t o = (uint64_t)lane * VB; o < row_bytes; o += 64 * VB)
    store_vec<VB>(d + o, load_vec<VB>(s + o));
}

template <typename K, bool F16>
__global__ __launch_bounds__(256) void table_accumulate_kernel(const K* keys, int64_t n,
                                                               const uint8_t* values,
                                                               int64_t value_stride,
                                                               uint8_t* table, uint64_t row_bytes,
                                                               uint64_t num_rows) {
  const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  if (i >= n) return;
  const uint64_t key = (uint64_t)(int64_t)keys[i];
  if (key >= num_rows) return;
  add_row<F16>(table + key * row_bytes, values + (uint64_t)i * (uint64_t)value_stride, row_bytes,
               threadIdx.x & 63, 64);
}

// ---------------------------------------------------------------------------
namespace {
int copy_vb(const void* a, const void* b, int64_t stride, uint64_t row_bytes) {
  const uint64_t x = (uint64_t)a | (uint64_t)b | (uint64_t)stride | row_bytes;
  return x % 16 == 0 ? 16 : x % 4 == 0 ? 4 : 1;
}
}  // namespace

hipError_t launch_update_records(const void* keys, int64_t n, int key_bytes, const void* tags,
                                 uint64_t num_sets, const uint8_t* values, int64_t value_stride,
                                 uint64_t* rec_slot, int64_t* rec_tag, uint64_t* rec_src,
                                 uint32_t* multi, bool own_tag, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  const dim3 grid((unsigned)((n + 255) / 256));
  if (key_bytes == 4)
    hipLaunchKernelGGL((update_records_kernel<int32_t, uint32_t>), grid, dim3(256), 0, stream,
                       (const int32_t*)keys, n, (const int32_t*)tags, (uint32_t)num_sets, values,
                       value_stride, rec_slot, rec_tag, rec_src, multi, own_tag);
  else
    hipLaunchKernelGGL((update_records_kernel<int64_t, uint64_t>), grid, dim3(256), 0, stream,
                       (const int64_t*)keys, n, (const int64_t*)tags, (uint64_t)num_sets, values,
                       value_stride, rec_slot, rec_tag, rec_src, multi, own_tag);
  return hipGetLastError();
}

hipError_t launch_update_more_records(const void* keys, int64_t n, int key_bytes, const void* tags,
                                      uint64_t num_sets, const uint8_t* values, int64_t value_stride,
                                      uint64_t* rec_slot, int64_t* rec_tag, uint64_t* rec_src,
                                      uint32_t* count, uint32_t cap, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  const dim3 grid((unsigned)((n + 255) / 256));
  if (key_bytes == 4)
    hipLaunchKernelGGL((update_more_records_kernel<int32_t, uint32_t>), grid, dim3(256), 0, stream,
                       (const int32_t*)keys, n, (const int32_t*)tags, (uint32_t)num_sets, values,
                       value_stride, rec_slot, rec_tag, rec_src, count, cap);
  else
    hipLaunchKernelGGL((update_more_records_kernel<int64_t, uint64_t>), grid, dim3(256), 0, stream,
                       (const int64_t*)keys, n, (const int64_t*)tags, (uint64_t)num_sets, values,
                       value_stride, rec_slot, rec_tag, rec_src, count, cap);
  return hipGetLastError();
}

hipError_t launch_accumulate_rows(const uint32_t* num, uint32_t max_records, const uint64_t* slot,
                                  const uint64_t* src, uint8_t* data, uint64_t row_bytes, int dtype,
                                  hipStream_t stream) {
  if (max_records == 0) return hipSuccess;
  const dim3 grid((unsigned)(((uint64_t)max_records * 64 + 255) / 256));
  if (dtype == kF16)
    hipLaunchKernelGGL(accumulate_rows_kernel<true>, grid, dim3(256), 0, stream, num, max_records,
                       slot, src, data, row_bytes);
  else if (dtype == kF32)
    hipLaunchKernelGGL(accumulate_rows_kernel<false>, grid, dim3(256), 0, stream, num, max_records,
                       slot, src, data, row_bytes);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_table_update(const void* keys, int64_t n, int key_bytes, const uint8_t* values,
                               int64_t value_stride, uint8_t* table, uint64_t row_bytes,
                               uint64_t num_rows, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  const dim3 grid((unsigned)(((uint64_t)n * 64 + 255) / 256));
  const int vb = copy_vb(values, table, value_stride, row_bytes);
#define L_UPD(K, V)                                                                            \
  hipLaunchKernelGGL((table_update_kernel<K, V>), grid, dim3(256), 0, stream, (const K*)keys, n, \
                     values, value_stride, table, row_bytes, num_rows)
  if (key_bytes == 4) {
    if (vb == 16) L_UPD(int32_t, 16); else if (vb == 4) L_UPD(int32_t, 4); else L_UPD(int32_t, 1);
  } else {
    if (vb == 16) L_UPD(int64_t, 16); else if (vb == 4) L_UPD(int64_t, 4); else L_UPD(int64_t, 1);
  }
#undef L_UPD
  return hipGetLastError();
}

hipError_t launch_table_accumulate(const void* keys, int64_t n, int key_bytes,
                                   const uint8_t* values, int64_t value_stride, uint8_t* table,
                                   uint64_t row_bytes, uint64_t num_rows, int dtype,
                                   hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  if (dtype != kF32 && dtype != kF16) return hipErrorInvalidValue;
  const dim3 grid((unsigned)(((uint64_t)n * 64 + 255) / 256));
#define L_ACC(K, F)                                                                           \
  hipLaunchKernelGGL((table_accumulate_kernel<K, F>), grid, dim3(256), 0, stream, (const K*)keys, \
                     n, values, value_stride, table, row_bytes, num_rows)
  if (key_bytes == 4) {
    if (dtype == kF16) L_ACC(int32_t, true); else L_ACC(int32_t, false);
  } else {
    if (dtype == kF16) L_ACC(int64_t, true); else L_ACC(int64_t, false);
  }
#undef L_ACC
  return hipGetLastError();
}

}  // namespace nve_amd
