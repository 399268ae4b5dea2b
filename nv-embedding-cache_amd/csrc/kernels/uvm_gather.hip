// uvm_gather.hip -- kernels of the SortGather and PipelineGather lookup modes.
//
// Reference behaviour restated:
//   SortGather      find + SortPairs + gather (ec_set_associative.cuh:814-1057):
//                   resolve every key, sort the lookups so that misses (read
//                   over the host link) and hits (read from HBM) run in
//                   separate waves, each group in key order, then copy.
//   PipelineGather  gather_flow_pipeline (pipeline_gather.cuh:203-412): the GPU
//                   copies the hits, host threads copy the missed rows into a
//                   staging buffer, the GPU scatters the staged rows.
// Every mode writes the same output as the direct lookup.
#include "device_common.cuh"
#include "uvm_gather_launch.hpp"

namespace nve_amd {

__global__ __launch_bounds__(256) void sortgather_keys_kernel(const void* keys, int64_t n,
                                                              int key_bytes, RowSource src,
                                                              int bits, uint64_t* sort_key,
                                                              uint32_t* pos,
                                                              unsigned long long* miss_counter,
                                                              unsigned long long* call_misses) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t all = (bits >= 64) ? ~0ull : ((1ull << bits) - 1);
  bool miss = false;
  if (i < n) {
    const int64_t key = load_key(keys, key_bytes, i);
    const uint64_t addr = resolve_row(src, key_bytes, key, i, &miss);
    const bool hit = addr != 0 && !miss;
    // the order inside a group only shapes the access pattern: clamp the key
    const uint64_t k = (addr != 0 && (uint64_t)key < all) ? (uint64_t)key : all;
    sort_key[i] = ((uint64_t)(hit ? 1 : 0) << bits) | k;
    pos[i] = (uint32_t)i;
  }
  if (miss_counter != nullptr) add_misses(miss_counter, miss ? 1u : 0u);
  if (call_misses != nullptr) add_misses(call_misses, miss ? 1u : 0u);
}

// keys in sorted order: out[j] = keys[pos[j]], in the key type
__global__ __launch_bounds__(256) void permute_keys_kernel(const void* keys, int key_bytes,
                                                           const uint32_t* pos, int64_t n,
                                                           void* out) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j < n) store_key(out, key_bytes, j, load_key(keys, key_bytes, pos[j]));
}

// one wave per staged row
template <int VB>
__global__ __launch_bounds__(256) void scatter_rows_kernel(const uint8_t* staging,
                                                           const uint32_t* pos, int64_t count,
                                                           uint64_t row_bytes, uint8_t* out,
                                                           int64_t out_stride) {
  const int64_t j = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (j >= count) return;
  const uint8_t* s = staging + (uint64_t)j * row_bytes;
  uint8_t* d = out + (uint64_t)gload<uint32_t>((uint64_t)(pos + j)) * (uint64_t)out_stride;
  for (uint64_t o = (uint64_t)lane * VB; o < row_bytes; o += 64 * VB)
    store_vec<VB>(d + o, load_vec<VB>(s + o));
}

hipError_t launch_sortgather_keys(const void* keys, int64_t n, int key_bytes, const RowSource& src,
                                  int bits, uint64_t* sort_key, uint32_t* pos,
                                  unsigned long long* miss_counter,
                                  unsigned long long* call_misses, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  if (bits < 1 || bits > 62) return hipErrorInvalidValue;
  hipLaunchKernelGGL(sortgather_keys_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     stream, keys, n, key_bytes, src, bits, sort_key, pos, miss_counter, call_misses);
  return hipGetLastError();
}

hipError_t launch_permute_keys(const void* keys, int key_bytes, const uint32_t* pos, int64_t n,
                               void* out, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(permute_keys_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                     keys, key_bytes, pos, n, out);
  return hipGetLastError();
}

hipError_t launch_scatter_rows(const uint8_t* staging, const uint32_t* pos, int64_t count,
                               uint64_t row_bytes, uint8_t* out, int64_t out_stride,
                               hipStream_t stream) {
  if (count <= 0) return hipSuccess;
  const dim3 grid((unsigned)(((uint64_t)count * 64 + 255) / 256));
  const uint64_t x = (uint64_t)staging | (uint64_t)out | (uint64_t)out_stride | row_bytes;
  if (x % 16 == 0)
    hipLaunchKernelGGL(scatter_rows_kernel<16>, grid, dim3(256), 0, stream, staging, pos, count,
                       row_bytes, out, out_stride);
  else if (x % 4 == 0)
    hipLaunchKernelGGL(scatter_rows_kernel<4>, grid, dim3(256), 0, stream, staging, pos, count,
                       row_bytes, out, out_stride);
  else
    hipLaunchKernelGGL(scatter_rows_kernel<1>, grid, dim3(256), 0, stream, staging, pos, count,
                       row_bytes, out, out_stride);
  return hipGetLastError();
}

}  // namespace nve_amd
