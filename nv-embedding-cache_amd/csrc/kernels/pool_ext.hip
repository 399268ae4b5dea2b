// pool_ext.hip -- find-and-pool instantiations for this build's two extra
// row formats (int8 with fp32 scale and offset; OCP fp8 e4m3 with fp32 scale).
#include "pool_kernel.cuh"
#include "pool_launch.hpp"

namespace nve_amd {

hipError_t launch_pool_ext(const PoolLaunch& a, const PoolGeometry& g, hipStream_t stream) {
  switch (a.stored_dtype) {
    case kXI8AF32: return launch_pool_bytes<kXI8AF32>(a, g, stream);
    case kXE4M3F32: return launch_pool_bytes<kXE4M3F32>(a, g, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace nve_amd
