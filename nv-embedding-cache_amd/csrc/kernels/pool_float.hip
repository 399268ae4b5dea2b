// pool_float.hip -- find-and-pool instantiations for fp32 and fp16 rows.
#include "pool_kernel.cuh"
#include "pool_launch.hpp"

namespace nve_amd {

hipError_t launch_pool_float(const PoolLaunch& a, const PoolGeometry& g, hipStream_t stream) {
  if (a.stored_dtype == kF32) {
    switch (g.vb) {
      case 16: return launch_pool_sv<kF32, 16>(a, g, stream);
      case 8: return launch_pool_sv<kF32, 8>(a, g, stream);
      case 4: return launch_pool_sv<kF32, 4>(a, g, stream);
      default: return hipErrorInvalidValue;
    }
  }
  if (a.stored_dtype == kF16) {
    switch (g.vb) {
      case 16: return launch_pool_sv<kF16, 16>(a, g, stream);
      case 8: return launch_pool_sv<kF16, 8>(a, g, stream);
      case 4: return launch_pool_sv<kF16, 4>(a, g, stream);
      case 2: return launch_pool_sv<kF16, 2>(a, g, stream);
      default: return hipErrorInvalidValue;
    }
  }
  return hipErrorInvalidValue;
}

}  // namespace nve_amd
