// pool_quant.hip -- find-and-pool instantiations for the reference's rowwise
// int8 / uint8 row formats (nve_types.hpp QInt8Rowwise*, QUint8Rowwise*).
#include "pool_kernel.cuh"
#include "pool_launch.hpp"

namespace nve_amd {

hipError_t launch_pool_quant(const PoolLaunch& a, const PoolGeometry& g, hipStream_t stream) {
  switch (a.stored_dtype) {
    case kQI8F32: return launch_pool_bytes<kQI8F32>(a, g, stream);
    case kQI8F16: return launch_pool_bytes<kQI8F16>(a, g, stream);
    case kQU8F32: return launch_pool_bytes<kQU8F32>(a, g, stream);
    case kQU8F16: return launch_pool_bytes<kQU8F16>(a, g, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace nve_amd
