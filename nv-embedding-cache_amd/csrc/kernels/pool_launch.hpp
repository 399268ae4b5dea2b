// pool_launch.hpp -- per-type-group launchers of the find-and-pool kernel
// (pool_float.hip, pool_quant.hip, pool_ext.hip), called by launch_pool once
// it has chosen the geometry.
#pragma once

#include "launch.hpp"

namespace nve_amd {

// kF32, kF16
hipError_t launch_pool_float(const PoolLaunch& a, const PoolGeometry& g, hipStream_t stream);
// kQI8F32, kQI8F16, kQU8F32, kQU8F16
hipError_t launch_pool_quant(const PoolLaunch& a, const PoolGeometry& g, hipStream_t stream);
// kXI8AF32, kXE4M3F32
hipError_t launch_pool_ext(const PoolLaunch& a, const PoolGeometry& g, hipStream_t stream);

// Long bags over one linear f16 / f32 table (pool_split.hip): the same sums
// as pool_kernel's split-bag path with fewer instructions.
bool pool_split_eligible(const PoolLaunch& a, const PoolGeometry& g);
hipError_t launch_pool_split(const PoolLaunch& a, const PoolGeometry& g, hipStream_t stream);
// Short bags (one lane group per bag) over linear f16 / f32 tables, one or
// several (pool_split.hip): the same sums as pool_kernel's one-group path.
bool pool_short_eligible(const PoolLaunch& a, const PoolGeometry& g);
hipError_t launch_pool_short(const PoolLaunch& a, const PoolGeometry& g, hipStream_t stream);

}  // namespace nve_amd
