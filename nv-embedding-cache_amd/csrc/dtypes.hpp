// dtypes.hpp -- stored-row formats shared by host and device code.
//
// Ids are the reference's DataType_t ids as exported through the C ABI
// (nve_c_api.h:70-88; nve_types.hpp:59-73), plus two row formats of this build
// that have no reference counterpart (declared in include/nve_amd_ext.h).
#pragma once

#include <stdint.h>

namespace nve_amd {

enum : int {
  kUnknown = 0,
  kF32 = 1,
  kBF16 = 2,
  kF16 = 3,
  kE4M3 = 4,
  kE5M2 = 5,
  kF64 = 6,
  kQI8F32 = 7,    // int8 values + f32 scale                  (nve_types.hpp:143-189)
  kQI8F16 = 8,    // int8 values + f16 scale
  kQU8F32 = 9,    // uint8 values + f32 scale + f32 offset
  kQU8F16 = 10,   // uint8 values + f16 scale + f16 offset
  kXI8AF32 = 32,  // extension: int8 values + f32 scale + f32 offset
  kXE4M3F32 = 33  // extension: OCP fp8 e4m3 values + f32 scale
};

inline constexpr bool is_rowwise(int dt) {
  return (dt >= kQI8F32 && dt <= kQU8F16) || dt == kXI8AF32 || dt == kXE4M3F32;
}

// bytes per stored value element
inline constexpr int value_elem_bytes(int dt) {
  return dt == kF32 ? 4 : (dt == kF16 || dt == kBF16) ? 2 : dt == kF64 ? 8 : 1;
}

// bytes of per-row metadata after the values
inline constexpr int meta_bytes(int dt) {
  switch (dt) {
    case kQI8F32: return 4;
    case kQI8F16: return 2;
    case kQU8F32: return 8;
    case kQU8F16: return 4;
    case kXI8AF32: return 8;
    case kXE4M3F32: return 4;
    default: return 0;
  }
}

// float precision of the dequantized value (quant_rowwise_output_dtype,
// nve_types.hpp:170-189): F16 for the f16-metadata types, else F32.
inline constexpr int native_out(int dt) {
  return (dt == kF16 || dt == kQI8F16 || dt == kQU8F16) ? kF16 : kF32;
}

// size in bytes of a plain (non-rowwise) element type
inline constexpr int dtype_size(int dt) {
  switch (dt) {
    case kF32: return 4;
    case kBF16:
    case kF16: return 2;
    case kE4M3:
    case kE5M2: return 1;
    case kF64: return 8;
    case kQI8F32:
    case kQI8F16:
    case kXI8AF32:
    case kXE4M3F32:
    case kQU8F32:
    case kQU8F16: return 1;
    default: return 0;
  }
}

}  // namespace nve_amd
