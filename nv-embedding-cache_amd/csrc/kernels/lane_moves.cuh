// lane_moves.cuh -- moving 32-bit values between the lanes of a G-lane group
// without LDS: DPP row_newbcast inside a 16-lane row, v_permlane16_swap
// across rows (gfx950), v_readlane for a whole-wave group.  The source lane is
// a compile-time constant, so a value can be broadcast from the lane that
// loaded it to every lane of its group in one or two VALU instructions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace nve_amd {

// DPP controls (row = 16 lanes)
constexpr int kDppRowNewBcast = 0x150;  // + n: every lane of a row reads lane n of that row
constexpr int kDppRowRor8 = 0x128;      // lane l reads lane (l + 8) mod 16 of its row: l ^ 8
constexpr int kDppRowShl1 = 0x101;      // lane l reads lane l + 1 of its row

// Every row and bank enabled and every source lane inside the wave, so each
// lane is written and no "old" value is needed.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_mov(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xf, 0xf, false);
}

// Value v of lane l + 1 of this lane's 16-lane row; the row's last lane has no
// source inside the row and takes `fallback`.  A DPP read from a lane that is
// switched off also yields `fallback`, so every lane of the row must be on:
// the compiler may sink an instruction whose result is only used under a
// condition into that condition's branch (it did so here, and the lanes past
// the branch read `fallback`), hence row_next_pin.
__device__ __forceinline__ uint32_t row_next(uint32_t v, uint32_t fallback) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)fallback, (int)v, kDppRowShl1, 0xf, 0xf, false);
}
// Four row_next moves whose results are pinned where they are computed (an
// empty asm that uses them), so none of them can be moved into a branch.
__device__ __forceinline__ void row_next_pin(uint32_t (&v)[4], const uint32_t (&fallback)[4]) {
  uint32_t r0 = row_next(v[0], fallback[0]);
  uint32_t r1 = row_next(v[1], fallback[1]);
  uint32_t r2 = row_next(v[2], fallback[2]);
  uint32_t r3 = row_next(v[3], fallback[3]);
  asm volatile("" : "+v"(r0), "+v"(r1), "+v"(r2), "+v"(r3));
  v[0] = r0;
  v[1] = r1;
  v[2] = r2;
  v[3] = r3;
}

// Value of lane J of this lane's G-lane group (groups aligned to G lanes);
// `lane` is this lane's index in the wave (0..63).
template <int G, int J>
__device__ __forceinline__ uint32_t group_bcast(uint32_t v, int lane) {
  static_assert(J >= 0 && J < G, "broadcast source outside the group");
  if constexpr (G == 64) {
    return (uint32_t)__builtin_amdgcn_readlane((int)v, J);
  } else if constexpr (G == 16) {
    return dpp_mov<kDppRowNewBcast + J>(v);
  } else if constexpr (G == 8) {
    const uint32_t lo = dpp_mov<kDppRowNewBcast + J>(v);
    const uint32_t hi = dpp_mov<kDppRowNewBcast + 8 + J>(v);
    return (lane & 8) ? hi : lo;
  } else {  // G == 32: lane J % 16 of each row, then the even or odd row of each pair
    static_assert(G == 32, "group of 8, 16, 32 or 64 lanes");
    const uint32_t b = dpp_mov<kDppRowNewBcast + (J & 15)>(v);
    const auto r = __builtin_amdgcn_permlane16_swap(b, b, false, false);
    return J < 16 ? r[0] : r[1];
  }
}

// f(integral_constant<int, b * U>) for b = B .. NB - 1, unrolled at compile time
template <int U, int B, int NB, typename F>
__device__ __forceinline__ void for_batches(F& f) {
  if constexpr (B < NB) {
    f(std::integral_constant<int, B * U>{});
    for_batches<U, B + 1, NB>(f);
  }
}

// f(integral_constant<int, I>) for I = B .. E - 1, unrolled at compile time
template <int B, int E, typename F>
__device__ __forceinline__ void for_each_const(F& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    for_each_const<B + 1, E>(f);
  }
}

}  // namespace nve_amd
