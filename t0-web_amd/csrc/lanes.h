// Cross-lane sums inside a wavefront through DPP lane moves and row swaps (VALU only: no LDS
// round trip, unlike __shfl_xor, which lowers to ds_bpermute on gfx950).
// Every lane of the group ends with the same value, summed in butterfly order
// ((a0+a1)+(a2+a3)) + ((a4+a5)+(a6+a7)) ..., so results equal the xor-shuffle
// form bit for bit.  Groups are aligned runs of 4 / 8 / 16 lanes (or the
// whole wave for rows_*); all their lanes must be active.
#pragma once

#include <hip/hip_runtime.h>

namespace t0h {

template <int CTRL>
__device__ __forceinline__ float dpp_move(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, true));
}

// quad_perm [1,0,3,2] and [2,3,0,1]: the xor-1 and xor-2 partners
__device__ __forceinline__ float lane_sum4(float x) {
  x += dpp_move<0xB1>(x);
  x += dpp_move<0x4E>(x);
  return x;
}
// row_half_mirror: lane i of each 8-lane half row reads lane 7-i (the other quad)
__device__ __forceinline__ float lane_sum8(float x) {
  x = lane_sum4(x);
  x += dpp_move<0x141>(x);
  return x;
}
// row_mirror: lane i of each 16-lane row reads lane 15-i (the other half row)
__device__ __forceinline__ float lane_sum16(float x) {
  x = lane_sum8(x);
  x += dpp_move<0x140>(x);
  return x;
}

// Across the four 16-lane rows (partners l^16, l^32, l^48) with the gfx950 row
// swaps: permlane16_swap of (x, x) leaves rows {0,0,2,2} in one result and
// {1,1,3,3} in the other; permlane32_swap does the same for the two halves.
// Combining the pair is symmetric, so the order matches the xor butterfly.
template <typename Op>
__device__ __forceinline__ float rows_reduce(float x, Op op) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = op(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return op(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float rows_sum(float x) {
  return rows_reduce(x, [](float a, float b) { return a + b; });
}
__device__ __forceinline__ float rows_max(float x) {
  return rows_reduce(x, [](float a, float b) { return fmaxf(a, b); });
}

}  // namespace t0h
