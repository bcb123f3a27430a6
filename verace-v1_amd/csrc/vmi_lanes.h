// Cross-lane sums for wave64 kernels on gfx950 (DPP row ops, v_permlane16_swap,
// v_permlane32_swap).
#pragma once
#include <hip/hip_runtime.h>

namespace vmi {

// Sum over the 16 lanes of a DPP row, result in every lane of the row.
template <int CTRL> __device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp_f32<0xB1>(x);   // quad_perm(1, 0, 3, 2)
  x += dpp_f32<0x4E>(x);   // quad_perm(2, 3, 0, 1)
  x += dpp_f32<0x141>(x);  // row_half_mirror
  x += dpp_f32<0x140>(x);  // row_mirror
  return x;
}
// Sum of the two 16-lane rows of each 32-lane half: v_permlane16_swap exchanges rows 1
// and 0 (3 and 2) between its two operands, so the two results add to row0 + row1.
__device__ __forceinline__ float row_pair_sum(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Sum of the two 32-lane halves of a wave (v_permlane32_swap, the same pattern).
__device__ __forceinline__ float half_pair_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

}  // namespace vmi
