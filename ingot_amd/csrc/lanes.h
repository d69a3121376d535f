// Lane exchanges within a 64-lane wave without an LDS round trip (gfx950).
#pragma once
#include <hip/hip_runtime.h>

namespace ih {

// x of lane (lane ^ H) without an LDS round trip (every lane of the wave active), from lane patterns that are their
// own inverse: DPP quad permutations and row mirrors within 16-lane rows (xor 4 = half-row mirror i ^ 7, then quad
// reversal i ^ 3; xor 8 = row mirror i ^ 15, then half-row mirror), the gfx950 row swaps for 16 and 32, which leave a
// lane its own value in one result and its partner's in the other (the partner's is the one that is not the lane's
// own bits; if both are, they are equal).
template <int CTRL>
__device__ __forceinline__ int dpp_mov(int b) {
  return __builtin_amdgcn_update_dpp(b, b, CTRL, 0xF, 0xF, false);
}
template <int H>
__device__ __forceinline__ float lane_xor(float v) {
  const int b = __float_as_int(v);
  if constexpr (H == 1) {
    return __int_as_float(dpp_mov<0xB1>(b));  // quad_perm [1,0,3,2]
  } else if constexpr (H == 2) {
    return __int_as_float(dpp_mov<0x4E>(b));  // quad_perm [2,3,0,1]
  } else if constexpr (H == 4) {
    return __int_as_float(dpp_mov<0x1B>(dpp_mov<0x141>(b)));  // row_half_mirror, then quad_perm [3,2,1,0]
  } else if constexpr (H == 8) {
    return __int_as_float(dpp_mov<0x141>(dpp_mov<0x140>(b)));  // row_mirror, then row_half_mirror
  } else {
    static_assert(H == 16 || H == 32, "lane_xor: H is a power of two below 64");
    unsigned p0, p1;
    if constexpr (H == 16) {
      const auto sw = __builtin_amdgcn_permlane16_swap(unsigned(b), unsigned(b), false, false);
      p0 = sw[0];
      p1 = sw[1];
    } else {
      const auto sw = __builtin_amdgcn_permlane32_swap(unsigned(b), unsigned(b), false, false);
      p0 = sw[0];
      p1 = sw[1];
    }
    return __uint_as_float(p0 == unsigned(b) ? p1 : p0);
  }
}

}  // namespace ih
