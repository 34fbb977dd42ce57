// Reductions over a 64-lane wave on gfx950 without LDS round trips (the
// __shfl_xor butterfly compiles to ds_bpermute_b32, ~100 cycles a step).
#pragma once

#include <hip/hip_runtime.h>

namespace tt {
namespace {

// Reductions over the wave without LDS round trips: DPP within each row of
// 16 lanes (neighbour swap quad_perm [1,0,3,2], pair swap [2,3,0,1], then the
// mirrored half row and the mirrored row, after each of which a lane holds
// the total of twice as many lanes), then permlane swaps across rows (with
// both operands x, the two results are x[lane] and x[lane ^ 16], resp. 32).
// Every lane combines the same two values at each step, so all 64 end with
// the same bits.
template <int kCtrl>
__device__ __forceinline__ float dpp_f32(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), kCtrl, 0xF, 0xF, false));
}

template <typename Op>
__device__ __forceinline__ float wave_reduce(float x, Op op) {
  x = op(x, dpp_f32<0xB1>(x));   // quad_perm [1,0,3,2]
  x = op(x, dpp_f32<0x4E>(x));   // quad_perm [2,3,0,1]
  x = op(x, dpp_f32<0x141>(x));  // row_half_mirror
  x = op(x, dpp_f32<0x140>(x));  // row_mirror
  const auto p16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = op(__uint_as_float(p16[0]), __uint_as_float(p16[1]));
  const auto p32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return op(__uint_as_float(p32[0]), __uint_as_float(p32[1]));
}

__device__ __forceinline__ float wave_max(float x) {
  return wave_reduce(x, [](float u, float v) { return fmaxf(u, v); });
}

// maximum that propagates NaN (IEEE-754-2019 maximum)
__device__ __forceinline__ float wave_max_nan(float x) {
  return wave_reduce(x, [](float u, float v) { return __builtin_elementwise_maximum(u, v); });
}

__device__ __forceinline__ float wave_sum(float x) {
  return wave_reduce(x, [](float u, float v) { return u + v; });
}

}  // namespace
}  // namespace tt
