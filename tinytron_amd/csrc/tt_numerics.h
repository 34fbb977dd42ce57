// Bit-exact rounding helpers shared by the gfx950 kernels.
//
// bf16: the reference rounds every elementwise result to bf16 under
// autocast (engine.py:180-185, attn.py:61-62); f32_to_bf16_bits is
// round-to-nearest-even with NaN kept quiet, the rounding torch applies.
// fp8-e4m3fn (OCP: bias 7, max 448, 0x7F/0xFF NaN, no inf): encoding is done
// in integer arithmetic so that rounding and edge cases are exactly those of
// torch's float8_e4m3fn cast: ties to even, magnitudes above 464 and
// non-finite inputs become NaN, 464 rounds to 448.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tt {

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) {
  return __uint_as_float(((uint32_t)h) << 16);
}

__device__ __forceinline__ float round_bf16(float f) {
  return bf16_bits_to_f32(f32_to_bf16_bits(f));
}

__device__ __forceinline__ uint8_t f32_to_e4m3fn(float x) {
  const uint32_t u = __float_as_uint(x);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x43e80000u) return (uint8_t)(sign | 0x7fu);  // |x| > 464, inf, NaN
  if (a < 0x3c800000u) {                                 // |x| < 2^-6: subnormal grid m * 2^-9
    const float v = __uint_as_float(a) * 512.0f;         // exact (power-of-two scale)
    return (uint8_t)(sign | (uint32_t)rintf(v));         // rintf: ties to even; 8 -> min normal
  }
  const uint32_t r = a + 0x7ffffu + ((a >> 20) & 1u);   // RNE at 3 mantissa bits
  const uint32_t e = (r >> 23) - 120u;                  // rebias 127 -> 7
  const uint32_t m = (r >> 20) & 7u;
  return (uint8_t)(sign | (e << 3) | m);
}

}  // namespace tt
