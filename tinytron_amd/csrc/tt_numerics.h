// Bit-exact rounding helpers shared by the gfx950 kernels.
//
// bf16: the reference rounds every elementwise result to bf16 under
// autocast (engine.py:180-185, attn.py:61-62); f32_to_bf16_bits is
// round-to-nearest-even with NaN kept quiet (upper half, quiet bit set), the
// rounding torch applies. gfx950 does it in one instruction
// (v_cvt_pk_bf16_f32, two values at a time); on every one of the 2^32 fp32
// patterns (NaN and denormals included, denormals not flushed) its result
// equals the integer formulation u + 0x7fff + lsb >> 16 (NaN: u >> 16 | 0x40).
// fp8-e4m3fn (OCP: bias 7, max 448, 0x7F/0xFF NaN, no inf): rounding and
// edge cases are exactly those of torch's float8_e4m3fn cast: ties to even,
// magnitudes above 464 and non-finite inputs become NaN with the input's
// sign, 464 rounds to 448. gfx950's v_cvt_pk_fp8_f32 (OCP e4m3, two values
// at a time) gives that byte for every fp32 pattern except positive NaN,
// which it encodes as 0xFF where torch writes 0x7F; f32_to_e4m3fn patches
// that one case. (Both instructions were compared with the integer
// formulations -- bf16: u + 0x7fff + lsb >> 16; e4m3: RNE at 3 mantissa
// bits, subnormals on the 2^-9 grid -- on every 32-bit pattern.)
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tt {

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}

// two values rounded to bf16 in one conversion: lo in bits 0-15, hi in 16-31
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) {
  return __uint_as_float(((uint32_t)h) << 16);
}

__device__ __forceinline__ float round_bf16(float f) {
  return bf16_bits_to_f32(f32_to_bf16_bits(f));
}

// 0x80 in byte k of the result when x is a positive NaN (bit pattern, as a
// signed integer, above +inf's)
__device__ __forceinline__ uint32_t e4m3fn_pos_nan_bit(float x, int k) {
  return (int32_t)__float_as_uint(x) > 0x7f800000 ? 0x80u << (8 * k) : 0u;
}

__device__ __forceinline__ uint8_t f32_to_e4m3fn(float x) {
  const uint32_t h = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(x, 0.0f, 0, false);
  return (uint8_t)((h & ~e4m3fn_pos_nan_bit(x, 0)) & 0xffu);
}

// four values, byte k = f32_to_e4m3fn of the k-th
__device__ __forceinline__ uint32_t pack_e4m3fn_x4(float a, float b, float c, float d) {
  uint32_t w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, (int)w, true);
  return w & ~(e4m3fn_pos_nan_bit(a, 0) | e4m3fn_pos_nan_bit(b, 1) | e4m3fn_pos_nan_bit(c, 2) |
               e4m3fn_pos_nan_bit(d, 3));
}

// fp8 cache rows (one scale per (token, KV head) row): scale = absmax / 448
// with a NaN-propagating absmax (IEEE-754-2019 maximum), codes e4m3fn(x /
// scale); an all-zero row stores zeros (scale 0), and a row holding a NaN or
// an infinity (scale not finite), which the format cannot represent, stores
// NaN codes (0x7F) throughout.
__device__ __forceinline__ float absmax2(float m, float x, float y) {
  return __builtin_elementwise_maximum(m, __builtin_elementwise_maximum(fabsf(x), fabsf(y)));
}

__device__ __forceinline__ uint8_t e4m3_row_code(float x, float scale) {
  if (scale == 0.f) return 0;
  if (!(scale <= 3.402823466e38f)) return 0x7F;
  return f32_to_e4m3fn(x / scale);
}

__device__ __forceinline__ uint32_t e4m3_row_codes4(const float (&x)[4], float scale) {
  if (scale == 0.f) return 0u;
  if (!(scale <= 3.402823466e38f)) return 0x7F7F7F7Fu;
  return pack_e4m3fn_x4(x[0] / scale, x[1] / scale, x[2] / scale, x[3] / scale);
}

}  // namespace tt
