// RoPE arithmetic shared by the append kernel and the fused decode kernel:
// element access in the activation type and the rotation of one
// rotate_half pair with the reference's rounding points (attn.py:56-62).
#pragma once

#include "tt_numerics.h"

namespace tt {

template <typename T>
struct Elem;

template <>
struct Elem<float> {
  static __device__ __forceinline__ float load(const void *p, int64_t i) {
    return static_cast<const float *>(p)[i];
  }
  static __device__ __forceinline__ void store(void *p, int64_t i, float v) {
    static_cast<float *>(p)[i] = v;
  }
  static __device__ __forceinline__ float rnd(float v) { return v; }
  static __device__ __forceinline__ void rnd2(float &, float &) {}
};

struct BF16Tag {};

template <>
struct Elem<BF16Tag> {
  static __device__ __forceinline__ float load(const void *p, int64_t i) {
    return bf16_bits_to_f32(static_cast<const uint16_t *>(p)[i]);
  }
  static __device__ __forceinline__ void store(void *p, int64_t i, float v) {
    static_cast<uint16_t *>(p)[i] = f32_to_bf16_bits(v);
  }
  static __device__ __forceinline__ float rnd(float v) { return round_bf16(v); }
  // two values rounded in one conversion
  static __device__ __forceinline__ void rnd2(float &x, float &y) {
    const uint32_t p = pack_bf16x2(x, y);
    x = __uint_as_float(p << 16);
    y = __uint_as_float(p & 0xffff0000u);
  }
};

// out1 = r(r(x1*c) + r(-x2*s)), out2 = r(r(x2*c) + r(x1*s)), r = rounding to
// the activation type; the three ops of attn.py:61 in the reference's order.
template <typename A>
__device__ __forceinline__ void rotate_pair(float x1, float x2, float c, float s, float &o1, float &o2) {
#pragma clang fp contract(off)
  float a1 = x1 * c, a2 = x2 * c;
  Elem<A>::rnd2(a1, a2);
  float b1 = (-x2) * s, b2 = x1 * s;
  Elem<A>::rnd2(b1, b2);
  o1 = a1 + b1;
  o2 = a2 + b2;
  Elem<A>::rnd2(o1, o2);
}

}  // namespace tt
