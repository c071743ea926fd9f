// Device-side scalar numerics of the W8A8 path: the rounding points and the
// sigmoid's exponential. Every function is a fixed sequence of IEEE f32
// operations; the library is compiled with -ffp-contract=off so nothing fuses.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace k2w8 {

// f32 -> bf16 -> f32, round to nearest even on the bit pattern
// (the rounding of src/numerics.rs:18-26 for finite values and infinities).
__device__ __forceinline__ float bf16_round(float x) {
  uint32_t u = __float_as_uint(x);
  u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
  return __uint_as_float(u);
}

__device__ __forceinline__ uint16_t bf16_bits(float x) {
  uint32_t u = __float_as_uint(x);
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ float bf16_value(uint16_t b) {
  return __uint_as_float((uint32_t)b << 16);
}

typedef float k2w8_f2 __attribute__((ext_vector_type(2)));
typedef __bf16 k2w8_bf2 __attribute__((ext_vector_type(2)));
typedef _Float16 k2w8_h2 __attribute__((ext_vector_type(2)));

// Two f32 values to packed bf16 (low half first) with the hardware conversion,
// round to nearest even: the same bits as bf16_bits for every non-NaN input.
__device__ __forceinline__ uint32_t bf16_pack2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(k2w8_f2{a, b}, k2w8_bf2));
}

// One value rounded to bf16 and widened back to f32 (bf16_round), in one hardware
// conversion: packing (0, x) puts bf16(x) in the high half over a zero low half, which
// is the widened value itself.
__device__ __forceinline__ float bf16_round1(float x) {
  return __builtin_bit_cast(float, __builtin_convertvector(k2w8_f2{0.0f, x}, k2w8_bf2));
}

// Two values rounded to bf16 and widened back to f32 (bf16_round on each): two
// conversions, against one conversion of the pair and two instructions to unpack it.
__device__ __forceinline__ void bf16_round2(float &a, float &b) {
  a = bf16_round1(a);
  b = bf16_round1(b);
}

// Two f32 values to packed f16 (low half first), round to nearest even.
__device__ __forceinline__ uint32_t f16_pack2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(k2w8_f2{a, b}, k2w8_h2));
}

// f32 -> f16 (hardware conversion, round to nearest even) and back.
__device__ __forceinline__ uint16_t f16_bits(float x) {
  _Float16 h = (_Float16)x;
  return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ float f16_value(uint16_t b) {
  return (float)__builtin_bit_cast(_Float16, b);
}

__device__ __forceinline__ float f16_round(float x) { return (float)(_Float16)x; }

// exp(x) for the sigmoids of the gated prepare and the SwiGLU epilogue:
// Cody-Waite reduction x = n*ln2 + r (two-part ln2), e^r = 1 + r + r^2 q(r) with a
// degree-4 least-squares q, then p * 2^n rounded once. The CPU definition scales by
// two power-of-two factors and branches to its special cases; this form uses ldexp
// and selects them, which gives the identical value for every f32 input.
__device__ __forceinline__ float sigmoid_exp(float x) {
  // Branch-free: the special cases are selected at the end (a wave would otherwise
  // branch around them per element).
  float n = __builtin_rintf(x * 0x1.715476p+0f);
  float r = __builtin_fmaf(n, -0x1.62e4p-1f, x);
  r = __builtin_fmaf(n, -0x1.7f7d1cp-20f, r);
  float q = __builtin_fmaf(0x1.6d4854p-10f, r, 0x1.121286p-7f);
  q = __builtin_fmaf(q, r, 0x1.5554e6p-5f);
  q = __builtin_fmaf(q, r, 0x1.5554d6p-3f);
  q = __builtin_fmaf(q, r, 0.5f);
  float r2 = r * r;
  float p = 1.0f + __builtin_fmaf(q, r2, r);
  // p * 2^n with one rounding (v_ldexp_f32). The CPU definition multiplies by 2^(n/2)
  // (exact: the product stays normal) and then by 2^(n - n/2), which rounds once: the
  // same value.
  float e = __builtin_amdgcn_ldexpf(p, (int)n);
  e = x > 0x1.62e42ep+6f ? __builtin_inff() : e;
  e = x < -0x1.9fe368p+6f ? 0.0f : e;
  return x != x ? x : e;
}

// 1 / (1 + exp(-g)), correctly rounded. For 1 <= d < 2^126 the hardware reciprocal
// (within 1 ulp) and one residual correction, res = 1 - d*y exactly by fma, then
// y + res*y rounded once, give the correctly rounded quotient: checked on the device
// for every such d. Larger d (subnormal quotients, and infinity) take the IEEE
// division. sigmoid_fast is the common path and returns d; sigmoid_fix redoes the
// quotient where d is that large.
__device__ __forceinline__ float sigmoid_fast(float g, float &den) {
  const float e = sigmoid_exp(0.0f - g);
  den = 1.0f + e;
  float y = __builtin_amdgcn_rcpf(den);
  const float res = __builtin_fmaf(-den, y, 1.0f);
  return __builtin_fmaf(res, y, y);
}

__device__ __forceinline__ float sigmoid_fix(float y, float den) { return den >= 0x1p126f ? 1.0f / den : y; }

// One sigmoid; the division runs only in a wave with a lane that needs it.
__device__ __forceinline__ float sigmoid(float g) {
  float den;
  float y = sigmoid_fast(g, den);
  if (__builtin_expect(den >= 0x1p126f, 0)) {
    asm volatile("");  // keeps the division out of the common path
    y = 1.0f / den;
  }
  return y;
}

// The SwiGLU products of N gate and up values (N even, each already rounded to bf16):
// g[k] <- bf16(bf16(g[k] * sigmoid(g[k])) * u[k]), the values of the per-element form.
// Every sigmoid's common path runs before the one branch to the division path (taken
// only by a wave with a lane that needs it), so the N operation chains interleave
// instead of each ending at a branch of its own.
template <int N>
__device__ __forceinline__ void swiglu_products(float (&g)[N], const float (&u)[N]) {
  static_assert(N % 2 == 0, "pairs");
  float y[N], den[N];
  bool slow = false;
#pragma unroll
  for (int k = 0; k < N; ++k) {
    y[k] = sigmoid_fast(g[k], den[k]);
    slow |= den[k] >= 0x1p126f;
  }
  if (__builtin_expect(slow, 0)) {
#pragma unroll
    for (int k = 0; k < N; ++k) y[k] = sigmoid_fix(y[k], den[k]);
  }
#pragma unroll
  for (int k = 0; k < N; k += 2) {
    float s0 = g[k] * y[k], s1 = g[k + 1] * y[k + 1];
    bf16_round2(s0, s1);
    float p0 = s0 * u[k], p1 = s1 * u[k + 1];
    bf16_round2(p0, p1);
    g[k] = p0;
    g[k + 1] = p1;
  }
}

}  // namespace k2w8
