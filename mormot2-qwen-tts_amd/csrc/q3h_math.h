// q3h_math.h - scalar device math whose results are fixed to the bit by IEEE
// operations alone, so that the int8 path reproduces a CPU evaluation of the
// same formulas exactly.
#pragma once

#include <hip/hip_runtime.h>

namespace q3h {

// e^x: Cody & Waite (1980) argument reduction x = k ln2 + r, k = rint(x
// log2 e), ln 2 split in a 16-bit head and its tail; e^r by its Taylor series
// to r^7 (|r| <= 0.35: truncation < 6e-9 relative) in Horner form with fused
// multiply-adds; times 2^k built from the exponent bits. Error < 1 ulp
// measured; 0 below -86 (no subnormal results), +inf above 88.
__device__ __forceinline__ float exp_ieee(float x) {
  if (x != x) return x;
  if (x < -86.0f) return 0.0f;
  if (x > 88.0f) return __builtin_inff();
  const float k = rintf(__fmul_rn(x, 0x1.715476p+0f));
  float r = fmaf(k, -0x1.62e4p-1f, x);
  r = fmaf(k, -0x1.7f7d1cp-20f, r);
  float p = 0x1.a01a02p-13f;       // 1/7!
  p = fmaf(p, r, 0x1.6c16c2p-10f);  // 1/6!
  p = fmaf(p, r, 0x1.111112p-7f);   // 1/5!
  p = fmaf(p, r, 0x1.555556p-5f);   // 1/4!
  p = fmaf(p, r, 0x1.555556p-3f);   // 1/3!
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  const float scale = __builtin_bit_cast(float, (unsigned)((int)k + 127) << 23);
  return __fmul_rn(p, scale);
}

// SiLU(g) * u = g / (1 + e^-g) * u, each operation rounded once
__device__ __forceinline__ float silu_mul_ieee(float g, float u) {
  return __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, exp_ieee(-g))), u);
}

// RoPE of the pair (a, b) = (x_i, x_{i + d/2}): a' = a c - b s, b' = b c + a s,
// the second product fused into the subtraction / addition
__device__ __forceinline__ void rope_pair(float &a, float &b, float c, float s) {
  const float a0 = a, b0 = b;
  a = fmaf(a0, c, -__fmul_rn(b0, s));
  b = fmaf(b0, c, __fmul_rn(a0, s));
}

// x = hi + mid + lo exactly, each a bf16 (returned as its 16 bits in the low
// half): hi the top 8 significant bits of x, mid the next 8, lo the last 8
// (an f32 significand has 24; each difference is exact in f32). The
// operands of the split-bf16 matrix-core products.
__device__ __forceinline__ void split3(float x, uint32_t &h, uint32_t &m, uint32_t &l) {
  const uint32_t u = __float_as_uint(x);
  const uint32_t hb = u & 0xffff0000u;
  const float r1 = x - __uint_as_float(hb);
  const uint32_t mb = __float_as_uint(r1) & 0xffff0000u;
  const float r2 = r1 - __uint_as_float(mb);
  h = hb >> 16;
  m = mb >> 16;
  l = __float_as_uint(r2) >> 16;
}

}  // namespace q3h
