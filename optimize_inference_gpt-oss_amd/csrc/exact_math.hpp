// The CPU's expf, bit for bit, for the exact attention path.
//
// The reference's CPU forward (run.cpp:335-353, softmax) calls the C
// library's expf. On x86-64 that is glibc's expf (sysdeps/ieee754/flt-32/
// e_expf.c with the table and coefficients of e_expf_data.c, ARM
// optimized-routines' algorithm), in the variant built with FMA, which the
// library selects on any CPU that has FMA:
//   z = x * 32/ln2 (in fp64), k = round(z), r = z - k  (|r| <= 1/2; the
//   compiler fuses the product into both, so z is never rounded)
//   2^(k/32) = 2^(k >> 5) * 2^((k mod 32)/32)  (the second factor from a table)
//   2^(r/32) ~ 1 + c2 r + c1 r^2 + c0 r^3  (three fused steps)
//   expf(x) = (float)(2^(r/32) * 2^(k/32))
// with inputs beyond the fp32 range handled first. The table and the
// coefficients have to be glibc's for the bits to agree: the table is
// 2^(i/32) rounded to fp64 (computed for this file from the definition),
// less i << 47 in its bits so that adding k << 47 scales it by 2^(k >> 5);
// the coefficients are glibc's published ones. tests/test_exact.py checks
// the function against the host expf on every fp32 input from -inf to the
// overflow bound.
#pragma once

#include <hip/hip_runtime.h>
#include <cmath>
#include <cstdint>
#include <cstring>

namespace gkv {

__host__ __device__ inline uint64_t exact_exp2_bits(int i) {
  // 2^(i/32) in fp64, minus i << 47 in the bits
  constexpr uint64_t t[32] = {
      0x3ff0000000000000, 0x3fefd9b0d3158574, 0x3fefb5586cf9890f, 0x3fef9301d0125b51,
      0x3fef72b83c7d517b, 0x3fef54873168b9aa, 0x3fef387a6e756238, 0x3fef1e9df51fdee1,
      0x3fef06fe0a31b715, 0x3feef1a7373aa9cb, 0x3feedea64c123422, 0x3feece086061892d,
      0x3feebfdad5362a27, 0x3feeb42b569d4f82, 0x3feeab07dd485429, 0x3feea47eb03a5585,
      0x3feea09e667f3bcd, 0x3fee9f75e8ec5f74, 0x3feea11473eb0187, 0x3feea589994cce13,
      0x3feeace5422aa0db, 0x3feeb737b0cdc5e5, 0x3feec49182a3f090, 0x3feed503b23e255d,
      0x3feee89f995ad3ad, 0x3feeff76f2fb5e47, 0x3fef199bdd85529c, 0x3fef3720dcef9069,
      0x3fef5818dcfba487, 0x3fef7c97337b9b5f, 0x3fefa4afa2a490da, 0x3fefd0765b6e4540,
  };
  return t[i];
}

__host__ __device__ inline uint32_t exact_f32_bits(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  return u;
}

__host__ __device__ inline double exact_f64_from_bits(uint64_t u) {
  double d;
  memcpy(&d, &u, 8);
  return d;
}

__host__ __device__ inline uint64_t exact_f64_bits(double d) {
  uint64_t u;
  memcpy(&u, &d, 8);
  return u;
}

__host__ __device__ inline float expf_cpu_exact(float x) {
#pragma clang fp contract(off)
  // the top 12 bits of x without the sign: 0x42b for |x| >= 88 and beyond
  const uint32_t top = (exact_f32_bits(x) >> 20) & 0x7ff;
  if (top >= 0x42b) {
    if (exact_f32_bits(x) == 0xff800000u) // -inf
      return 0.0f;
    if (top >= 0x7f8) // +inf or NaN
      return x + x;
    if (x > 0x1.62e42ep6f) // above ln(FLT_MAX)
      return INFINITY;
    if (x < -0x1.9fe368p6f) // below the smallest subnormal's log
      return 0.0f;
  }
  const double n_over_ln2 = 0x1.71547652b82fep0 * 32;
  const double round_shift = 0x1.8p52; // adding it rounds to an integer in the low bits
  const double c0 = 0x1.c6af84b912394p-5 / (32.0 * 32.0 * 32.0);
  const double c1 = 0x1.ebfce50fac4f3p-3 / (32.0 * 32.0);
  const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
  // z = x * 32/ln2 is never rounded on its own: the FMA build fuses the
  // product into both of its uses (z + shift and z - k)
  double kd = fma(n_over_ln2, (double)x, round_shift);
  const uint64_t ki = exact_f64_bits(kd);
  kd -= round_shift;
  const double r = fma(n_over_ln2, (double)x, -kd);
  const double s = exact_f64_from_bits(exact_exp2_bits((int)(ki & 31)) + (ki << 47));
  const double p = fma(c0, r, c1);
  double y = fma(c2, r, 1.0);
  y = fma(p, r * r, y);
  return (float)(y * s);
}

} // namespace gkv
