// rh_math.h -- expf and sqrtf with the bits of the CPU path's.
//
// rusticide's f32::exp (softmax, SiLU) is libm's expf: on Linux, glibc's,
// which since 2.27 is the published algorithm of ARM's optimized-routines
// (Szabolcs Nagy): x * 32/ln2 split into an integer k and a remainder r;
// 2^(k/32) from a 32-entry table of 2^(i/32) with k's high bits added to the
// exponent; 2^(r/32) from a cubic in double precision; one rounding to float.
// The x86-64 build glibc selects on FMA hardware fuses the products it can
// (r = fma(x, 32/ln2, -k) among them); that is the form restated here. It
// equals glibc's expf on every one of the 2^32 inputs, checked on the host
// (tests/test_math.py samples it; the exhaustive sweep takes a minute), and
// the device build runs the same IEEE double operations.
//
// The table entries are 2^(i/32) rounded to double, minus i << 47, so that
// adding k << 47 scales by 2^(k/32).
#pragma once

#include <stdint.h>

namespace rh {

__host__ __device__ inline float expf_ref(float x) {
  constexpr uint64_t kTable[32] = {
    0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL,
    0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL,
    0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
    0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL,
    0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL,
    0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
    0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL,
    0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL,
  };
  constexpr double kInvLn2N = 0x1.71547652b82fep+0 * 32;
  constexpr double kShift = 0x1.8p+52;
  constexpr double kC0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
  constexpr double kC1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
  constexpr double kC2 = 0x1.62e42ff0c52d6p-1 / 32;
  const uint32_t bits = __builtin_bit_cast(uint32_t, x);
  const uint32_t abstop = (bits >> 20) & 0x7ffu;
  if (abstop >= 0x42bu) {  // |x| >= 88, or x is inf / nan
    if (bits == 0xff800000u) return 0.0f;
    if (abstop >= 0x7f8u) return x + x;
    if (x > 0x1.62e42ep6f) return __builtin_inff();  // past log(2^128)
    if (x < -0x1.9fe368p6f) return 0.0f;             // below log(2^-150)
  }
  const double xd = static_cast<double>(x);
  double kd = __builtin_fma(kInvLn2N, xd, kShift);
  const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
  kd -= kShift;
  const double r = __builtin_fma(kInvLn2N, xd, -kd);
  const uint64_t t = kTable[ki % 32u] + (ki << 47);
  const double s = __builtin_bit_cast(double, t);
  const double z = __builtin_fma(kC0, r, kC1);
  const double r2 = r * r;
  double y = __builtin_fma(kC2, r, 1.0);
  y = __builtin_fma(z, r2, y);
  y = y * s;
  return static_cast<float>(y);
}

}  // namespace rh

namespace rh {

// sqrtf rounded to nearest, as the CPU's sqrtss gives it. The device's
// __fsqrt_rn maps to the native v_sqrt_f32, which is within one ulp but not
// always the nearest float; sqrt_fix corrects any start within one ulp.
//
// Why the correction is exact: take neighbouring floats a < b = a + u and
// x >= 2^-64 (so that every quantity below is a normal float). sqrt(x) rounds
// up to b or beyond exactly when sqrt(x) > (a + b) / 2, i.e. when
// x - a*b > u^2/4. Here a, b are multiples of u and x of a power of two that
// is at least u^2, so x - a*b is a multiple of u^2: the test is x - a*b > 0,
// and fma(-a, b, x) carries that sign exactly (it rounds the exact residual
// once). sqrt(x) is never exactly the midpoint, whose square is not a
// multiple of u^2. Checked on the host against sqrtss for every normal
// x >= 2^-64 from starts one ulp below, at and above the nearest float.
__host__ __device__ inline float sqrt_fix(float x, float s) {
  const uint32_t b = __builtin_bit_cast(uint32_t, s);
  const float up = __builtin_bit_cast(float, b + 1u);
  const float down = __builtin_bit_cast(float, b - 1u);
  if (__builtin_fmaf(-s, up, x) > 0.0f) return up;
  if (__builtin_fmaf(-down, s, x) <= 0.0f) return down;
  return s;
}

__host__ __device__ inline float sqrt_rn(float x) {
  if (x >= 0x1p-64f && x < __builtin_inff()) return sqrt_fix(x, __builtin_sqrtf(x));
  if (x > 0.0f) {  // tiny and subnormal x: scale by 2^96, exact both ways
    const float y = x * 0x1p96f;
    return sqrt_fix(y, __builtin_sqrtf(y)) * 0x1p-48f;
  }
  return __builtin_sqrtf(x);  // zero, +inf, negative, nan
}

}  // namespace rh
