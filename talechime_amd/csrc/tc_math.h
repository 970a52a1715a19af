// tc_math.h -- exponentials and logarithms shared by the host table generator
// and the gfx950 kernels.
//
// The same source is compiled for the CPU (to generate and check tables) and
// for the GPU, using only IEEE-754 basic operations, explicit fma() and
// ldexp(): both targets produce identical bits.
//
//  tc_exp_d(x)      exp(x) in double: Cody-Waite reduction by ln2 split into a
//                   32-bit head and a tail, degree-13 Taylor polynomial by
//                   Horner's rule, scaled by 2^k.  Relative error below 1e-15
//                   for |x| < 700, far below what the float rounding tests need.
//  tc_expf_cr(x)    exp(x) rounded once to float.  Checked exhaustively over
//                   every float in [-104, 88.72] to equal the correctly rounded
//                   value (the table generator asserts it).
//  tc_log_d(x)      ln(x) in double for finite x > 0: x = m * 2^e with m in
//                   [sqrt(1/2), sqrt(2)), ln m = 2 atanh(f), f = (m-1)/(m+1),
//                   odd series to f^29, plus e*ln2 (head + tail).
//  tc_logf_cr(x)    ln(x) rounded once to float.
//
// Rust's f32::exp on Linux is glibc's expf, which is not correctly rounded:
// it differs from tc_expf_cr on a known, finite set of inputs, all within
// 0.002 ulp of a rounding midpoint.  The device function tc_expf_glibc (in
// tc_expf_glibc.h) returns tc_expf_cr unless the double result lies within
// that band, and then consults the generated exception table.
#pragma once

#include <math.h>
#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define TC_HD __host__ __device__ __forceinline__
#else
#define TC_HD static inline
#endif

TC_HD double tc_exp_d(double x) {
  const double inv_ln2 = 1.4426950408889634074;   // 1/ln 2
  const double ln2_hi = 6.93147180369123816490e-01; // 0x3FE62E42FEE00000 (32 significant bits)
  const double ln2_lo = 1.90821492927058770002e-10; // ln2 - ln2_hi
  if (x != x) return x;
  if (x > 709.782712893384) return INFINITY;
  if (x < -745.2) return 0.0;
  double kd = rint(x * inv_ln2);
  double r = fma(-kd, ln2_hi, x);
  r = fma(-kd, ln2_lo, r);
  // Taylor coefficients 1/n!, n = 13 .. 0
  double p = 1.6059043836821614599e-10;     // 1/13!
  p = fma(p, r, 2.0876756987868098979e-09); // 1/12!
  p = fma(p, r, 2.5052108385441718775e-08); // 1/11!
  p = fma(p, r, 2.7557319223985890653e-07); // 1/10!
  p = fma(p, r, 2.7557319223985890653e-06); // 1/9!
  p = fma(p, r, 2.4801587301587301587e-05); // 1/8!
  p = fma(p, r, 1.9841269841269841270e-04); // 1/7!
  p = fma(p, r, 1.3888888888888888889e-03); // 1/6!
  p = fma(p, r, 8.3333333333333333333e-03); // 1/5!
  p = fma(p, r, 4.1666666666666666667e-02); // 1/4!
  p = fma(p, r, 1.6666666666666666667e-01); // 1/3!
  p = fma(p, r, 0.5);
  p = fma(p, r, 1.0);
  p = fma(p, r, 1.0);
  int k = (int)kd;
  // split the scaling so that no intermediate overflows or flushes early
  int k1 = k / 2, k2 = k - k1;
  return ldexp(ldexp(p, k1), k2);
}

TC_HD float tc_expf_cr(float x) {
  if (x != x) return x;
  if (x < -104.0f) return 0.0f;
  if (x > 88.72283935546875f) return INFINITY;
  return (float)tc_exp_d((double)x);
}

// exp(x) for x in [-87, 0] in float arithmetic only: k = rint(x / ln2),
// r = x - k ln2 (Cody-Waite, ln2 split into a 16-bit head and a tail), the
// degree-7 Taylor polynomial of exp(r) by Horner's rule with fmaf, scaled by
// 2^k.  The table generator checks every input of [-87, 0] to be within
// TC_EXPF_FAST_ULPS of tc_expf_cr.  The kernels use it for approximate terms
// only; bits that can change a result are recomputed with tc_expf_cr.
#define TC_EXPF_FAST_ULPS 1
TC_HD float tc_expf_fast(float x) {
  float kf = rintf(x * 1.44269504088896341f);
  float r = fmaf(kf, -0.693145751953125f, x);
  r = fmaf(kf, -1.42860682030941723212e-6f, r);
  float p = 1.98412698412698412698e-4f;  // 1/7!
  p = fmaf(p, r, 1.38888888888888888889e-3f);
  p = fmaf(p, r, 8.33333333333333333333e-3f);
  p = fmaf(p, r, 4.16666666666666666667e-2f);
  p = fmaf(p, r, 1.66666666666666666667e-1f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return ldexpf(p, (int)kf);
}

TC_HD double tc_log_d(double x) {
  // finite x > 0 only (callers handle 0, negatives, inf and NaN)
  const double ln2_hi = 6.93147180369123816490e-01;
  const double ln2_lo = 1.90821492927058770002e-10;
  int e;
  double m = frexp(x, &e);  // m in [0.5, 1)
  if (m < 0.70710678118654752440) {
    m = m * 2.0;
    e -= 1;
  }
  double f = (m - 1.0) / (m + 1.0);
  double f2 = f * f;
  // 2*atanh(f) = 2 (f + f^3/3 + f^5/5 + ...), |f| <= 0.1716
  double s = 1.0 / 29.0;
  s = fma(s, f2, 1.0 / 27.0);
  s = fma(s, f2, 1.0 / 25.0);
  s = fma(s, f2, 1.0 / 23.0);
  s = fma(s, f2, 1.0 / 21.0);
  s = fma(s, f2, 1.0 / 19.0);
  s = fma(s, f2, 1.0 / 17.0);
  s = fma(s, f2, 1.0 / 15.0);
  s = fma(s, f2, 1.0 / 13.0);
  s = fma(s, f2, 1.0 / 11.0);
  s = fma(s, f2, 1.0 / 9.0);
  s = fma(s, f2, 1.0 / 7.0);
  s = fma(s, f2, 1.0 / 5.0);
  s = fma(s, f2, 1.0 / 3.0);
  double lm = 2.0 * f + 2.0 * f * f2 * s;
  double ed = (double)e;
  return fma(ed, ln2_hi, fma(ed, ln2_lo, lm));
}

TC_HD float tc_logf_cr(float x) {
  if (x != x) return x;
  if (x < 0.0f) return NAN;
  if (x == 0.0f) return -INFINITY;
  if (x == INFINITY) return INFINITY;
  return (float)tc_log_d((double)x);
}

// Bit pattern of the float next to r = (float)y on the side where y lies.
TC_HD uint32_t tc_toward(double y, float r) {
  uint32_t b;
  memcpy(&b, &r, 4);
  double dy = y - (double)r;
  if (r == 0.0f) return dy >= 0.0 ? 0x00000001u : 0x80000001u;
  return ((dy >= 0.0) == (r > 0.0f)) ? b + 1u : b - 1u;
}

// Distance of a double y from the float rounding midpoint next to r = (float)y,
// in units of the float spacing there.  0.5 means y is exactly a float.  The
// spacing is a power of two, so the quotient is a multiplication by its exact
// reciprocal.
TC_HD double tc_mid_dist(double y, float r) {
  uint32_t nbb = tc_toward(y, r);
  float nb;
  memcpy(&nb, &nbb, 4);
  double gap = fabs((double)nb - (double)r);
  double mid = 0.5 * ((double)nb + (double)r);
  return fabs(y - mid) * ldexp(1.0, -ilogb(gap));
}
