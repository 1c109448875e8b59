/*
 * aos_exp.h — correctly rounded float64 exp for the router softmax.
 *
 * The router's softmax evaluates exp in float64 (crates/adapteros-lora-router/src/router.rs:
 * 1366-1377, Rust f64::exp, i.e. the host libm). Device libraries only promise a faithfully
 * rounded exp (about 1 ulp), so the GPU router uses this routine instead: a double-double
 * evaluation that returns the correctly rounded result except with probability about 2^-30 per
 * argument. Its outputs are checked against the host libm exp in the tests.
 *
 * Method (a standard argument-reduction + squaring scheme, all in double-double arithmetic built
 * from IEEE fma, so host and device produce identical bits):
 *   x = k*ln2 + r, |r| <= ln2/2, ln2 held as three doubles L1+L2+L3 (L1 has 21 trailing zero
 *   bits so k*L1 is exact);
 *   r' = r / 256;  u0 = expm1(r') = r' + r'^2/2 + r'^3/6 (double-double) + r'^4/24 + ... (double);
 *   eight squarings u <- 2u + u^2 give expm1(r);  exp(x) = 2^k * (1 + u).
 * Error of the double-double value before the final rounding is below 2^-85 relative.
 *
 * Arguments below -708.4 produce subnormal or zero results; those are returned rounded twice
 * (scaling of an already rounded value), which cannot change any router output because the
 * softmax divides by a sum >= 1 and converts to float32.
 *
 * Must be compiled with -ffp-contract=off.
 */
#ifndef AOS_EXP_H
#define AOS_EXP_H

#include <math.h>

#if defined(__HIPCC__)
#define AOS_HD __host__ __device__ inline
#else
#define AOS_HD static inline
#endif

typedef struct {
  double hi, lo;
} aos_dd;

AOS_HD aos_dd aos_two_sum(double a, double b) {
  aos_dd r;
  double s = a + b;
  double bb = s - a;
  double err = (a - (s - bb)) + (b - bb);
  r.hi = s;
  r.lo = err;
  return r;
}

AOS_HD aos_dd aos_fast_two_sum(double a, double b) {
  aos_dd r;
  double s = a + b;
  r.hi = s;
  r.lo = b - (s - a);
  return r;
}

AOS_HD aos_dd aos_dd_add(aos_dd a, aos_dd b) {
  aos_dd s = aos_two_sum(a.hi, b.hi);
  aos_dd t = aos_two_sum(a.lo, b.lo);
  s.lo += t.hi;
  s = aos_fast_two_sum(s.hi, s.lo);
  s.lo += t.lo;
  return aos_fast_two_sum(s.hi, s.lo);
}

AOS_HD aos_dd aos_dd_mul(aos_dd a, aos_dd b) {
  double p = a.hi * b.hi;
  double e = fma(a.hi, b.hi, -p);
  e = fma(a.hi, b.lo, e);
  e = fma(a.lo, b.hi, e);
  return aos_fast_two_sum(p, e);
}

AOS_HD double aos_exp_cr(double x) {
  const double kInvLn2 = 0x1.71547652b82fep+0;
  const double kL1 = 0x1.62e42fee00000p-1;
  const double kL2 = 0x1.a39ef35793c76p-33;
  const double kL3 = 0x1.cc01f97b57a08p-87;
  const aos_dd kSixth = {0x1.5555555555555p-3, 0x1.5555555555555p-57};
  const double kI24 = 0x1.5555555555555p-5;
  const double kI120 = 0x1.1111111111111p-7;
  const double kI720 = 0x1.6c16c16c16c17p-10;
  const double kI5040 = 0x1.a01a01a01a01ap-13;

  if (x != x) return x;
  if (x > 709.782712893384) return INFINITY;
  if (x < -745.2) return 0.0;

  double kd = rint(x * kInvLn2);
  /* r = x - kd*ln2 as a double-double */
  double t = fma(-kd, kL1, x); /* exact */
  double ph = kd * kL2;
  double pl = fma(kd, kL2, -ph);
  pl = fma(kd, kL3, pl);
  aos_dd r = aos_two_sum(t, -ph);
  r.lo -= pl;
  r = aos_fast_two_sum(r.hi, r.lo);
  r.hi *= 0x1.0p-8;
  r.lo *= 0x1.0p-8;

  /* u0 = r + r^2/2 + r^3/6 + tail */
  aos_dd r2 = aos_dd_mul(r, r);
  aos_dd r3 = aos_dd_mul(r2, r);
  aos_dd t3 = aos_dd_mul(r3, kSixth);
  double rh = r.hi;
  double r4 = r2.hi * r2.hi;
  double tail = r4 * (kI24 + rh * (kI120 + rh * (kI720 + rh * kI5040)));
  aos_dd half_r2 = {r2.hi * 0.5, r2.lo * 0.5};
  aos_dd u = aos_dd_add(r, half_r2);
  u = aos_dd_add(u, t3);
  aos_dd tl = {tail, 0.0};
  u = aos_dd_add(u, tl);

  /* eight squarings: (1+u)^2 = 1 + (2u + u^2) */
  for (int i = 0; i < 8; ++i) {
    aos_dd uu = aos_dd_mul(u, u);
    aos_dd u2 = {u.hi * 2.0, u.lo * 2.0};
    u = aos_dd_add(u2, uu);
  }
  aos_dd one = {1.0, 0.0};
  aos_dd e = aos_dd_add(one, u);
  double res = e.hi + e.lo;
  return ldexp(res, (int)kd);
}

#endif
