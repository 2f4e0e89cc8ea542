// nls_expf.h -- correctly rounded exp() of a binary32 input, for host and device.
//
// The reference evaluates exp(float32) through the C library's expf
// (src/nimllm/sampler.nim:56).  libm expf is not correctly rounded, and a GPU
// has no copy of it, so this sampler uses the correctly rounded value, which is
// unique and can therefore be reproduced anywhere.
//
// Two float64 evaluations of e^x, written from the mathematics:
//
//   expf_as_double (no table; for a few exponentials where a table read
//   would add its latency):  k = rint(x / ln2);  r = x - k*ln2 with ln2 split
//   in a 44-bit head (so k*head and x - k*head are exact) and a float64 tail;
//   e^r by its Taylor series to degree 13 (|r| <= ln2/2: truncation < 5e-18),
//   Horner with fused multiply-adds; y = e^r * 2^k exactly.
//
//   expf_as_double_t (Tang's table-driven method, ACM TOMS 15(2), 1989; for
//   whole rows, the table in LDS):  k = rint(x * 64/ln2), x = k*ln2/64 + r
//   with |r| <= ln2/128; ln2/64 split in a 36-bit head (k*head and
//   x - k*head are exact for |k| < 2^14) and a float64 tail;
//   e^x = 2^(k >> 6) * 2^((k & 63)/64) * (1 + q), the 64 powers 2^(j/64)
//   correctly rounded to float64 (computed to 60 digits) and
//   q = r + r^2 (1/2 + r/6 + r^2/24 + r^3/120) (the first omitted term,
//   r^6/720, is below 2^-54.6).
//
// Each result is within NLS_EXPF_REL_ERR of e^x.  When every value in
// [y(1-err), y(1+err)] rounds to the same float, that float is the correctly
// rounded result.  The remaining inputs (where a binary32 rounding boundary
// lies inside the interval of either evaluation) are listed with their
// correctly rounded results in nls_expf_table.h, produced by an exhaustive
// scan of every binary32 input with a finite non-zero result
// (nls_expf_scan.c++, which also checks both functions on every input).
//
// Every float64 operation here is an IEEE-754 correctly rounded +, *, fma or
// rint, so the host build and the gfx950 build return identical bits; the
// file must be compiled without fast-math.
#pragma once
#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define NLS_HD __host__ __device__
#else
#define NLS_HD
#endif

#include "nls_expf_table.h"

namespace nls {

// Relative error bound of the float64 evaluations below (measured maxima over
// all binary32 inputs: 2^-52.65 for the Taylor form, 2^-51.96 for the table
// form; the bound used leaves a margin of 2^4.9).
#define NLS_EXPF_REL_ERR 0x1p-47

NLS_HD inline double expf_as_double(float xf) {
  const double x = (double)xf;
  const double kInvLn2 = 0x1.71547652b82fep+0;
  const double kLn2Hi = 0x1.62e42fefa3800p-1;  // ln2 truncated to 44 bits
  const double kLn2Lo = 0x1.ef35793c76730p-45;  // ln2 - kLn2Hi
  const double kd = __builtin_rint(x * kInvLn2);
  double r = __builtin_fma(-kd, kLn2Hi, x);  // exact
  r = __builtin_fma(-kd, kLn2Lo, r);
  // 1/n!, n = 13 .. 0
  double p = 0x1.6124613a86d09p-33;
  p = __builtin_fma(p, r, 0x1.1eed8eff8d898p-29);
  p = __builtin_fma(p, r, 0x1.ae64567f544e4p-26);
  p = __builtin_fma(p, r, 0x1.27e4fb7789f5cp-22);
  p = __builtin_fma(p, r, 0x1.71de3a556c734p-19);
  p = __builtin_fma(p, r, 0x1.a01a01a01a01ap-16);
  p = __builtin_fma(p, r, 0x1.a01a01a01a01ap-13);
  p = __builtin_fma(p, r, 0x1.6c16c16c16c17p-10);
  p = __builtin_fma(p, r, 0x1.1111111111111p-7);
  p = __builtin_fma(p, r, 0x1.5555555555555p-5);
  p = __builtin_fma(p, r, 0x1.5555555555555p-3);
  p = __builtin_fma(p, r, 0x1.0000000000000p-1);
  p = __builtin_fma(p, r, 1.0);
  p = __builtin_fma(p, r, 1.0);
  const int k = (int)kd;
  const uint64_t two_k_bits = (uint64_t)(int64_t)(k + 1023) << 52;
  double two_k;
  memcpy(&two_k, &two_k_bits, sizeof two_k);
  return p * two_k;  // exact: p in [0.7, 1.42], 2^k a normal float64
}

// 2^(j/64), j = 0 .. 63, correctly rounded
constexpr int kExpfPow2Count = 64;
constexpr double kExpfPow2J64[kExpfPow2Count] = {
    0x1.0000000000000p+0, 0x1.02c9a3e778061p+0, 0x1.059b0d3158574p+0,
    0x1.0874518759bc8p+0, 0x1.0b5586cf9890fp+0, 0x1.0e3ec32d3d1a2p+0,
    0x1.11301d0125b51p+0, 0x1.1429aaea92de0p+0, 0x1.172b83c7d517bp+0,
    0x1.1a35beb6fcb75p+0, 0x1.1d4873168b9aap+0, 0x1.2063b88628cd6p+0,
    0x1.2387a6e756238p+0, 0x1.26b4565e27cddp+0, 0x1.29e9df51fdee1p+0,
    0x1.2d285a6e4030bp+0, 0x1.306fe0a31b715p+0, 0x1.33c08b26416ffp+0,
    0x1.371a7373aa9cbp+0, 0x1.3a7db34e59ff7p+0, 0x1.3dea64c123422p+0,
    0x1.4160a21f72e2ap+0, 0x1.44e086061892dp+0, 0x1.486a2b5c13cd0p+0,
    0x1.4bfdad5362a27p+0, 0x1.4f9b2769d2ca7p+0, 0x1.5342b569d4f82p+0,
    0x1.56f4736b527dap+0, 0x1.5ab07dd485429p+0, 0x1.5e76f15ad2148p+0,
    0x1.6247eb03a5585p+0, 0x1.6623882552225p+0, 0x1.6a09e667f3bcdp+0,
    0x1.6dfb23c651a2fp+0, 0x1.71f75e8ec5f74p+0, 0x1.75feb564267c9p+0,
    0x1.7a11473eb0187p+0, 0x1.7e2f336cf4e62p+0, 0x1.82589994cce13p+0,
    0x1.868d99b4492edp+0, 0x1.8ace5422aa0dbp+0, 0x1.8f1ae99157736p+0,
    0x1.93737b0cdc5e5p+0, 0x1.97d829fde4e50p+0, 0x1.9c49182a3f090p+0,
    0x1.a0c667b5de565p+0, 0x1.a5503b23e255dp+0, 0x1.a9e6b5579fdbfp+0,
    0x1.ae89f995ad3adp+0, 0x1.b33a2b84f15fbp+0, 0x1.b7f76f2fb5e47p+0,
    0x1.bcc1e904bc1d2p+0, 0x1.c199bdd85529cp+0, 0x1.c67f12e57d14bp+0,
    0x1.cb720dcef9069p+0, 0x1.d072d4a07897cp+0, 0x1.d5818dcfba487p+0,
    0x1.da9e603db3285p+0, 0x1.dfc97337b9b5fp+0, 0x1.e502ee78b3ff6p+0,
    0x1.ea4afa2a490dap+0, 0x1.efa1bee615a27p+0, 0x1.f50765b6e4540p+0,
    0x1.fa7c1819e90d8p+0,
};

// The table form; pow2 holds kExpfPow2J64 (a copy in LDS on the device).
NLS_HD inline double expf_as_double_t(float xf, const double* pow2) {
  const double x = (double)xf;
  const double kInvStep = 0x1.71547652b82fep+6;  // 64 / ln2
  const double kStepHi = 0x1.62e42fefa0000p-7;   // ln2 / 64, leading 36 bits
  const double kStepLo = 0x1.cf79abc9e3b3ap-46;  // ln2 / 64 - kStepHi
  const double kd = __builtin_rint(x * kInvStep);
  double r = __builtin_fma(-kd, kStepHi, x);  // exact
  r = __builtin_fma(-kd, kStepLo, r);
  const int k = (int)kd;
  double u = __builtin_fma(0x1.1111111111111p-7, r, 0x1.5555555555555p-5);  // 1/120, 1/24
  u = __builtin_fma(u, r, 0x1.5555555555555p-3);                            // 1/6
  u = __builtin_fma(u, r, 0.5);
  const double q = __builtin_fma(u, r * r, r);
  const double t = pow2[k & (kExpfPow2Count - 1)];
  const uint64_t two_m_bits = (uint64_t)(int64_t)((k >> 6) + 1023) << 52;  // k >> 6 = floor(k / 64)
  double two_m;
  memcpy(&two_m, &two_m_bits, sizeof two_m);
  return __builtin_fma(t, q, t) * two_m;  // exact scaling: a normal float64
}

// 0 when the float64 evaluation alone decides the rounding, 1 otherwise.
NLS_HD inline int expf_is_hard(double y) {
  const float lo = (float)(y * (1.0 - NLS_EXPF_REL_ERR));
  const float hi = (float)(y * (1.0 + NLS_EXPF_REL_ERR));
  return lo != hi;
}

NLS_HD inline float expf_hard_lookup(float x, float fallback) {
  uint32_t bits;
  memcpy(&bits, &x, sizeof bits);
  int lo = 0, hi = NLS_EXPF_HARD_COUNT - 1;
  while (lo <= hi) {
    const int mid = (lo + hi) >> 1;
    const uint32_t key = kExpfHardInputs[mid];
    if (key == bits) {
      const uint32_t rb = kExpfHardResults[mid];
      float res;
      memcpy(&res, &rb, sizeof res);
      return res;
    }
    if (key < bits)
      lo = mid + 1;
    else
      hi = mid - 1;
  }
  return fallback;
}

// Correctly rounded e^x for binary32 x.
NLS_HD inline float expf_cr(float x) {
  if (!(x > -104.0f)) {            // exp(-104) < 2^-150: rounds to +0
    return (x != x) ? x + x : 0.0f;  // NaN propagates
  }
  if (x > 89.0f) return __builtin_inff();
  const double y = expf_as_double(x);
  const float f = (float)y;
  if (expf_is_hard(y)) return expf_hard_lookup(x, f);
  return f;
}

// The same value through the table form (pow2 as for expf_as_double_t).
NLS_HD inline float expf_cr_t(float x, const double* pow2) {
  if (!(x > -104.0f)) {
    return (x != x) ? x + x : 0.0f;
  }
  if (x > 89.0f) return __builtin_inff();
  const double y = expf_as_double_t(x, pow2);
  const float f = (float)y;
  if (expf_is_hard(y)) return expf_hard_lookup(x, f);
  return f;
}

}  // namespace nls
