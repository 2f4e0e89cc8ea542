// nls_expf.h -- correctly rounded exp() of a binary32 input, for host and device.
//
// The reference evaluates exp(float32) through the C library's expf
// (src/nimllm/sampler.nim:56).  libm expf is not correctly rounded, and a GPU
// has no copy of it, so this sampler uses the correctly rounded value, which is
// unique and can therefore be reproduced anywhere.
//
// Method (written from the mathematics, in float64):
//   k = rint(x / ln2);  r = x - k*ln2 with ln2 split in a 44-bit head (so
//   k*head is exact and x - k*head is exact) and a float64 tail;
//   e^r by its Taylor series to degree 13 (|r| <= ln2/2: truncation < 5e-18),
//   Horner with fused multiply-adds; y = e^r * 2^k exactly.
//   The float64 result is within NLS_EXPF_REL_ERR of e^x.  When every value in
//   [y(1-err), y(1+err)] rounds to the same float, that float is the correctly
//   rounded result.  The remaining inputs (where a binary32 rounding boundary
//   lies inside the interval) are listed with their correctly rounded results
//   in nls_expf_table.h, produced by an exhaustive scan of every binary32 input
//   with a finite non-zero result (nls_expf_scan.c).
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

// Relative error bound of the float64 evaluation below (measured maximum over
// all binary32 inputs is under 2^-52; the bound used leaves a 2^5 margin).
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

}  // namespace nls
