// nls_exp64.h -- float64 exp for the row log-sum-exp of perplexity's
// per-position term (src/nimllm/model.nim:581: exp(float(l - mx)), l - mx a
// float32 <= 0).
//
// Tang's table-driven method (ACM TOMS 15(2), 1989): x = (64 m + j) ln2/64 + r
// with |r| <= ln2/128, exp(x) = 2^m * 2^(j/64) * (1 + p(r)), where p is the
// degree-5 Taylor polynomial of e^r - 1 (the first omitted term, r^6/720, is
// below 4e-17).  ln2/64 is split Cody-Waite style into a 36-bit head, so that
// k * head is exact for |k| < 2^17, and the rest; both come from ln 2 taken to
// 60 digits.  The 64 entries 2^(j/64) are computed once per workgroup with the
// library's exp2.  The result is within a few ulps of exp(x): the kernel's
// parity bar is float64 rounding of the sum (relative 1e-12), and the function
// is checked against the C library on the CPU (tests/test_runs_cpu.py).
#pragma once
#include <math.h>

#if defined(__HIPCC__) || defined(__HIP__)
#define NLS_E64 __host__ __device__ __forceinline__
#else
#define NLS_E64 static inline
#endif

namespace nls {

constexpr int kExp64Table = 64;
constexpr double kExp64InvStep = 0x1.71547652b82fep+6;   // 64 / ln 2
constexpr double kExp64StepHi = 0x1.62e42fefa0000p-7;    // ln 2 / 64, leading 36 bits
constexpr double kExp64StepLo = 0x1.cf79abc9e3b3ap-46;   // ln 2 / 64 - kExp64StepHi

NLS_E64 double exp64_table_entry(int j) { return exp2((double)j / kExp64Table); }

// exp(x) for x <= 0 (larger x and NaN go to the library); t[j] = 2^(j/64).
NLS_E64 double exp64(double x, const double* t) {
  if (x != x || x > 0.0) return exp(x);
  if (x < -745.5) return 0.0;  // below half the smallest subnormal
  const double kf = rint(x * kExp64InvStep);
  const int k = (int)kf;  // |k| < 2^17
  const double r = (x - kf * kExp64StepHi) - kf * kExp64StepLo;
  const double p = r + r * r * (0.5 + r * (1.0 / 6.0 + r * (1.0 / 24.0 + r * (1.0 / 120.0))));
  const double tj = t[k & (kExp64Table - 1)];
  return ldexp(tj + tj * p, k >> 6);  // k >> 6 = floor(k / 64)
}

}  // namespace nls
