// Host build of nim.llm_amd/csrc/nls_expf.h (the correctly rounded exp of a
// binary32 input that every sampler kernel uses) as a small shared library,
// so tests/test_expf_mpmath.py can check it against high-precision values.
// The same header is compiled as device code; every operation in it is a
// correctly rounded IEEE-754 float64 operation, so the bits are the same.
#include <stdint.h>
#include <string.h>

#include "../nim.llm_amd/csrc/nls_expf.h"

extern "C" {

// out_cr[i] = expf_cr(x[i]), out_t[i] = expf_cr_t(x[i]) (the table form),
// raw_d[i] = expf_as_double(x[i]), raw_t[i] = expf_as_double_t(x[i]) for
// x[i] in (-104, 89] (0 elsewhere).
void expf_batch(const float* x, int64_t n, float* out_cr, float* out_t, double* raw_d,
                double* raw_t) {
  for (int64_t i = 0; i < n; ++i) {
    out_cr[i] = nls::expf_cr(x[i]);
    out_t[i] = nls::expf_cr_t(x[i], nls::kExpfPow2J64);
    const bool in = x[i] > -104.0f && x[i] <= 89.0f;
    raw_d[i] = in ? nls::expf_as_double(x[i]) : 0.0;
    raw_t[i] = in ? nls::expf_as_double_t(x[i], nls::kExpfPow2J64) : 0.0;
  }
}

// 1 when the float64 evaluation alone decides the rounding of y
int expf_decided(double y) { return !nls::expf_is_hard(y); }

int64_t pow2_table(double* out) {
  for (int j = 0; j < nls::kExpfPow2Count; ++j) out[j] = nls::kExpfPow2J64[j];
  return nls::kExpfPow2Count;
}

// The hard-case table; with null pointers only its length.
int64_t hard_table(uint32_t* inputs, uint32_t* results) {
  if (!inputs || !results) return NLS_EXPF_HARD_COUNT;
  memcpy(inputs, nls::kExpfHardInputs, sizeof nls::kExpfHardInputs);
  memcpy(results, nls::kExpfHardResults, sizeof nls::kExpfHardResults);
  return NLS_EXPF_HARD_COUNT;
}

double rel_err_bound() { return NLS_EXPF_REL_ERR; }
}
