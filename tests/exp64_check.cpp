// Checks nim.llm_amd/csrc/nls_exp64.h (the float64 exp of the row
// log-sum-exp) against the C library's exp on float32 arguments <= 0: every
// float32 in a sweep over [-746, 0], the ends of the range and the table
// boundaries.  Built and run by tests/test_runs_cpu.py.
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "../nim.llm_amd/csrc/nls_exp64.h"

int main() {
  double t[nls::kExp64Table];
  for (int j = 0; j < nls::kExp64Table; ++j) t[j] = nls::exp64_table_entry(j);
  double worst = 0.0;
  long n = 0, bad = 0;
  auto check = [&](float xf) {
    const double x = (double)xf;
    const double want = exp(x), got = nls::exp64(x, t);
    ++n;
    if (want == 0.0 || want < 1e-300) {  // underflow region: no relative bar
      if (!(got >= 0.0 && got < 1e-290)) ++bad;
      return;
    }
    const double rel = fabs(got - want) / want;
    if (rel > worst) worst = rel;
    if (!(rel <= 2e-15)) {
      if (bad < 10) fprintf(stderr, "x=%a want=%a got=%a rel=%g\n", x, want, got, rel);
      ++bad;
    }
  };
  // every 61st float32 bit pattern from -0 down to -746
  uint32_t u = 0x80000000u;
  for (;;) {
    float f;
    memcpy(&f, &u, 4);
    if (!(f >= -746.0f)) break;
    check(f);
    u += 61;
  }
  const float edges[] = {0.0f, -0.0f, -1e-30f, -0.0054f, -0.0108f, -0.69314718f, -1.0f, -87.3f,
                         -103.9f, -708.3f, -708.4f, -744.4f, -745.1f, -745.2f, -1000.0f};
  for (float f : edges) check(f);
  // every table boundary k * ln2/64 and its neighbours
  for (int k = -68800; k <= 0; k += 7) {
    const float f = (float)(k * 0.010830424696249145);
    check(f);
    check(nextafterf(f, 0.0f));
    check(nextafterf(f, -1e9f));
  }
  const bool nan_ok = isnan(nls::exp64(NAN, t)) && nls::exp64(-INFINITY, t) == 0.0;
  printf("exp64_check: %ld arguments, worst relative error %.3g, %ld failures%s\n", n, worst, bad,
         nan_ok ? "" : ", NaN/-inf wrong");
  return (bad || !nan_ok) ? 1 : 0;
}
