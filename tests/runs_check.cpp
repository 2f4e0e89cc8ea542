// Checks the closed forms of nls_runs.h against the plain sequential fp32
// loops they stand for (the reference's order of operations,
// src/nimllm/sampler.nim:51-57, :103-120), on random and constructed runs:
// ties to even, binade crossings, long runs, targets on and near the exact
// partial sums.  Built and run by tests/test_runs_cpu.py.
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <random>

#include "../nim.llm_amd/csrc/nls_runs.h"

static uint32_t bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

// The loops below are the definition: one rounded fp32 operation per step.
static float add_loop(float acc, float y, uint32_t c) {
  for (uint32_t i = 0; i < c; ++i) {
    volatile float t = acc + y;
    acc = t;
  }
  return acc;
}
static uint32_t add_until_loop(float& acc, float y, uint32_t c, double target) {
  for (uint32_t i = 0; i < c; ++i) {
    volatile float t = acc + y;
    acc = t;
    if ((double)acc >= target) return i + 1;
  }
  return 0;
}
static uint32_t sub_until_loop(float& r, float y, uint32_t c) {
  for (uint32_t i = 0; i < c; ++i) {
    volatile float t = r - y;
    r = t;
    if (r <= 0.0f) return i + 1;
  }
  return 0;
}

int main(int argc, char** argv) {
  const int iters = argc > 1 ? atoi(argv[1]) : 20000;
  std::mt19937_64 g(12345);
  std::uniform_real_distribution<double> U01(0.0, 1.0);
  long fails = 0, ties = 0;
  for (int it = 0; it < iters; ++it) {
    // start value and term over a wide range of ratios
    const int ex = (int)(g() % 40) - 20;
    float acc = (float)ldexp(0.5 + 0.5 * U01(g), ex);
    if (it % 7 == 0) acc = 0.0f;  // a sum's first step
    int ey = ex - (int)(g() % 30);
    float y = (float)ldexp(0.5 + 0.5 * U01(g), ey);
    if (it % 3 == 0) {
      // a term that is an odd multiple of half the spacing of acc: a tie
      double a, Uu;
      if (acc > 0.0f) {
        nls::run_binade(acc, a, Uu);
        const uint64_t m = (g() % 4096) * 2 + 1;
        y = (float)(Uu * 0.5 * (double)m);
        ++ties;
      }
    }
    if (it % 11 == 0) y = 0.0f;
    uint32_t c = (uint32_t)(g() % (it % 50 == 0 ? 3000000 : 2000)) + 1;
    // add
    {
      float ref = add_loop(acc, y, c);
      float got = acc;
      int budget = 1 << 20;
      const bool more = nls::run_add(got, y, c, budget);
      if (budget < 0) {
        fprintf(stderr, "add: budget exhausted\n");
        ++fails;
      } else if (more) {
        if (bits(got) != bits(ref)) {
          fprintf(stderr, "add mismatch acc=%a y=%a c=%u ref=%a got=%a\n", acc, y, c, ref, got);
          ++fails;
        }
      } else {
        // the run reported that acc no longer changes: the loop must agree
        if (bits(add_loop(ref, y, 5)) != bits(ref)) {
          fprintf(stderr, "add: reported stop but acc still changes acc=%a y=%a\n", acc, y);
          ++fails;
        }
        if (bits(got) != bits(ref)) {
          fprintf(stderr, "add(stop) mismatch acc=%a y=%a c=%u ref=%a got=%a\n", acc, y, c, ref, got);
          ++fails;
        }
      }
    }
    // add until a target: a target on a reachable partial sum, near it, or beyond
    {
      float full = add_loop(acc, y, c);
      double target;
      const int mode = it % 4;
      if (mode == 0) {
        float mid = add_loop(acc, y, c / 2 + 1);
        target = (double)mid;
      } else if (mode == 1) {
        float mid = add_loop(acc, y, c / 3 + 1);
        target = (double)mid + 1e-12;
      } else if (mode == 2) {
        target = (double)full * (1.0 + 1e-9) + 1e-30;
      } else {
        target = (double)acc + (double)y * (double)c * U01(g);
      }
      float r1 = acc, r2 = acc;
      const uint32_t j1 = add_until_loop(r1, y, c, target);
      int budget = 1 << 20;
      bool more;
      const uint32_t j2 = nls::run_add_until(r2, y, c, target, budget, &more);
      if (budget < 0) {
        fprintf(stderr, "add_until: budget exhausted\n");
        ++fails;
      } else if (j1 != j2 || (j1 && bits(r1) != bits(r2)) || (!j1 && more && bits(r1) != bits(r2))) {
        fprintf(stderr, "add_until mismatch acc=%a y=%a c=%u t=%.17g j %u/%u r %a/%a\n", acc, y, c,
                target, j1, j2, r1, r2);
        ++fails;
      }
    }
    // subtract until <= 0
    {
      float r0 = acc > 0.0f ? acc : (float)ldexp(0.5 + 0.5 * U01(g), ex);
      if (it % 13 == 0) r0 = 0.0f;
      float y2 = y;
      if (it % 2 == 0 && r0 > 0.0f) {
        // a term so that the run ends inside it
        y2 = (float)((double)r0 / ((double)c * (0.3 + U01(g))));
      }
      float r1 = r0, r2 = r0;
      const uint32_t j1 = sub_until_loop(r1, y2, c);
      int budget = 1 << 20;
      bool more;
      const uint32_t j2 = nls::run_sub_until(r2, y2, c, budget, &more);
      if (budget < 0) {
        fprintf(stderr, "sub: budget exhausted\n");
        ++fails;
      } else if (j1 != j2 || (j1 && bits(r1) != bits(r2)) || (!j1 && more && bits(r1) != bits(r2))) {
        fprintf(stderr, "sub mismatch r=%a y=%a c=%u j %u/%u r %a/%a\n", r0, y2, c, j1, j2, r1, r2);
        ++fails;
      }
    }
  }
  printf("runs_check: %d cases, %ld tie runs, %ld failures\n", iters, ties, fails);
  return fails ? 1 : 0;
}
