// nls_runs.h -- exact closed forms of a run of equal terms in a sequential
// IEEE binary32 (round to nearest, ties to even) sum or difference.
//
// The reference's sort path adds and subtracts its candidates one at a time
// in candidate order (src/nimllm/sampler.nim:51-57 for the softmax sum,
// :103-108 top-p, :115-116 total, :117-120 the draw).  Candidates of equal
// value are adjacent in that order and contribute equal terms, so a run of c
// equal terms can be applied in closed form instead of c dependent adds:
//
//   Let x > 0 lie in the binade [2^(k-1), 2^k); its spacing there is
//   U = 2^(k-24) and x = a*U with a an integer in [2^23, 2^24).  For a term
//   y >= 0 put d = y/U (exact: a power-of-two scaling).
//   * x + y: while a + d < 2^24 the exact sum lies inside the binade (or
//     rounds up to its end 2^k), so the rounded sum is (a + R(d))*U, where
//     R rounds d to the nearest integer.  When d has fraction exactly 1/2
//     the tie goes to the even neighbour: the result a' is even.  Once a is
//     even every later tie adds q = floor(d) rounded up to even, and a stays
//     even.
//   * x - y: the same with a - R(d) while a - d >= 2^23.
//   So a run needs one real add per binade crossing and per entry into a
//   tie, and plain integer arithmetic in between.  Every step that the closed
//   form does not cover is the hardware's own fp32 operation.
//
// The closed forms run in 32-bit integers and exact float operations: a, the
// integer part of d and the step q are integers below 2^25, d = y * 2^(24-k)
// is an exact power-of-two scaling of y (it only matters when 1/2 <= d <
// 2^24), and d's fraction is exact.  The number of steps that stay in the
// binade comes from the integer inequalities below, so no step is rounded
// differently from the sequential loop.
#pragma once
#include <math.h>
#include <stdint.h>

#if defined(__HIPCC__) || defined(__HIP__)
#define NLS_RD __host__ __device__ __forceinline__
#else
#define NLS_RD static inline
#endif

namespace nls {

// x = a * U with a in [2^23, 2^24) for a positive normal x; returns k with
// U = 2^(k-24).  The scalings are exact (ldexp by a power of two).
NLS_RD int run_binade(float x, double& a, double& U) {
  int k;
  (void)frexpf(x, &k);  // x = m * 2^k, m in [1/2, 1)
  U = ldexp(1.0, k - 24);
  a = ldexp((double)x, 24 - k);
  return k;
}

NLS_RD bool run_fast_ok(float x) {
  // positive, normal, and not in the top binade (whose end 2^128 overflows)
  return x >= 0x1p-125f && x < 0x1p126f;
}

// The integer form of x (positive, normal): x = a * 2^(k-24), a in
// [2^23, 2^24); returns k.
NLS_RD int run_split(float x, int32_t& a) {
  int k;
  const float m = frexpf(x, &k);  // m in [1/2, 1)
  a = (int32_t)ldexpf(m, 24);
  return k;
}

// One step of a run in units of the spacing: y / 2^(k-24) = fl + fr with fl
// an integer and fr in [0, 1).  Returns false when y is at least 2^24 units
// (the step leaves the binade at once).
NLS_RD bool run_units(float y, int k, int32_t& fl, float& fr) {
  const float d = ldexpf(y, 24 - k);  // exact, or 0 / subnormal when tiny
  if (!(d < 0x1p24f)) return false;
  const float f = floorf(d);
  fl = (int32_t)f;
  fr = d - f;  // exact
  return true;
}

// Per-step integer change of the closed form: the rounded d (ties to the
// even result, given an even a), or -1 when the step must be a real
// operation (an odd a facing a tie).
NLS_RD int32_t run_step(int32_t a, int32_t fl, float fr) {
  if (fr != 0.5f) return fr > 0.5f ? fl + 1 : fl;
  if (a & 1) return -1;
  return (fl & 1) ? fl + 1 : fl;
}

// floor(n / q) for 0 <= n < 2^26 and 1 <= q < 2^26.
NLS_RD int32_t run_div(int32_t n, int32_t q) {
  int32_t t = (int32_t)((float)n / (float)q);  // within one of the answer
  while (t > 0 && t * q > n) --t;
  while ((t + 1) * q <= n) ++t;
  return t;
}

// Steps (1-based j) that stay on the binade's grid when adding: a + (j-1)q +
// fl + fr < 2^24, which for integer (j-1)q is (j-1)q <= 2^24 - a - fl - 1.
NLS_RD int32_t run_steps_add(int32_t a, int32_t fl, int32_t q) {
  const int32_t D = (1 << 24) - a - fl;
  return D >= 1 ? run_div(D - 1, q) + 1 : 0;
}

// Steps that stay in the binade when subtracting: a - (j-1)q - fl - fr >=
// 2^23, i.e. (j-1)q <= a - fl - 2^23, less one when fr > 0.
NLS_RD int32_t run_steps_sub(int32_t a, int32_t fl, float fr, int32_t q) {
  const int32_t E = a - fl - (1 << 23) - (fr > 0.0f ? 1 : 0);
  return E >= 0 ? run_div(E, q) + 1 : 0;
}

// acc <- fl(acc + y), c times (acc >= 0, y >= 0).  Returns false when the
// sum can no longer change for this y or any smaller term (y < half the
// spacing of acc, or a tie that keeps acc), so that the caller may stop.
// `budget` counts the real operations; the run gives up (returns true with
// budget < 0) when it is exhausted.
NLS_RD bool run_add(float& acc, float y, uint32_t c, int& budget) {
  while (c > 0) {
    if (!(y > 0.0f)) return y == 0.0f ? false : true;  // +0 leaves acc; NaN is not handled here
    if (!run_fast_ok(acc)) {
      if (--budget < 0) return true;
      acc = acc + y;
      --c;
      continue;
    }
    if (c == 1) {  // one real add; an add that leaves acc means no smaller term moves it
      if (--budget < 0) return true;
      const float nx = acc + y;
      const bool moved = nx != acc;
      acc = nx;
      return moved;
    }
    int32_t a, fl;
    float fr;
    const int k = run_split(acc, a);
    int32_t t = 0;
    if (run_units(y, k, fl, fr)) {
      if (fl == 0 && fr < 0.5f) return false;  // d < 1/2
      const int32_t q = run_step(a, fl, fr);
      if (q == 0) return false;  // ties that keep an even acc
      if (q > 0) {
        t = run_steps_add(a, fl, q);
        if ((uint32_t)t > c) t = (int32_t)c;
      }
      if (t >= 1) {
        a += t * q;
        acc = ldexpf((float)a, k - 24);
        c -= (uint32_t)t;
        continue;
      }
    }
    if (--budget < 0) return true;
    acc = acc + y;
    --c;
  }
  return true;
}

// As run_add, stopping at the first step j (1-based) after which
// (double)acc >= target; returns j, or 0 when no step of the run reaches it
// (then *more reports whether acc can still change).
NLS_RD uint32_t run_add_until(float& acc, float y, uint32_t c, double target, int& budget,
                              bool* more) {
  uint32_t done = 0;
  *more = true;
  while (done < c) {
    if (y == 0.0f) {  // acc + 0 == acc: every step gives the same answer
      *more = false;
      return (double)acc >= target ? done + 1 : 0;
    }
    if (!(y > 0.0f) || !run_fast_ok(acc)) {
      if (--budget < 0) return 0;
      acc = acc + y;
      ++done;
      if ((double)acc >= target) return done;
      continue;
    }
    if (c - done == 1) {
      if (--budget < 0) return 0;
      const float nx = acc + y;
      *more = nx != acc;
      acc = nx;
      return (double)acc >= target ? done + 1 : 0;
    }
    int32_t a, fl;
    float fr;
    const int k = run_split(acc, a);
    int32_t t = 0, q = 1;
    if (run_units(y, k, fl, fr)) {
      q = (fl == 0 && fr < 0.5f) ? 0 : run_step(a, fl, fr);
      if (q == 0) {
        *more = false;
        return (double)acc >= target ? done + 1 : 0;
      }
      if (q > 0) {
        t = run_steps_add(a, fl, q);
        if ((uint32_t)t > c - done) t = (int32_t)(c - done);
      }
    }
    if (t >= 1) {
      // (double)acc >= target after step j  <=>  a + j q >= target / U, an
      // exact scaling; a + j q is an integer, so against its ceiling C
      const double C = ceil(ldexp(target, 24 - k));
      if ((double)(a + t * q) >= C) {
        int32_t j = 1;
        const int32_t need = (int32_t)C - a;  // C <= a + t q < 2^26 here
        if (need > q) j = run_div(need - 1, q) + 1;
        acc = ldexpf((float)(a + j * q), k - 24);
        return done + (uint32_t)j;
      }
      a += t * q;
      acc = ldexpf((float)a, k - 24);
      done += (uint32_t)t;
    } else {
      if (--budget < 0) return 0;
      acc = acc + y;
      ++done;
      if ((double)acc >= target) return done;
    }
  }
  return 0;
}

// r <- fl(r - y), c times, stopping at the first step j (1-based) after which
// r <= 0; returns j, or 0 when no step of the run gets there (then *more
// reports whether r can still change).  r > 0, y >= 0.
NLS_RD uint32_t run_sub_until(float& r, float y, uint32_t c, int& budget, bool* more) {
  uint32_t done = 0;
  *more = true;
  while (done < c) {
    if (y == 0.0f) {  // r - 0 == r
      *more = false;
      return r <= 0.0f ? done + 1 : 0;
    }
    if (!(y > 0.0f) || !run_fast_ok(r)) {
      if (--budget < 0) return 0;
      r = r - y;
      ++done;
      if (r <= 0.0f) return done;
      continue;
    }
    if (c - done == 1) {
      if (--budget < 0) return 0;
      const float nx = r - y;
      *more = nx != r;
      r = nx;
      return r <= 0.0f ? done + 1 : 0;
    }
    int32_t a, fl;
    float fr;
    const int k = run_split(r, a);
    int32_t t = 0, q = 1;
    if (run_units(y, k, fl, fr)) {
      q = (fl == 0 && fr < 0.5f) ? 0 : run_step(a, fl, fr);
      if (q == 0) {
        *more = false;
        return 0;
      }
      if (q > 0) {
        // every step inside the binade leaves r >= 2^(k-1) > 0
        t = run_steps_sub(a, fl, fr, q);
        if ((uint32_t)t > c - done) t = (int32_t)(c - done);
      }
    }
    if (t >= 1) {
      a -= t * q;
      r = ldexpf((float)a, k - 24);
      done += (uint32_t)t;
    } else {
      if (--budget < 0) return 0;
      r = r - y;
      ++done;
      if (r <= 0.0f) return done;
    }
  }
  return 0;
}

}  // namespace nls
