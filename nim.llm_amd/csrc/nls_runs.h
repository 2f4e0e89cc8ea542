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
// All arithmetic on a, d and U is exact in binary64: a < 2^25 is an integer
// and d carries at most 24 significant bits at or above 2^-25 when it matters
// (d >= 1/2), so every sum used below fits in 53 bits.
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

// Per-step integer change of the closed form, or -1 when the next step must
// be taken as a real operation (an odd a facing a tie).  d >= 1/2.
NLS_RD double run_step_q(double a, double d) {
  const double fl = floor(d);
  const double fr = d - fl;
  if (fr != 0.5) return fr > 0.5 ? fl + 1.0 : fl;
  if (fmod(a, 2.0) != 0.0) return -1.0;
  return fmod(fl, 2.0) == 0.0 ? fl : fl + 1.0;
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
    double a, U;
    const int k = run_binade(acc, a, U);
    const double d = ldexp((double)y, 24 - k);
    if (d < 0.5) return false;
    const double q = run_step_q(a, d);
    if (q == 0.0) return false;  // ties that keep an even acc
    double t = 0.0;
    if (q > 0.0) {
      // step j (1-based) stays on this binade's grid iff a + (j-1)q + d < 2^24
      const double lim = 0x1p24 - a - d;
      if (lim > 0.0) {
        t = floor(lim / q) + 1.0;
        while (t > 0.0 && !(a + (t - 1.0) * q + d < 0x1p24)) t -= 1.0;
        while (a + t * q + d < 0x1p24) t += 1.0;
        if (t > (double)c) t = (double)c;
      }
    }
    if (t >= 1.0) {
      a += t * q;
      acc = (float)(a * U);
      c -= (uint32_t)t;
    } else {
      if (--budget < 0) return true;
      acc = acc + y;
      --c;
    }
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
    double a, U;
    const int k = run_binade(acc, a, U);
    const double d = ldexp((double)y, 24 - k);
    const double q = d < 0.5 ? 0.0 : run_step_q(a, d);
    if (q == 0.0) {
      *more = false;
      return (double)acc >= target ? done + 1 : 0;
    }
    double t = 0.0;
    if (q > 0.0) {
      const double lim = 0x1p24 - a - d;
      if (lim > 0.0) {
        t = floor(lim / q) + 1.0;
        while (t > 0.0 && !(a + (t - 1.0) * q + d < 0x1p24)) t -= 1.0;
        while (a + t * q + d < 0x1p24) t += 1.0;
        const double left = (double)(c - done);
        if (t > left) t = left;
      }
    }
    if (t >= 1.0) {
      // the first j <= t with (a + j q) U >= target, if any
      if ((a + t * q) * U >= target) {
        double j = ceil((ldexp(target, 24 - k) - a) / q);
        if (j < 1.0) j = 1.0;
        if (j > t) j = t;
        while (j > 1.0 && (a + (j - 1.0) * q) * U >= target) j -= 1.0;
        while (!((a + j * q) * U >= target)) j += 1.0;
        acc = (float)((a + j * q) * U);
        return done + (uint32_t)j;
      }
      a += t * q;
      acc = (float)(a * U);
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
    double a, U;
    const int k = run_binade(r, a, U);
    const double d = ldexp((double)y, 24 - k);
    const double q = d < 0.5 ? 0.0 : run_step_q(a, d);
    if (q == 0.0) {
      *more = false;
      return 0;
    }
    double t = 0.0;
    if (q > 0.0) {
      // step j stays in the binade (and so positive) iff a - (j-1)q - d >= 2^23
      const double lim = a - d - 0x1p23;
      if (lim >= 0.0) {
        t = floor(lim / q) + 1.0;
        while (t > 0.0 && !(a - (t - 1.0) * q - d >= 0x1p23)) t -= 1.0;
        while (a - t * q - d >= 0x1p23) t += 1.0;
        const double left = (double)(c - done);
        if (t > left) t = left;
      }
    }
    if (t >= 1.0) {
      a -= t * q;
      r = (float)(a * U);
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
