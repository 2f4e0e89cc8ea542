// nls_grouped.h -- the sort path of `sample` (src/nimllm/sampler.nim:96-121)
// replayed over groups of equal values instead of the sorted row.
//
// On the sort path the candidates are the whole row in stable descending
// order (:97), and every later step is a sequential fp32 chain over that
// order: the softmax sum (:51-57), the top-p running sum (:103-108), the
// total (:115-116) and the draw (:117-120).  Candidates of equal value sit
// next to each other and contribute equal terms, so each chain can be run
// over the distinct values in descending order, each with its multiplicity,
// using the exact run closed forms of nls_runs.h.
//
// Which groups are needed.  The first candidate is the maximum, whose
// exp(l - mx) is exactly 1, so the softmax sum s is at least 1 and a term
// below 2^-24 never changes it.  A value with fl(v - mx) < kGroupFloor has
// exp below 2^-25, so the groups hold every value at or above that floor
// (`complete` says whether they hold the whole row).  The later chains need
// groups only up to the candidate where they end; when a chain would need
// candidates past the groups of an incomplete table, the walk reports
// kGroupNeedAll and the caller takes the whole-row path instead.
#pragma once
#include <stdint.h>

#include "nls_runs.h"
#if defined(__HIP_DEVICE_COMPILE__)
#include "nls_primitives.h"  // wave_incl_scan
#endif

namespace nls {

constexpr float kGroupFloor = -17.5f;  // expf(-17.5) < 2^-25
constexpr int kGroupBudget = 1 << 16;  // real fp32 operations allowed per chain

enum GroupStatus : int32_t { kGroupOk = 0, kGroupNeedAll = 1, kGroupBudgetOut = 2 };

// ---- look-ahead over groups --------------------------------------------
// Starting at group g with the running value acc, the groups whose whole run
// stays on acc's binade grid with no tie can be applied together: each adds
// (or takes away) c_h * q_h spacings, q_h = R(y_h / U), so the running value
// after them is a prefix sum of integers.  group_skip applies the longest
// such stretch of groups [g, g + m) and returns m; the group where it stops
// (a binade crossing, a tie, a term below half a spacing, the target reached,
// the count cap passed) is left to the run closed forms, one group at a time.
// The stretch is found 64 groups at a time: on the device every lane of the
// calling wave takes one group (the wave must be converged and its values
// uniform), on the host a loop stands in for the lanes.
//   SUB = false: acc += y (runs of run_add / run_add_until); with has_target,
//                stops at the group where (double)acc first reaches target.
//   SUB = true:  acc -= y (runs of run_sub_until); acc stays >= 2^(k-1) > 0.
// *skipped gets the candidates of the applied groups; their sum may not pass
// `cap`.
constexpr int kSkipLanes = 64;

// One group against binade k: its step q (in spacings), integer part fl and
// fraction fr of y / U; false when the group needs the closed forms (y not
// positive, y / U below 1/2 or at least 2^24, or a tie).
NLS_RD bool skip_setup(float y, int k, int32_t& q, int32_t& fl, float& fr) {
  if (!(y > 0.0f)) return false;
  if (!run_units(y, k, fl, fr)) return false;
  if (fl == 0 && fr < 0.5f) return false;
  if (fr == 0.5f) return false;
  q = fr > 0.5f ? fl + 1 : fl;
  return true;
}

// Whether group h, whose run ends at integer position E = A + P (adds) or
// A - P (subtractions) after P spacings in all, stays on the grid.
template <bool SUB>
NLS_RD bool skip_stays(double A, double P, int32_t q, int32_t fl, float fr, bool has_target,
                       double target, double U) {
  if (!SUB) {
    // last step: a_h + (c - 1) q + fl + fr < 2^24 with a_h + c q = A + P
    if (!(A + P - q + fl < 0x1p24)) return false;
    return !(has_target && (A + P) * U >= target);
  }
  // last step: a_h - (c - 1) q - fl - fr >= 2^23
  return A - P + q - fl - (fr > 0.0f ? 1 : 0) >= 0x1p23;
}

// On the device the window's step totals are 32-bit integers: a group's c * q
// is clamped to 2^25 - 1, so the 64 lanes' sum stays below 2^31.  A group
// whose c * q reaches the clamp fails its stay test whatever the value (its
// run alone spans at least 2^24 spacings), so only groups after the stopping
// one ever see a clamped total.
constexpr int32_t kSkipClamp = (1 << 25) - 1;

template <bool SUB>
NLS_RD int group_skip(float& acc, const float* y, const uint32_t* c, int g, int gend, bool has_target,
                      double target, int64_t cap, int64_t* skipped) {
  *skipped = 0;
  if (g >= gend || !run_fast_ok(acc)) return 0;
  int32_t a0;
  const int k = run_split(acc, a0);
  const double U = ldexp(1.0, k - 24);
  double A = (double)a0, S = 0.0;
  int done = 0;
  for (int base = g; base < gend; base += kSkipLanes) {
    const int nv = gend - base < kSkipLanes ? gend - base : kSkipLanes;
    int m = nv;
    double Pm = 0.0, Sm = 0.0;
#if defined(__HIP_DEVICE_COMPILE__)
    {
      const int lane = (int)(threadIdx.x & (kSkipLanes - 1));
      const bool valid = lane < nv;
      const float yh = valid ? y[base + lane] : 0.0f;
      const uint32_t ch = valid ? c[base + lane] : 0u;
      int32_t q = 0, fl = 0;
      float fr = 0.0f;
      bool ok = valid && skip_setup(yh, k, q, fl, fr);
      const int64_t cq = ok ? (int64_t)ch * q : 0;
      const int32_t P = wave_incl_scan((int32_t)(cq < kSkipClamp ? cq : kSkipClamp));
      const int32_t Sc = wave_incl_scan((int32_t)ch);  // a row's counts: below 2^31
      if (ok) ok = skip_stays<SUB>(A, (double)P, q, fl, fr, has_target, target, U) && S + Sc <= (double)cap;
      const uint64_t bad = __ballot(valid && !ok);
      if (bad) m = __ffsll((unsigned long long)bad) - 1;
      if (m > 0) {
        Pm = (double)__shfl(P, m - 1, kSkipLanes);
        Sm = (double)__shfl(Sc, m - 1, kSkipLanes);
      }
    }
#else
    {
      double P = 0.0, Sc = 0.0;
      for (int l = 0; l < nv; ++l) {
        int32_t q = 0, fl = 0;
        float fr = 0.0f;
        bool ok = skip_setup(y[base + l], k, q, fl, fr);
        P += ok ? (double)c[base + l] * (double)q : 0.0;
        Sc += (double)c[base + l];
        if (ok) ok = skip_stays<SUB>(A, P, q, fl, fr, has_target, target, U) && S + Sc <= (double)cap;
        if (!ok) {
          m = l;
          break;
        }
        Pm = P;
        Sm = Sc;
      }
    }
#endif
    A = SUB ? A - Pm : A + Pm;
    S += Sm;
    done += m;
    if (m < nv) break;
  }
  if (done > 0) acc = ldexpf((float)A, k - 24);
  *skipped = (int64_t)S;
  return done;
}

// The candidates the groups hold, sum of gc[0..G) (on the device the calling
// wave adds 64 groups per step).
NLS_RD int64_t group_count_sum(const uint32_t* gc, int G) {
  int64_t held = 0;
#if defined(__HIP_DEVICE_COMPILE__)
  const int lane = (int)(threadIdx.x & (kSkipLanes - 1));
  for (int base = 0; base < G; base += kSkipLanes) {
    double c = base + lane < G ? (double)gc[base + lane] : 0.0;
#pragma unroll
    for (int o = kSkipLanes / 2; o > 0; o >>= 1) c += __shfl_xor(c, o, kSkipLanes);
    held += (int64_t)c;
  }
#else
  for (int g = 0; g < G; ++g) held += gc[g];
#endif
  return held;
}

// s = the softmax sum (:55-56) over the groups' exponentials ge[] (group g
// repeated gc[g] times), in order.  Returns false when the budget ran out.
NLS_RD bool group_sum(const float* ge, const uint32_t* gc, int G, float& s) {
  float acc = 0.0f;
  int budget = kGroupBudget;
  int64_t sk;
  for (int g = 0; g < G; ++g) {
    g += group_skip<false>(acc, ge, gc, g, G, false, 0.0, INT64_MAX, &sk);
    if (g >= G) break;
    const bool more = run_add(acc, ge[g], gc[g], budget);
    if (budget < 0) return false;
    if (!more) break;
  }
  s = acc;
  return true;
}

struct GroupDraw {
  int32_t status;  // GroupStatus
  int64_t pos;     // drawn candidate position (0-based, in sorted order)
  int64_t n;       // candidates kept after top-p and min-p
  float total;     // fp32 sum of the first n probabilities (:115-116)
};

// Top-p, min-p, total and the draw (:101-121) over the groups'
// probabilities pg[] (pg[g] = ge[g] / s), group g holding gc[g] candidates.
NLS_RD GroupDraw group_cut_draw(const float* pg, const uint32_t* gc, int G, bool complete,
                                int64_t V, bool topp_active, double topP, bool minp_active,
                                float minP32, double u) {
  GroupDraw out;
  out.status = kGroupOk;
  out.pos = 0;
  out.n = V;
  out.total = 0.0f;
  int budget = kGroupBudget;
  int64_t n = V;
  // The total (:115-116) adds the same probabilities in the same order from
  // the same 0 as the top-p running sum: where top-p sets n and min-p keeps
  // it, the running sum at the cut is the total.
  bool cut_sum = false;
  float cum_at_cut = 0.0f;
  // top-p (:103-108): n = first i + 1 with (double)cum >= topP
  if (topp_active) {
    float cum = 0.0f;
    int64_t pos = 0;
    bool found = false, more = true;
    for (int g = 0; g < G; ++g) {
      int64_t sk;
      g += group_skip<false>(cum, pg, gc, g, G, true, topP, INT64_MAX, &sk);
      pos += sk;
      if (g >= G) break;
      const uint32_t j = run_add_until(cum, pg[g], gc[g], topP, budget, &more);
      if (budget < 0) {
        out.status = kGroupBudgetOut;
        return out;
      }
      if (j) {
        n = pos + j;
        found = true;
        cut_sum = true;
        cum_at_cut = cum;
        break;
      }
      pos += gc[g];
      if (!more) break;  // cum stays below topP for every later candidate
    }
    if (!found && more && !complete) {
      out.status = kGroupNeedAll;
      return out;
    }
  }
  // min-p (:110-114): m = 1; while m < n and probs[m] >= thr: m++
  if (minp_active) {
    const float thr = pg[0] * minP32;
    int64_t cnt = 0;
    bool ended = false;
    for (int g = 0; g < G; ++g) {
      if (pg[g] >= thr) {
        cnt += gc[g];
      } else {
        ended = true;
        break;
      }
    }
    if (!ended && !complete && cnt < n) {
      out.status = kGroupNeedAll;
      return out;
    }
    int64_t m = cnt < 1 ? 1 : cnt;
    if (m < n) {
      n = m;
      cut_sum = false;
    }
  }
  // total (:115-116) over the first n candidates
  float total = 0.0f;
  if (cut_sum) {
    total = cum_at_cut;
  } else {
    int64_t pos = 0;
    bool more = true;
    for (int g = 0; g < G && pos < n; ++g) {
      int64_t sk;
      g += group_skip<false>(total, pg, gc, g, G, false, 0.0, n - pos, &sk);
      pos += sk;
      if (g >= G || pos >= n) break;
      const int64_t left = n - pos;
      const uint32_t c = (int64_t)gc[g] < left ? gc[g] : (uint32_t)left;
      more = run_add(total, pg[g], c, budget);
      if (budget < 0) {
        out.status = kGroupBudgetOut;
        return out;
      }
      pos += c;
      if (!more) break;
    }
    if (pos < n && more && !complete) {
      out.status = kGroupNeedAll;
      return out;
    }
  }
  // the draw (:117-121): r = f32(u) * total; r -= probs[i] until r <= 0
  float r = (float)u * total;
  int64_t hit = -1;
  {
    int64_t pos = 0;
    for (int g = 0; g < G && pos < n; ++g) {
      int64_t sk;
      if (r > 0.0f) {
        g += group_skip<true>(r, pg, gc, g, G, false, 0.0, n - pos, &sk);
        pos += sk;
      }
      if (g >= G || pos >= n) break;
      const int64_t left = n - pos;
      const uint32_t c = (int64_t)gc[g] < left ? gc[g] : (uint32_t)left;
      bool more = true;
      const uint32_t j = run_sub_until(r, pg[g], c, budget, &more);
      if (budget < 0) {
        out.status = kGroupBudgetOut;
        return out;
      }
      if (j) {
        hit = pos + j - 1;
        break;
      }
      pos += c;
      if (!more) break;  // r stays positive: the last candidate is drawn
    }
  }
  if (hit < 0) hit = n - 1;  // (:121)
  // the drawn candidate must lie inside the groups
  const int64_t held = complete ? V : group_count_sum(gc, G);
  if (hit >= held) {
    out.status = kGroupNeedAll;
    return out;
  }
  out.pos = hit;
  out.n = n;
  out.total = total;
  return out;
}

}  // namespace nls
