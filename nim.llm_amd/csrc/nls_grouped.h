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

namespace nls {

constexpr float kGroupFloor = -17.5f;  // expf(-17.5) < 2^-25
constexpr int kGroupBudget = 1 << 16;  // real fp32 operations allowed per chain

enum GroupStatus : int32_t { kGroupOk = 0, kGroupNeedAll = 1, kGroupBudgetOut = 2 };

// s = the softmax sum (:55-56) over the groups' exponentials ge[] (group g
// repeated gc[g] times), in order.  Returns false when the budget ran out.
NLS_RD bool group_sum(const float* ge, const uint32_t* gc, int G, float& s) {
  float acc = 0.0f;
  int budget = kGroupBudget;
  for (int g = 0; g < G; ++g) {
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
  // top-p (:103-108): n = first i + 1 with (double)cum >= topP
  if (topp_active) {
    float cum = 0.0f;
    int64_t pos = 0;
    bool found = false, more = true;
    for (int g = 0; g < G; ++g) {
      const uint32_t j = run_add_until(cum, pg[g], gc[g], topP, budget, &more);
      if (budget < 0) {
        out.status = kGroupBudgetOut;
        return out;
      }
      if (j) {
        n = pos + j;
        found = true;
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
    n = m < n ? m : n;
  }
  // total (:115-116) over the first n candidates
  float total = 0.0f;
  {
    int64_t pos = 0;
    bool more = true;
    for (int g = 0; g < G && pos < n; ++g) {
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
  int64_t held = 0;
  for (int g = 0; g < G; ++g) held += gc[g];
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
