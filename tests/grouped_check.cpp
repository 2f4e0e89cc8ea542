// Host build of the grouped sort path (nim.llm_amd/csrc/nls_grouped.h) for
// tests/test_runs_cpu.py: groups a row's values the way the kernel does (the
// distinct values with fl(v - mx) >= kGroupFloor, descending, with their
// multiplicities), runs the group walk, and picks the drawn candidate (the
// t-th lowest index among the members of its group, as the stable sort at
// src/nimllm/sampler.nim:97 orders equal values).  The test compares the
// result with the oracle's sort path.
#include <stdint.h>
#include <string.h>

#include <map>
#include <vector>

#include "../nim.llm_amd/csrc/nls_expf.h"
#include "../nim.llm_amd/csrc/nls_grouped.h"

extern "C" int grouped_sample(const float* x, int64_t V, float invT, int topp_active, double topP,
                              int minp_active, float minP32, double u, int64_t* id, int64_t* n,
                              float* total, int32_t* groups) {
  std::vector<float> v((size_t)V);
  float mx = -__builtin_inff();
  for (int64_t i = 0; i < V; ++i) {
    const float t = x[i] * invT;
    v[i] = t + 0.0f;  // -0 joins +0
    if (v[i] != v[i]) return -1;
    if (v[i] > mx) mx = v[i];
  }
  if (!(mx > -__builtin_inff() && mx < __builtin_inff())) return -1;
  std::map<float, uint32_t, std::greater<float>> tab;
  int64_t held = 0;
  for (int64_t i = 0; i < V; ++i) {
    const float d = v[i] - mx;
    if (d >= nls::kGroupFloor) {
      ++tab[v[i]];
      ++held;
    }
  }
  const bool complete = held == V;
  std::vector<float> gv, ge, pg;
  std::vector<uint32_t> gc;
  for (auto& kv : tab) {
    gv.push_back(kv.first);
    gc.push_back(kv.second);
    const float d = kv.first - mx;
    ge.push_back(nls::expf_cr(d));
  }
  const int G = (int)gv.size();
  *groups = G;
  float s;
  if (!nls::group_sum(ge.data(), gc.data(), G, s)) return -2;
  for (int g = 0; g < G; ++g) {
    const float p = ge[g] / s;
    pg.push_back(p);
  }
  const nls::GroupDraw d = nls::group_cut_draw(pg.data(), gc.data(), G, complete, V, topp_active != 0,
                                               topP, minp_active != 0, minP32, u);
  if (d.status != nls::kGroupOk) return 10 + d.status;
  int64_t pos = d.pos;
  int g = 0;
  while (pos >= (int64_t)gc[g]) pos -= gc[g++];
  int64_t seen = 0;
  for (int64_t i = 0; i < V; ++i) {
    if (v[i] == gv[g]) {
      if (seen == pos) {
        *id = i;
        break;
      }
      ++seen;
    }
  }
  *n = d.n;
  *total = d.total;
  return 0;
}
