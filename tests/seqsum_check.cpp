// seqsum_check.cpp -- CPU check of the parallel evaluation of the sequential
// fp32 sum (nim.llm_amd/csrc/nls_seqsum.h) against plain one-at-a-time adds.
//
// The device routine seq_sum_block runs the parity-map scan over a workgroup
// of 1024 threads; this program runs the same steps (the same per-term codes,
// clamped integer increments of waves without ties and packed maps of the
// others, window sizes, the zero codes past a thread's terms, the integer
// scan of plain wave totals, replays and binade changes; the scans run
// Hillis-Steele over each wave and over the waves' totals, a grouping of the
// same associative composition) with the threads as loops,
// on term arrays chosen to break a wrong rounding rule: softmax exponentials
// of many spreads, exact ties at every scale, subnormals and zeros, a dynamic
// range of 2^160, runs that park the sum at 2^24, and NaN / +inf terms.
// Prints one line per case and exits non-zero on the first mismatch.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

#include "../nim.llm_amd/csrc/nls_seqsum.h"

using namespace nls;

static float plain_sum(const std::vector<float>& e, float s) {
  for (float v : e) s = s + v;
  return s;
}

static long g_windows = 0;
static long g_terms = 0;  // terms composed, over all windows

static float block_sum_chunk(const float* e, int len, float s, int& J, int done, int serial) {
  const int NT = 1024, W = 64, NW = NT / W;
  int pos = 0;
  if (done == 0 && serial > 0 && len > 0) {
    // the first terms one at a time (kSeqSerial on the device)
    const int n0 = std::min(len, serial);
    for (int i = 0; i < n0; ++i) s = s + e[i];
    pos = n0;
    J = seq_next_j(n0);
  }
  while (pos < len) {
    ++g_windows;
    if (!(s <= 3.4028234663852886e38f)) {
      for (int i = pos; i < len; ++i) s = s + e[i];
      return s;
    }
    const int E = seq_binade(s);
    const int S0 = (int)seq_ldexp(s, 23 - E);
    const int jn = std::min(J, (len - pos + NT - 1) / NT);
    g_terms += std::min(NT * jn, len - pos);
    std::vector<SeqMap> m(NT, sm_identity()), inc(NT, sm_identity());
    std::vector<int> A(NT), incA(NT);
    std::vector<bool> wodd(NW, false);
    for (int t = 0; t < NT; ++t) {
      const int b = pos + t * jn, end = std::min(b + jn, len);
      // the device's template width: 1, 2, 4, 8, 12 or 16 terms; the run
      // summed as if tie-free (clamped at 2^24), with the parity maps
      // formed for every lane of a wave where one lane met a tie or a term
      // too large
      const int jb = jn <= 1 ? 1 : jn <= 2 ? 2 : jn <= 4 ? 4 : jn <= 8 ? 8 : jn <= 12 ? 12 : 16;
      int a = 0;
      bool odd = false;
      for (int j = 0; j < jb; ++j) {
        const float v = b + j < end ? e[std::min(b + j, len - 1)] : 0.0f;
        const float q = seq_ldexp(v, 23 - E);
        const bool ok = q < 16777216.0f;
        const float qc = ok ? q : 0.0f;
        const float fr = seq_fract(qc);
        a += (int)qc + (fr > 0.5f ? 1 : 0);
        odd = odd || !ok || fr == 0.5f;
      }
      A[t] = std::min(a, 1 << 24);
      wodd[t / W] = wodd[t / W] || odd;
    }
    for (int t = 0; t < NT; ++t) {
      if (!wodd[t / W]) continue;
      const int b = pos + t * jn, end = std::min(b + jn, len);
      const int jb = jn <= 1 ? 1 : jn <= 2 ? 2 : jn <= 4 ? 4 : jn <= 8 ? 8 : jn <= 12 ? 12 : 16;
      SeqRun run;
      for (int j = 0; j < jb; ++j) run.add(b + j < end ? e[std::min(b + j, len - 1)] : 0.0f, E);
      m[t] = run.map();
    }
    // wave-level inclusive scans (Hillis-Steele, as the shuffles do): maps in
    // waves with a tie, integers in the others
    inc = m;
    incA = A;
    for (int o = 1; o < W; o <<= 1) {
      std::vector<SeqMap> nx = inc;
      std::vector<int> nxA = incA;
      for (int t = 0; t < NT; ++t)
        if (t % W >= o) {
          nx[t] = sm_then(inc[t - o], inc[t]);
          nxA[t] = incA[t - o] + incA[t];
        }
      inc = nx;
      incA = nxA;
    }
    // the waves' maps; scanned as integers when every one is plain
    std::vector<SeqMap> wt(NW);
    bool plain = true;
    for (int w = 0; w < NW; ++w) {
      const int l = w * W + W - 1;
      wt[w] = wodd[w] ? inc[l] : sm_make(incA[l], incA[l] & 1, incA[l], (incA[l] + 1) & 1);
      const bool pl = (wt[w].a >> 1) == (wt[w].c >> 1) && ((wt[w].a ^ wt[w].c) & 1) != 0;
      if (wodd[w] && pl) {
        printf("   a wave with a tie has a plain map\n");
        return NAN;
      }
      plain = plain && pl;
    }
    std::vector<SeqMap> wpre(NW, sm_identity());
    int Send;
    if (plain) {
      int d = 0;
      for (int w = 0; w < NW; ++w) {
        wpre[w] = sm_make(d, d & 1, d, (d + 1) & 1);
        d += wt[w].a >> 1;
      }
      Send = S0 + d;
    } else {
      for (int o = 1; o < NW; o <<= 1) {
        std::vector<SeqMap> nx = wt;
        for (int l = o; l < NW; ++l) nx[l] = sm_then(wt[l - o], wt[l]);
        wt = nx;
      }
      for (int w = 1; w < NW; ++w) wpre[w] = wt[w - 1];
      Send = S0 + sm_inc(wt[NW - 1], S0);
    }
    if (Send < (1 << 24)) {
      // no term of the window leaves the binade
      s = seq_ldexp((float)Send, E - 23);
      pos = std::min(pos + NT * jn, len);
      J = std::min(J * 2, kSeqMaxJ);
      continue;
    }
    int kstop = -1;
    float sstop = 0.0f;
    int replays = 0;
    for (int t = 0; t < NT; ++t) {
      const int wv = t / W, lane = t % W;
      int Sin, Sout;
      if (!wodd[wv]) {
        Sin = S0 + sm_inc(wpre[wv], S0) + (incA[t] - A[t]);
        Sout = Sin + A[t];
      } else {
        SeqMap pre = wpre[wv];
        if (lane > 0) pre = sm_then(pre, inc[t - 1]);
        Sin = S0 + sm_inc(pre, S0);
        Sout = Sin < (1 << 24) ? Sin + sm_inc(m[t], Sin) : Sin;
      }
      if (Sin < (1 << 24) && Sout >= (1 << 24)) {
        // the replay: one term per lane of a row, their maps scanned in order
        ++replays;
        const int b = pos + t * jn, end = std::min(b + jn, len);
        std::vector<SeqMap> incl(kSeqMaxJ);
        std::vector<int> code(kSeqMaxJ, 0);
        for (int j = 0; j < kSeqMaxJ; ++j) {
          code[j] = b + j < end ? seq_code(e[b + j], E) : 0;
          incl[j] = seq_code_map(code[j]);
        }
        for (int o = 1; o < kSeqMaxJ; o <<= 1) {
          std::vector<SeqMap> nx = incl;
          for (int j = o; j < kSeqMaxJ; ++j) nx[j] = sm_then(incl[j - o], incl[j]);
          incl = nx;
        }
        for (int j = 0; j < kSeqMaxJ && b + j < end; ++j) {
          const int Sb = Sin + (j > 0 ? sm_inc(incl[j - 1], Sin) : 0);
          const int Sa = Sin + sm_inc(incl[j], Sin);
          if (Sa >= (1 << 24)) {
            kstop = b + j;
            sstop = seq_ldexp((float)Sb, E - 23) + e[b + j];
            break;
          }
        }
        if (kstop < 0) {
          printf("   replay found no stop\n");
          return NAN;
        }
      }
    }
    if (replays > 1) {
      printf("   %d threads replayed one window\n", replays);
      return NAN;
    }
    if (kstop < 0) {
      printf("   a window reached 2^24 without a thread where it does\n");
      return NAN;
    }
    s = sstop;
    J = seq_next_j(done + kstop);
    pos = kstop + 1;
  }
  return s;
}

// the sum over chunks of 12288 terms, the window width carried across them,
// as the softmax kernels call it; `serial` first terms added one at a time
// (the device adds kSeqSerial; 0 runs every term through the windows)
static float block_sum(const std::vector<float>& e, float s, int serial) {
  const int CH = 12288;
  int J = 1;
  for (size_t c0 = 0; c0 < e.size(); c0 += CH)
    s = block_sum_chunk(e.data() + c0, (int)std::min<size_t>(CH, e.size() - c0), s, J, (int)c0, serial);
  return s;
}

static int g_fail = 0;

static void check_one(const char* name, const std::vector<float>& e, float s0, int serial) {
  const long w0 = g_windows, t0 = g_terms;
  const float a = plain_sum(e, s0), b = block_sum(e, s0, serial);
  uint32_t ba, bb;
  memcpy(&ba, &a, 4);
  memcpy(&bb, &b, 4);
  const bool ok = ba == bb || (a != a && b != b);
  printf("%-44s n=%7zu serial=%4d sum=%-14.8g %s (windows %ld, terms composed %.2f n)\n", name, e.size(), serial,
         (double)a, ok ? "ok" : "MISMATCH", g_windows - w0,
         (double)(g_terms - t0) / std::max<size_t>(e.size(), 1));
  if (!ok) {
    printf("   plain %a  block %a\n", (double)a, (double)b);
    g_fail = 1;
  }
}

// every case with all terms through the windows, and as the device runs it
static void check(const char* name, const std::vector<float>& e, float s0 = 0.0f) {
  check_one(name, e, s0, 0);
  check_one(name, e, s0, kSeqSerial);
}

int main() {
  std::mt19937_64 rng(12345);
  std::normal_distribution<double> nd(0.0, 1.0);
  std::uniform_real_distribution<double> ud(0.0, 1.0);
  char name[128];
  // softmax exponentials (correctly rounded exp of l - max, as the kernels use)
  for (double sigma : {0.25, 1.0, 2.5, 5.0, 20.0}) {
    for (int n : {1, 2, 3, 1000, 1025, 32000, 128256, 151936}) {
      std::vector<float> x(n);
      float mx = -INFINITY;
      for (auto& v : x) {
        v = (float)(nd(rng) * sigma);
        mx = std::max(mx, v);
      }
      std::vector<float> e(n);
      for (int i = 0; i < n; ++i) e[i] = expf(x[i] - mx);
      snprintf(name, sizeof name, "softmax terms, sigma %.2f", sigma);
      check(name, e);
    }
  }
  // ties: small dyadic numbers, so e/u lands on halves often
  for (int k : {0, 3, 8, 12, 20}) {
    std::vector<float> e(100000);
    for (auto& v : e) v = std::ldexp((float)(rng() % 4096), -k);
    snprintf(name, sizeof name, "dyadic multiples of 2^-%d", k);
    check(name, e);
  }
  {
    std::vector<float> e(200000);
    for (size_t i = 0; i < e.size(); ++i) e[i] = std::ldexp(1.0f, -(int)(rng() % 40));
    check("powers of two 2^0 .. 2^-39", e);
  }
  // a sum parked at 2^24 (1 + 2^24 rounds back), and halves at large sums
  check("ones past 2^24", std::vector<float>(17000000, 1.0f));
  check("halves from 2^23", std::vector<float>(300000, 0.5f), 8388608.0f);
  check("1.5 from 2^24", std::vector<float>(300000, 1.5f), 16777216.0f);
  // dynamic range and subnormals
  {
    std::vector<float> e(150000);
    for (auto& v : e) v = (float)std::ldexp(1.0 + ud(rng), (int)(rng() % 160) - 150);
    check("magnitudes 2^-150 .. 2^10", e);
  }
  {
    std::vector<float> e(50000);
    for (auto& v : e) {
      const uint32_t bits = (uint32_t)(rng() % 0x00800000u);  // subnormals and 0
      memcpy(&v, &bits, 4);
    }
    check("subnormals and zeros", e);
  }
  {
    std::vector<float> e(60000, 0.0f);
    check("all zeros", e);
    for (size_t i = 0; i < e.size(); i += 7) e[i] = 1e-30f;
    check("sparse tiny terms", e);
  }
  // increasing and decreasing terms (a binade change every few terms / none)
  {
    std::vector<float> e(40000);
    for (size_t i = 0; i < e.size(); ++i) e[i] = (float)std::exp(i * 0.002 - 60);
    check("increasing exponentials", e);
    std::vector<float> r(e.rbegin(), e.rend());
    check("decreasing exponentials", r);
  }
  // not-a-number and infinite terms
  {
    std::vector<float> e(30000);
    for (auto& v : e) v = (float)ud(rng);
    e[12345] = NAN;
    check("a NaN term", e);
    e[12345] = INFINITY;
    check("an infinite term", e);
    e[20000] = NAN;
    check("infinite then NaN", e);
  }
  // random starting sums
  for (int t = 0; t < 20; ++t) {
    std::vector<float> e(5000 + rng() % 40000);
    const float sc = (float)std::ldexp(1.0, (int)(rng() % 40) - 30);
    for (auto& v : e) v = (float)(ud(rng) * sc);
    const float s0 = (float)std::ldexp(ud(rng), (int)(rng() % 60) - 30);
    snprintf(name, sizeof name, "start %.3g, terms up to %.3g", (double)s0, (double)sc);
    check(name, e, s0);
  }
  printf(g_fail ? "FAILED\n" : "all sums bit-identical\n");
  return g_fail;
}
