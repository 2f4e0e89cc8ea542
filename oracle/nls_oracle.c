/*
 * nls_oracle.c -- CPU restatement of nimllm's sampler (TEST INFRASTRUCTURE).
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * this file's library.  It is the checker the HIP sampler is compared with;
 * it is never part of the product path.
 *
 * Each function cites the reference line it restates.  Build flags:
 * -O2 -ffp-contract=off, no fast-math (the reference's test build has no FMA:
 * tests/config.nims:1-3 builds -d:release without -march=native).
 *
 * Pinning (what checks this file, besides the reference it restates):
 *   RNG next/skipRandomNumbers  -> GF(2) matrix power (the jump must equal
 *                                  2^64 applications of `next`)
 *   rand(1.0)                   -> closed form (x >> 12) * 2^-52
 *   initRand seed split/seed 0  -> parity unpinned (no Nim toolchain here)
 *   penalties, bias, temperature-> closed forms / brute force on tiny rows
 *   argmax                      -> numpy.argmax (first maximum)
 *   heap path                   -> Python heapq simulation + closed-form rule
 *   sort path                   -> Python stable sorted()
 *   softmax, cutoffs, draw      -> independent Python restatement on numpy
 *                                  float32 scalars + libm expf via ctypes,
 *                                  and invariants (u=0 -> first candidate,
 *                                  k=1 -> argmax, sum of post-filter p = 1)
 */
#include "nls_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* Nim std/random (xoroshiro128+), used at sampler.nim:39 and :117.          */
/* ------------------------------------------------------------------------ */

static inline uint64_t rotl64(uint64_t x, unsigned k) {
  return (x << k) | (x >> (64u - k));
}

/* std/random `next`: result = a0 + a1, then the 55/14/36 state update. */
uint64_t nlo_next(nlo_rand* r) {
  const uint64_t s0 = r->a0;
  uint64_t s1 = r->a1;
  const uint64_t result = s0 + s1;
  s1 ^= s0;
  r->a0 = rotl64(s0, 55) ^ s1 ^ (s1 << 14);
  r->a1 = rotl64(s1, 36);
  return result;
}

/* std/random `skipRandomNumbers`: the xoroshiro128+ jump (2^64 steps). */
void nlo_skip_random_numbers(nlo_rand* r) {
  static const uint64_t jump[2] = {0xbeac0467eba5facbULL, 0xd86b048b86aa9922ULL};
  uint64_t s0 = 0, s1 = 0;
  for (int i = 0; i < 2; ++i) {
    for (int b = 0; b < 64; ++b) {
      if (jump[i] & (1ULL << b)) {
        s0 ^= r->a0;
        s1 ^= r->a1;
      }
      (void)nlo_next(r);
    }
  }
  r->a0 = s0;
  r->a1 = s1;
}

/* std/random `initRand(seed)`: seed 0 becomes int32.high; a0 = seed shr 16,
 * a1 = seed and 0xffff; jump; discard one `next`.  (Used by newSampler,
 * sampler.nim:39, for seed >= 0.) */
void nlo_init_rand(nlo_rand* r, int64_t seed) {
  const int64_t s = seed != 0 ? seed : 2147483647LL;
  r->a0 = (uint64_t)(s >> 16);
  r->a1 = (uint64_t)(s & 0xffff);
  nlo_skip_random_numbers(r);
  (void)nlo_next(r);
}

/* std/random `rand(max: float)`: 52 random mantissa bits under exponent 0. */
double nlo_rand_float(nlo_rand* r, double max) {
  const uint64_t x = nlo_next(r);
  const uint64_t bits = (0x3FFULL << 52) | (x >> 12);
  double f;
  memcpy(&f, &bits, sizeof f);
  return (f - 1.0) * max;
}

void nlo_uniforms(int64_t seed, int64_t n, double* out) {
  nlo_rand r;
  nlo_init_rand(&r, seed);
  for (int64_t i = 0; i < n; ++i) out[i] = nlo_rand_float(&r, 1.0);
}

/* ------------------------------------------------------------------------ */
/* exp(float32): the reference binds C expf (sampler.nim:56).                */
/* ------------------------------------------------------------------------ */

float nlo_expf_cr(float x) { return (float)expl((long double)x); }

float nlo_expf(float x, int mode) {
  return mode == NLO_EXPF_CR ? nlo_expf_cr(x) : expf(x);
}

/* ------------------------------------------------------------------------ */
/* argmax / softmaxInPlace / topTokens                                       */
/* ------------------------------------------------------------------------ */

/* sampler.nim:45-49 -- strict `>` keeps the first maximum. */
int64_t nlo_argmax(const float* x, int64_t n) {
  int64_t best = 0;
  for (int64_t i = 1; i < n; ++i)
    if (x[i] > x[best]) best = i;
  return best;
}

/* Nim `max(x, y)` on floats. */
static inline float nim_maxf(float a, float b) { return a <= b ? b : a; }

/* sampler.nim:51-57 -- sequential max, exp + running fp32 sum, divide. */
void nlo_softmax_inplace(float* x, int64_t n, int expf_mode) {
  float mx = -INFINITY;
  for (int64_t i = 0; i < n; ++i) mx = nim_maxf(mx, x[i]);
  float s = 0.0f;
  for (int64_t i = 0; i < n; ++i) {
    x[i] = nlo_expf(x[i] - mx, expf_mode);
    s += x[i];
  }
  for (int64_t i = 0; i < n; ++i) x[i] /= s;
}

/* Nim `cmp` on floats: 0 when equal (so -0.0 ties with 0.0). */
static inline int nim_cmpf(float a, float b) {
  if (a == b) return 0;
  if (a < b) return -1;
  return 1;
}

/* algorithm.sort is a stable merge sort; restated as a top-down merge sort
 * with the reference's comparator cmp(v[b], v[a]) (descending by value). */
static void merge_sort_desc(int64_t* idx, int64_t* tmp, int64_t n, const float* v) {
  if (n < 2) return;
  /* bottom-up merge sort, stable */
  int64_t* src = idx;
  int64_t* dst = tmp;
  for (int64_t width = 1; width < n; width *= 2) {
    for (int64_t lo = 0; lo < n; lo += 2 * width) {
      int64_t mid = lo + width < n ? lo + width : n;
      int64_t hi = lo + 2 * width < n ? lo + 2 * width : n;
      int64_t i = lo, j = mid, k = lo;
      while (i < mid && j < hi) {
        /* take from the right run only when it is strictly before */
        if (nim_cmpf(v[src[j]], v[src[i]]) > 0)
          dst[k++] = src[j++];
        else
          dst[k++] = src[i++];
      }
      while (i < mid) dst[k++] = src[i++];
      while (j < hi) dst[k++] = src[j++];
    }
    int64_t* t = src;
    src = dst;
    dst = t;
  }
  if (src != idx) memcpy(idx, src, (size_t)n * sizeof(int64_t));
}

/* sampler.nim:123-130 */
int64_t nlo_top_tokens(const float* logits, int64_t V, int64_t n, int expf_mode,
                       int64_t* ids, float* probs) {
  float* pr = (float*)malloc((size_t)V * sizeof(float));
  int64_t* idx = (int64_t*)malloc((size_t)V * sizeof(int64_t));
  int64_t* tmp = (int64_t*)malloc((size_t)V * sizeof(int64_t));
  memcpy(pr, logits, (size_t)V * sizeof(float));
  nlo_softmax_inplace(pr, V, expf_mode);
  for (int64_t i = 0; i < V; ++i) idx[i] = i;
  merge_sort_desc(idx, tmp, V, pr);
  int64_t m = n < V ? n : V;
  for (int64_t i = 0; i < m; ++i) {
    ids[i] = idx[i];
    probs[i] = pr[idx[i]];
  }
  free(pr);
  free(idx);
  free(tmp);
  return m;
}

/* perplexity's per-position term (src/nimllm/model.nim:578-583): the float32
 * maximum of the row (Nim's max(mx, v) keeps mx when v is NaN), the float64
 * sum in index order of exp(float64(l - mx)) (the subtraction in float32),
 * and -(float64(l[target] - mx) - ln(s)). */
double nlo_row_nll(const float* logits, int64_t V, int64_t target) {
  float mx = -INFINITY;
  for (int64_t k = 0; k < V; ++k)
    if (mx <= logits[k]) mx = logits[k];
  double s = 0.0;
  for (int64_t k = 0; k < V; ++k) s += exp((double)(logits[k] - mx));
  return -((double)(logits[target] - mx) - log(s));
}

/* logProb (nimllm-doc-en.md:1700-1707): `var p = logits; softmaxInPlace(p);
 * result += ln(p[id].float)` -- the float32 probability, widened, then the
 * float64 natural log (Nim's ln is the C library's log). */
double nlo_log_prob(const float* logits, int64_t V, int64_t target, int expf_mode, float* p_out) {
  if (target < 0 || target >= V) {
    if (p_out) *p_out = NAN;
    return NAN;
  }
  float* p = (float*)malloc((size_t)V * sizeof(float));
  memcpy(p, logits, (size_t)V * sizeof(float));
  nlo_softmax_inplace(p, V, expf_mode);
  const float pt = p[target];
  free(p);
  if (p_out) *p_out = pt;
  return log((double)pt);
}

/* ------------------------------------------------------------------------ */
/* HeapQueue[(float32, int)] (sampler.nim:88-95): binary min-heap ordered by */
/* Nim's lexicographic tuple `<`, which compares fields with `cmp`.          */
/* ------------------------------------------------------------------------ */

typedef struct {
  float v;
  int64_t i;
} heap_item;

static inline int item_less(heap_item a, heap_item b) {
  int c = nim_cmpf(a.v, b.v);
  if (c < 0) return 1;
  if (c > 0) return 0;
  return a.i < b.i;
}

static void sift_up(heap_item* h, int64_t pos) {
  heap_item it = h[pos];
  while (pos > 0) {
    int64_t parent = (pos - 1) >> 1;
    if (!item_less(it, h[parent])) break;
    h[pos] = h[parent];
    pos = parent;
  }
  h[pos] = it;
}

static void sift_down(heap_item* h, int64_t n, int64_t pos) {
  heap_item it = h[pos];
  for (;;) {
    int64_t c = 2 * pos + 1;
    if (c >= n) break;
    if (c + 1 < n && item_less(h[c + 1], h[c])) c++;
    if (!item_less(h[c], it)) break;
    h[pos] = h[c];
    pos = c;
  }
  h[pos] = it;
}

/* ------------------------------------------------------------------------ */
/* sample (sampler.nim:59-121)                                               */
/* ------------------------------------------------------------------------ */

static int cmp_i64(const void* a, const void* b) {
  int64_t x = *(const int64_t*)a, y = *(const int64_t*)b;
  return (x > y) - (x < y);
}

int64_t nlo_sample(const nlo_params* p, const float* logits_in, int64_t V,
                   const int64_t* hist, int64_t hlen,
                   const int64_t* bias_ids, const double* bias_vals, int64_t nbias,
                   double u, int expf_mode, nlo_result* res,
                   int64_t* cand_out, float* probs_out, float* final_logits) {
  nlo_result rr;
  memset(&rr, 0, sizeof rr);
  rr.id = -1;
  if (V <= 0) {
    if (res) *res = rr;
    return -1; /* the reference raises IndexDefect at :121 */
  }

  /* :62 -- private copy; the input is never modified */
  float* l = (float*)malloc((size_t)V * sizeof(float));
  memcpy(l, logits_in, (size_t)V * sizeof(float));

  /* :64-74 -- penalties over the last repeatLastN accepted ids */
  if (hlen > 0 && (p->repeatPenalty != 1.0 || p->presencePenalty != 0 ||
                   p->frequencyPenalty != 0)) {
    int64_t start = 0;
    if (p->repeatLastN > 0) {
      start = hlen - p->repeatLastN;
      if (start < 0) start = 0;
    }
    int64_t w = hlen - start;
    /* CountTable: only the multiset of counts matters, each distinct id is
     * updated exactly once, so counting through a sorted copy is equivalent */
    int64_t* win = (int64_t*)malloc((size_t)w * sizeof(int64_t));
    memcpy(win, hist + start, (size_t)w * sizeof(int64_t));
    qsort(win, (size_t)w, sizeof(int64_t), cmp_i64);
    const float rp32 = (float)p->repeatPenalty;
    for (int64_t a = 0; a < w;) {
      int64_t b = a;
      while (b < w && win[b] == win[a]) ++b;
      const int64_t tok = win[a];
      const int64_t cnt = b - a;
      a = b;
      if (tok < 0 || tok >= V) continue; /* :70 */
      if (p->repeatPenalty != 1.0) {     /* :71-73 */
        if (l[tok] > 0)
          l[tok] /= rp32;
        else
          l[tok] *= rp32;
      }
      /* :74 -- float64 multiply and add, one rounding to float32 */
      const double pen = (double)cnt * p->frequencyPenalty + p->presencePenalty;
      l[tok] -= (float)pen;
    }
    free(win);
  }
  /* :75-76 -- logit bias, after the penalties */
  for (int64_t j = 0; j < nbias; ++j) {
    const int64_t tok = bias_ids[j];
    if (tok >= 0 && tok < V) l[tok] += (float)bias_vals[j];
  }

  /* :77-78 -- greedy: argmax, no RNG draw */
  if (p->temperature <= 0) {
    rr.id = nlo_argmax(l, V);
    rr.greedy = 1;
    if (final_logits) memcpy(final_logits, l, (size_t)V * sizeof(float));
    free(l);
    if (res) *res = rr;
    return rr.id;
  }

  /* :80-81 -- temperature as a float32 multiply by float32(1/T) */
  const float invT = (float)(1.0 / p->temperature);
  for (int64_t i = 0; i < V; ++i) l[i] *= invT;
  if (final_logits) memcpy(final_logits, l, (size_t)V * sizeof(float));

  /* :83-97 -- candidate order */
  int64_t* idx = (int64_t*)malloc((size_t)V * sizeof(int64_t));
  for (int64_t i = 0; i < V; ++i) idx[i] = i;
  const int64_t k = p->topK > 0 ? (p->topK < V ? p->topK : V) : V;
  int64_t ncand;
  if (k < V) {
    /* :88-95 -- size-k min-heap; replace when strictly greater than the min */
    heap_item* h = (heap_item*)malloc((size_t)k * sizeof(heap_item));
    int64_t hn = 0;
    for (int64_t i = 0; i < V; ++i) {
      if (hn < k) {
        h[hn].v = l[i];
        h[hn].i = i;
        sift_up(h, hn);
        ++hn;
      } else if (l[i] > h[0].v) {
        h[0].v = l[i];
        h[0].i = i;
        sift_down(h, hn, 0);
      }
    }
    /* pop ascending, then reverse -> descending (value, index) */
    ncand = 0;
    while (hn > 0) {
      idx[ncand++] = h[0].i;
      h[0] = h[hn - 1];
      --hn;
      if (hn > 0) sift_down(h, hn, 0);
    }
    for (int64_t a = 0, b = ncand - 1; a < b; ++a, --b) {
      int64_t t = idx[a];
      idx[a] = idx[b];
      idx[b] = t;
    }
    free(h);
    rr.heap = 1;
  } else {
    /* :97 -- stable sort by value, descending */
    int64_t* tmp = (int64_t*)malloc((size_t)V * sizeof(int64_t));
    merge_sort_desc(idx, tmp, V, l);
    free(tmp);
    ncand = V;
  }
  rr.ncand = ncand;

  /* :98-100 -- gather and softmax in candidate order */
  float* probs = (float*)malloc((size_t)ncand * sizeof(float));
  for (int64_t i = 0; i < ncand; ++i) probs[i] = l[idx[i]];
  {
    float mx = -INFINITY;
    for (int64_t i = 0; i < ncand; ++i) mx = nim_maxf(mx, probs[i]);
    float s = 0.0f;
    for (int64_t i = 0; i < ncand; ++i) {
      probs[i] = nlo_expf(probs[i] - mx, expf_mode);
      s += probs[i];
    }
    for (int64_t i = 0; i < ncand; ++i) probs[i] /= s;
    rr.sum = s;
  }
  if (cand_out)
    for (int64_t i = 0; i < ncand; ++i) cand_out[i] = idx[i];
  if (probs_out) memcpy(probs_out, probs, (size_t)ncand * sizeof(float));

  int64_t n = ncand;
  /* :103-108 -- top-p: fp32 running sum compared in float64 */
  rr.margin_topp = INFINITY;
  if (p->topP > 0 && p->topP < 1) {
    float cum = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
      cum += probs[i];
      double m = fabs((double)cum - p->topP);
      if (m < rr.margin_topp) rr.margin_topp = m;
      if ((double)cum >= p->topP) {
        n = i + 1;
        break;
      }
    }
  }
  /* :110-114 -- min-p prefix, after top-p */
  rr.margin_minp = INFINITY;
  if (p->minP > 0) {
    const float thr = probs[0] * (float)p->minP;
    rr.thr = thr;
    int64_t m = 1;
    while (m < n && probs[m] >= thr) ++m;
    if (m < n) rr.margin_minp = fabs((double)probs[m] - thr) / thr;
    if (m > 1) {
      double d = fabs((double)probs[m - 1] - thr) / thr;
      if (d < rr.margin_minp) rr.margin_minp = d;
    }
    n = m;
  }
  rr.n = n;
  /* :115-121 -- draw by subtracting from float32(u) * total */
  float total = 0.0f;
  for (int64_t i = 0; i < n; ++i) total += probs[i];
  rr.total = total;
  float r = (float)u * total;
  rr.r0 = r;
  int64_t pos = n - 1;
  double mprev = fabs((double)r);
  rr.margin_draw = INFINITY;
  for (int64_t i = 0; i < n; ++i) {
    r -= probs[i];
    double mcur = fabs((double)r);
    if (r <= 0) {
      pos = i;
      rr.margin_draw = (mcur < mprev ? mcur : mprev) / (double)total;
      break;
    }
    mprev = mcur;
  }
  rr.pos = pos;
  rr.id = idx[pos];
  free(probs);
  free(idx);
  free(l);
  if (res) *res = rr;
  return rr.id;
}

/* ------------------------------------------------------------------------ */
/* Batch driver for the CPU baseline                                         */
/* ------------------------------------------------------------------------ */

typedef struct {
  const nlo_params* p;
  const float* logits;
  int64_t V;
  const int64_t* hist;
  int64_t H;
  const int64_t* hlen;
  const int64_t* bias_ids;
  const double* bias_vals;
  int64_t NB;
  const int64_t* nb;
  const double* u;
  int expf_mode;
  int64_t* out;
  nlo_result* res;
  int64_t cap;         /* candidates kept per row in cand_ids / cand_probs */
  int64_t* cand_ids;   /* [B, cap] or NULL */
  float* cand_probs;   /* [B, cap] or NULL */
  int64_t r0, r1;
} batch_job;

static void* batch_worker(void* arg) {
  batch_job* j = (batch_job*)arg;
  const int want = j->cap > 0 && j->cand_ids && j->cand_probs;
  int64_t* ci = want ? (int64_t*)malloc((size_t)j->V * sizeof(int64_t)) : NULL;
  float* cp = want ? (float*)malloc((size_t)j->V * sizeof(float)) : NULL;
  for (int64_t r = j->r0; r < j->r1; ++r) {
    nlo_result rr;
    j->out[r] = nlo_sample(&j->p[r], j->logits + r * j->V, j->V,
                           j->hist ? j->hist + r * j->H : NULL, j->hlen ? j->hlen[r] : 0,
                           j->bias_ids ? j->bias_ids + r * j->NB : NULL,
                           j->bias_vals ? j->bias_vals + r * j->NB : NULL,
                           j->nb ? j->nb[r] : 0, j->u[r], j->expf_mode, &rr, ci, cp, NULL);
    if (j->res) j->res[r] = rr;
    if (want) {
      const int64_t m = rr.ncand < j->cap ? rr.ncand : j->cap;
      for (int64_t i = 0; i < j->cap; ++i) {
        j->cand_ids[r * j->cap + i] = i < m ? ci[i] : -1;
        j->cand_probs[r * j->cap + i] = i < m ? cp[i] : 0.0f;
      }
    }
  }
  free(ci);
  free(cp);
  return NULL;
}

void nlo_sample_batch(const nlo_params* p, const float* logits, int64_t B, int64_t V,
                      const int64_t* hist, int64_t H, const int64_t* hlen,
                      const int64_t* bias_ids, const double* bias_vals, int64_t NB,
                      const int64_t* nb, const double* u, int expf_mode,
                      int64_t* out_ids, int nthreads) {
  nlo_sample_batch_res(p, logits, B, V, hist, H, hlen, bias_ids, bias_vals, NB, nb, u, expf_mode,
                       out_ids, NULL, nthreads);
}

void nlo_sample_batch_res(const nlo_params* p, const float* logits, int64_t B, int64_t V,
                          const int64_t* hist, int64_t H, const int64_t* hlen,
                          const int64_t* bias_ids, const double* bias_vals, int64_t NB,
                          const int64_t* nb, const double* u, int expf_mode,
                          int64_t* out_ids, nlo_result* res, int nthreads) {
  nlo_sample_batch_cand(p, logits, B, V, hist, H, hlen, bias_ids, bias_vals, NB, nb, u, expf_mode,
                        out_ids, res, 0, NULL, NULL, nthreads);
}

void nlo_sample_batch_cand(const nlo_params* p, const float* logits, int64_t B, int64_t V,
                           const int64_t* hist, int64_t H, const int64_t* hlen,
                           const int64_t* bias_ids, const double* bias_vals, int64_t NB,
                           const int64_t* nb, const double* u, int expf_mode,
                           int64_t* out_ids, nlo_result* res, int64_t cap, int64_t* cand_ids,
                           float* cand_probs, int nthreads) {
  if (nthreads < 1) nthreads = 1;
  if (nthreads > B) nthreads = (int)(B > 0 ? B : 1);
  batch_job* jobs = (batch_job*)calloc((size_t)nthreads, sizeof(batch_job));
  pthread_t* th = (pthread_t*)calloc((size_t)nthreads, sizeof(pthread_t));
  for (int t = 0; t < nthreads; ++t) {
    batch_job* j = &jobs[t];
    j->p = p;
    j->logits = logits;
    j->V = V;
    j->hist = hist;
    j->H = H;
    j->hlen = hlen;
    j->bias_ids = bias_ids;
    j->bias_vals = bias_vals;
    j->NB = NB;
    j->nb = nb;
    j->u = u;
    j->expf_mode = expf_mode;
    j->out = out_ids;
    j->res = res;
    j->cap = cap;
    j->cand_ids = cand_ids;
    j->cand_probs = cand_probs;
    j->r0 = B * t / nthreads;
    j->r1 = B * (t + 1) / nthreads;
  }
  if (nthreads == 1) {
    batch_worker(&jobs[0]);
  } else {
    for (int t = 0; t < nthreads; ++t) pthread_create(&th[t], NULL, batch_worker, &jobs[t]);
    for (int t = 0; t < nthreads; ++t) pthread_join(th[t], NULL);
  }
  free(jobs);
  free(th);
}
