/*
 * nls_oracle.h -- CPU restatement of nimllm's token sampler.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.  The
 * product path (nim.llm_amd/, include/) never links or calls it.
 *
 * It restates, statement by statement, src/nimllm/sampler.nim:59-121
 * (`sample`), :45-49 (`argmax`), :51-57 (`softmaxInPlace`), :123-130
 * (`topTokens`) and the parts of Nim's std/random the sampler uses
 * (`initRand(seed)`, `next`, `skipRandomNumbers`, `rand(max: float)`).
 * fp32 arithmetic is performed in the order the reference performs it and the
 * file is compiled with -O2 -ffp-contract=off (no FMA, no fast-math), as the
 * reference's own test build does (tests/config.nims:1-3).
 */
#ifndef NLS_ORACLE_H
#define NLS_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Mirror of SamplerParams (sampler.nim:11-21) minus the logitBias table,
 * which is passed as (ids, vals, count) with unique ids. */
typedef struct {
  double temperature;
  int64_t topK;
  double topP;
  double minP;
  double repeatPenalty;
  int64_t repeatLastN;
  double presencePenalty;
  double frequencyPenalty;
  int64_t seed;
} nlo_params;

/* Nim std/random `Rand`: two 64-bit words. */
typedef struct {
  uint64_t a0, a1;
} nlo_rand;

void nlo_init_rand(nlo_rand* r, int64_t seed);
uint64_t nlo_next(nlo_rand* r);
void nlo_skip_random_numbers(nlo_rand* r);
double nlo_rand_float(nlo_rand* r, double max);
/* First n values of rand(1.0) from initRand(seed). */
void nlo_uniforms(int64_t seed, int64_t n, double* out);

enum { NLO_EXPF_LIBM = 0, NLO_EXPF_CR = 1 };

/* Correctly rounded expf, computed as (float)expl(x) (64-bit significand). */
float nlo_expf_cr(float x);
float nlo_expf(float x, int mode);

typedef struct {
  int64_t id;       /* returned token id */
  int32_t greedy;   /* 1 when temperature <= 0 returned argmax */
  int32_t heap;     /* 1 when the top-k heap path ran, 0 for the full sort */
  int64_t ncand;    /* idx.len: k on the heap path, V on the sort path */
  int64_t n;        /* candidates kept after top-p and min-p */
  int64_t pos;      /* position of `id` in candidate order */
  float sum;        /* softmax denominator s */
  float total;      /* sum of the first n probabilities */
  float r0;         /* float32(u) * total */
  float thr;        /* min-p threshold (0 when min-p is off) */
  double margin_draw; /* min |r| around the chosen step, relative to total */
  double margin_topp; /* |cum - topP| at the last two steps of the top-p scan */
  double margin_minp; /* |p_m - thr| / thr at the min-p stop */
} nlo_result;

/*
 * One call of `sample` (sampler.nim:59-121) on one row.
 *   logits[V]            row of logits; never modified
 *   hist[hlen]           the sampler's history (accepted ids, any int64)
 *   bias_ids/vals[nbias] logitBias entries (unique ids)
 *   u                    the value rand(1.0) would return at :117
 * Optional outputs (NULL to skip):
 *   cand[ncand]   candidate ids in the order `idx` holds them after :85-97
 *   probs[ncand]  softmax probabilities after :100
 *   final_logits[V] logits after penalties, bias and temperature
 */
int64_t nlo_sample(const nlo_params* p, const float* logits, int64_t V,
                   const int64_t* hist, int64_t hlen,
                   const int64_t* bias_ids, const double* bias_vals, int64_t nbias,
                   double u, int expf_mode, nlo_result* res,
                   int64_t* cand, float* probs, float* final_logits);

/*
 * B independent rows, each with its own params, history and bias, run on
 * `nthreads` POSIX threads (rows split in contiguous blocks).  Used as the
 * CPU baseline.  hist is [B x H] with hlen[B] valid entries per row; bias is
 * [B x NB] with nb[B] valid entries per row.
 */
void nlo_sample_batch(const nlo_params* p, const float* logits, int64_t B, int64_t V,
                      const int64_t* hist, int64_t H, const int64_t* hlen,
                      const int64_t* bias_ids, const double* bias_vals, int64_t NB,
                      const int64_t* nb, const double* u, int expf_mode,
                      int64_t* out_ids, int nthreads);

/* nlo_sample_batch that also fills res[B] (NULL: skip) with every row's
 * nlo_result: n, total and the distances of the draw, the top-p cutoff and
 * the min-p cutoff from their boundaries (the exception classes). */
void nlo_sample_batch_res(const nlo_params* p, const float* logits, int64_t B, int64_t V,
                          const int64_t* hist, int64_t H, const int64_t* hlen,
                          const int64_t* bias_ids, const double* bias_vals, int64_t NB,
                          const int64_t* nb, const double* u, int expf_mode,
                          int64_t* out_ids, nlo_result* res, int nthreads);

/* nlo_sample_batch_res that also writes the first cap candidates of every
 * row (ids and probabilities, as nlo_sample's cand / probs give them) into
 * cand_ids[B, cap] and cand_probs[B, cap]; entries past ncand hold -1 / 0. */
void nlo_sample_batch_cand(const nlo_params* p, const float* logits, int64_t B, int64_t V,
                           const int64_t* hist, int64_t H, const int64_t* hlen,
                           const int64_t* bias_ids, const double* bias_vals, int64_t NB,
                           const int64_t* nb, const double* u, int expf_mode,
                           int64_t* out_ids, nlo_result* res, int64_t cap, int64_t* cand_ids,
                           float* cand_probs, int nthreads);

/* argmax (sampler.nim:45-49): first index of the greatest value. */
int64_t nlo_argmax(const float* x, int64_t n);
/* softmaxInPlace (sampler.nim:51-57). */
void nlo_softmax_inplace(float* x, int64_t n, int expf_mode);
/* topTokens (sampler.nim:123-130); returns min(n, V) entries. */
int64_t nlo_top_tokens(const float* logits, int64_t V, int64_t n, int expf_mode,
                       int64_t* ids, float* probs);
/* perplexity's per-position negative log-likelihood (model.nim:578-583). */
double nlo_row_nll(const float* logits, int64_t V, int64_t target);
/* logProb's per-token term (nimllm-doc-en.md:1700-1707): p = softmaxInPlace of
 * a copy of the row (sampler.nim:51-57), then ln(float64(p[target])); *p_out
 * receives p[target].  target outside [0, V) gives NaN. */
double nlo_log_prob(const float* logits, int64_t V, int64_t target, int expf_mode, float* p_out);

#ifdef __cplusplus
}
#endif
#endif
