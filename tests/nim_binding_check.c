/*
 * nim_binding_check.c -- makes exactly the C-ABI calls of the Nim binding
 * a Nim maintainer adds to src/nimllm/sampler.nim (a `Sampler` whose sample/accept forward to a
 * one-row handle) and checks every sampled id against the oracle.
 *
 * The reference loop it follows: src/nimllm/chat.nim:204-208 (sample, stop on
 * an end-of-generation id without accepting it, accept) with the sampler of
 * src/nimllm/sampler.nim:37-43,59-121.  The binding:
 *   newSampler(p)        Nim side only: params, rng = initRand(seed), history
 *   first sample(logits) nls_create(&c, 1, len(logits), NULL, &h);
 *                        nls_set_rng_state(h, 0, rng.a0, rng.a1);
 *                        nls_accept(h, history, len(history))
 *   sample(logits)       nls_sample_host(h, logits, &id)
 *   accept(id)           history.add id; nls_accept(h, &id, 1)
 * The oracle consumes rand(1.0) from its own copy of the row's stream on
 * non-greedy calls only, as the reference does.
 *
 * Built by __graft_entry__.build() (tests/Makefile) against the product
 * library and the oracle; run by tests/test_gpu_parity.py on a GPU.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../include/nimllm_sampler.h"
#include "../oracle/nls_oracle.h"

static uint64_t g_state = 0x9E3779B97F4A7C15ULL;
static uint64_t next_u64(void) { /* splitmix64 */
  uint64_t z = (g_state += 0x9E3779B97F4A7C15ULL);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}
static double unit(void) { return (double)(next_u64() >> 11) * (1.0 / 9007199254740992.0); }
static float gauss(void) {
  const double a = unit() + 1e-300, b = unit();
  return (float)(sqrt(-2.0 * log(a)) * cos(6.283185307179586 * b));
}

typedef struct {
  nls_params c;          /* the binding's copy of SamplerParams */
  nlo_params o;          /* the oracle's */
  int64_t bias_ids[4];
  double bias_vals[4];
  nlo_rand rng;          /* Nim `Rand` of the Sampler (newSampler) */
  nlo_rand oracle_rng;   /* the oracle's copy of the same stream */
  int64_t* hist;
  int64_t hlen;
  nls_sampler* h;        /* created at the first sample call */
} nim_sampler;

static int fail(const char* what, int st) {
  printf("FAIL %s: %s (%s)\n", what, nls_status_string(st), nls_last_error());
  return 1;
}

/* sample(s, logits): the binding's lazy create, then nls_sample_host */
static int binding_sample(nim_sampler* s, const float* logits, int64_t V, int64_t* id) {
  int st;
  if (!s->h) {
    if ((st = nls_create(&s->c, 1, V, NULL, &s->h))) return fail("nls_create", st);
    if ((st = nls_set_rng_state(s->h, 0, s->rng.a0, s->rng.a1))) return fail("set_rng_state", st);
    if (s->hlen > 0 && (st = nls_accept(s->h, s->hist, (int32_t)s->hlen))) return fail("replay", st);
  }
  if ((st = nls_sample_host(s->h, logits, id))) return fail("nls_sample_host", st);
  return 0;
}

static int binding_accept(nim_sampler* s, int64_t id) {
  s->hist[s->hlen++] = id;
  if (s->h) {
    int st = nls_accept(s->h, &id, 1);
    if (st) return fail("nls_accept", st);
  }
  return 0;
}

int main(void) {
  const int64_t V = 32000;
  const int steps = 40;
  const int64_t eog[2] = {1, 2};
  float* x = (float*)malloc(sizeof(float) * V);
  nim_sampler rows[4];
  memset(rows, 0, sizeof rows);
  for (int r = 0; r < 4; ++r) {
    nim_sampler* s = &rows[r];
    s->c = nls_default_sampling(); /* T 0.7, k 40, p 0.95, min-p 0.05, rp 1.1 over 64 */
    s->c.seed = 1000 + r;
    if (r == 1) { /* greedySampling with a penalty window */
      s->c = nls_greedy_sampling();
      s->c.repeat_penalty = 1.3;
      s->c.repeat_last_n = 16;
    }
    if (r == 2) { /* full-sort path: top-k off, frequency/presence penalties */
      s->c.top_k = 0;
      s->c.top_p = 0.9;
      s->c.frequency_penalty = 0.4;
      s->c.presence_penalty = 0.2;
      s->c.repeat_last_n = 0;
    }
    if (r == 3) { /* logit bias, one id banned */
      s->bias_ids[0] = 5;
      s->bias_vals[0] = -INFINITY;
      s->bias_ids[1] = 77;
      s->bias_vals[1] = 2.5;
      s->c.logit_bias_ids = s->bias_ids;
      s->c.logit_bias_values = s->bias_vals;
      s->c.logit_bias_count = 2;
    }
    s->o.temperature = s->c.temperature;
    s->o.topK = s->c.top_k;
    s->o.topP = s->c.top_p;
    s->o.minP = s->c.min_p;
    s->o.repeatPenalty = s->c.repeat_penalty;
    s->o.repeatLastN = s->c.repeat_last_n;
    s->o.presencePenalty = s->c.presence_penalty;
    s->o.frequencyPenalty = s->c.frequency_penalty;
    s->o.seed = s->c.seed;
    nlo_init_rand(&s->rng, s->c.seed);
    s->oracle_rng = s->rng;
    s->hist = (int64_t*)calloc((size_t)steps + 8, sizeof(int64_t));
    /* a history accepted before the first sample call is replayed at create */
    for (int j = 0; j < 3; ++j) s->hist[s->hlen++] = (int64_t)(next_u64() % (uint64_t)V);
  }
  int ended = 0;
  for (int t = 0; t < steps; ++t) {
    for (int r = 0; r < 4; ++r) {
      nim_sampler* s = &rows[r];
      for (int64_t i = 0; i < V; ++i) x[i] = 2.0f * gauss();
      if (unit() < 0.25) x[eog[t & 1]] += 14.0f; /* end the turn now and then */
      int64_t id = -1;
      if (binding_sample(s, x, V, &id)) return 1;
      const double u = s->o.temperature > 0 ? nlo_rand_float(&s->oracle_rng, 1.0) : 0.0;
      nlo_result res;
      const int64_t want = nlo_sample(&s->o, x, V, s->hist, s->hlen, s->bias_ids, s->bias_vals,
                                      s->c.logit_bias_count, u, NLO_EXPF_CR, &res, NULL, NULL, NULL);
      if (id != want) {
        printf("FAIL step %d row %d: device %lld, oracle %lld\n", t, r, (long long)id,
               (long long)want);
        return 1;
      }
      if (id == eog[0] || id == eog[1]) {
        ++ended; /* chat.nim:206-207: the turn ends, nothing is accepted */
        continue;
      }
      if (binding_accept(s, id)) return 1;
    }
  }
  for (int r = 0; r < 4; ++r) {
    uint64_t a0, a1;
    int st = nls_get_rng_state(rows[r].h, 0, &a0, &a1);
    if (st) return fail("get_rng_state", st);
    if (a0 != rows[r].oracle_rng.a0 || a1 != rows[r].oracle_rng.a1) {
      printf("FAIL row %d: RNG state differs from the oracle's stream\n", r);
      return 1;
    }
    nls_destroy(rows[r].h);
    free(rows[r].hist);
  }
  free(x);
  printf("nim binding sequence ok: 4 rows x %d steps bit-exact, %d turns ended\n", steps, ended);
  return 0;
}
