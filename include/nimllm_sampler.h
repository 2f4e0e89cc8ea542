/*
 * nimllm_sampler.h -- C ABI of the MI355X (gfx950) token sampler.
 *
 * A batched, device-resident replacement for nimllm's `Sampler`
 * (src/nimllm/sampler.nim).  One handle holds B independent samplers ("rows"),
 * each with its own SamplerParams, RNG stream and accepted-token history,
 * exactly as B separate `newSampler` objects would.  Every call is ordered on
 * the handle's HIP stream; only the *_host variants block.
 *
 * The pipeline per row is the reference's (sampler.nim:59-121): penalties ->
 * logit bias -> temperature -> top-k -> softmax -> top-p -> min-p -> draw, and
 * temperature <= 0 is greedy argmax with no RNG draw.  Sampled ids are
 * bit-exact with the reference's fp32 semantics (sequential fp32 sums in
 * candidate order, float64 top-p compare, Nim's heap tie order on the top-k
 * path, stable descending order on the full-sort path).  exp(float32) is
 * evaluated correctly rounded.
 *
 * No symbol here allocates on the caller's behalf except nls_create (and
 * nls_accept* when a row's history window outgrows its ring).
 */
#ifndef NIMLLM_SAMPLER_H
#define NIMLLM_SAMPLER_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes: every entry point returns one.  Nothing throws across the ABI. */
enum {
  NLS_OK = 0,
  NLS_ERR_INVALID_ARGUMENT = 1, /* NULL handle/pointer, batch < 1, bad row, ... */
  NLS_ERR_EMPTY_VOCAB = 2,      /* vocab == 0 (the reference raises IndexDefect, sampler.nim:121) */
  NLS_ERR_HIP = 3,              /* a HIP runtime call failed (see nls_last_error) */
  NLS_ERR_OUT_OF_MEMORY = 4,
  NLS_ERR_NO_DEVICE = 5,        /* no usable gfx950 device */
  NLS_ERR_UNSUPPORTED = 6       /* a size beyond what this build supports */
};

/*
 * Mirror of SamplerParams (sampler.nim:11-21), field for field.  float64 and
 * int64 fields are kept because the reference compares top-p in float64
 * (sampler.nim:107) and forms the penalty in float64 (:74).  `logitBias`
 * (Table[int, float]) becomes (ids, values, count); when an id repeats, the
 * last value wins, as assigning into the table would.  Nim zero-initialises
 * omitted fields: a zero repeat_penalty is *active* (rp != 1), exactly as in
 * the reference -- start from nls_default_sampling() to avoid that.
 */
typedef struct nls_params {
  double temperature;        /* <= 0: greedy argmax                       */
  int64_t top_k;             /* 0: off                                    */
  double top_p;              /* >= 1 or <= 0: off                         */
  double min_p;              /* <= 0: off                                 */
  double repeat_penalty;     /* 1.0: off                                  */
  int64_t repeat_last_n;     /* <= 0: whole history                       */
  double presence_penalty;
  double frequency_penalty;
  int64_t seed;              /* < 0: non-reproducible seed                */
  const int64_t* logit_bias_ids;    /* may be NULL when count == 0        */
  const double* logit_bias_values;  /* -INFINITY forbids a token          */
  int64_t logit_bias_count;
} nls_params;

typedef struct nls_sampler nls_sampler; /* opaque */

/* Optional per-call inspection output (all device pointers, may be NULL). */
typedef struct nls_debug {
  int32_t* n;            /* [B] candidates kept after top-p/min-p (0 for greedy rows)  */
  int32_t* ncand;        /* [B] candidates before the cutoffs (k, or V on the sort path) */
  int32_t* cand_ids;     /* [B x cap] candidate ids in reference order, first min(n, cap) */
  float* cand_probs;     /* [B x cap] softmax probabilities of those candidates           */
  float* total;          /* [B] fp32 sum of the first n probabilities                     */
  int32_t* path;         /* [B] NLS_PATH_* taken by the row                                */
  int32_t cap;
} nls_debug;

enum {
  NLS_PATH_GREEDY = 1,     /* argmax                                          */
  NLS_PATH_TOPK = 2,       /* chunked top-k candidates + exact merge          */
  NLS_PATH_FULL = 3,       /* full-vocabulary (sort) path, fast prefix kernel */
  NLS_PATH_GENERIC = 4,    /* whole-row sort; rows the fast kernels hand off  */
  NLS_PATH_WINDOW = 5,     /* whole-row kernel, top-k members without a sort  */
  /* Flag OR-ed into the path of a sampling row with a NaN among its
   * candidates.  The reference's heap and merge-sort comparisons
   * (sampler.nim:88-97) make the result of a row with any NaN final logit
   * depend on element order, so such a row is outside the parity claim.
   * Here a NaN with the sign bit clear (the NaN the GPU's arithmetic makes)
   * orders above +inf and is always a candidate, so its row is always
   * flagged; one with the sign bit set orders below -inf and is flagged when
   * it is a candidate (full-sort rows, or k above the row's other values).
   * Greedy rows follow argmax (sampler.nim:45-49) exactly, NaN included, and
   * are never flagged. */
  NLS_PATH_NAN = 0x100
};

/* Presets: defaultSampling (sampler.nim:28-31) and greedySampling (:33-35). */
nls_params nls_default_sampling(void);
nls_params nls_greedy_sampling(void);

/*
 * newSampler (sampler.nim:37-39), batched.  per_row[batch] gives each row's
 * params (copied; bias arrays are read during the call only).  The RNG of
 * row b is initRand(seed_b), or a time/entropy seed when seed_b < 0.
 * `stream` is a hipStream_t (NULL = the default stream).
 */
int nls_create(const nls_params* per_row, int32_t batch, int64_t vocab, void* stream,
               nls_sampler** out);
int nls_destroy(nls_sampler* s);
int nls_set_stream(nls_sampler* s, void* stream);
int32_t nls_batch(const nls_sampler* s);
int64_t nls_vocab(const nls_sampler* s);

/*
 * accept (sampler.nim:41-43), batched.  Appends up to `count` ids to every
 * row's history: ids is host memory [batch x count], row-major.  Any int64 is
 * accepted; ids outside [0, vocab) occupy a history slot and are skipped by
 * the penalties, as in the reference (:70).  The one exception is
 * NLS_ACCEPT_SKIP, which appends nothing: a batched generation loop passes it
 * for rows that accept nothing this step (the reference loop never accepts an
 * end-of-generation id, src/nimllm/chat.nim:206-208).
 */
#define NLS_ACCEPT_SKIP INT64_MIN
#define NLS_ACCEPT_SKIP32 INT32_MIN /* the same for nls_accept_device's int32 ids */
int nls_accept(nls_sampler* s, const int64_t* ids, int32_t count);
/* accept for one row only (NLS_ACCEPT_SKIP entries append nothing). */
int nls_accept_row(nls_sampler* s, int32_t row, const int64_t* ids, int32_t count);
/* Appends one id per row straight from device memory (e.g. the previous
 * nls_sample output), without a host round trip.  d_ids: device [batch];
 * a row whose entry is NLS_ACCEPT_SKIP32 appends nothing. */
int nls_accept_device(nls_sampler* s, const int32_t* d_ids);

/* One step of batched generation (several contexts' decode loops sharing this
 * handle, one row each; src/nimllm/chat.nim:204-208 per row): every row with
 * d_done[b] == 0 samples as nls_sample does (d_u or the row's own RNG); a row
 * whose id is one of the end-of-generation ids d_eog[0..n_eog) gets
 * d_done[b] = 1 and accepts nothing, the others accept their id on the device.
 * A row with d_done[b] != 0 on entry samples nothing, draws nothing from its
 * RNG and gets d_out[b] = -1, as a finished context stops calling sample.
 * d_done: device [batch], zeroed by the caller before the first step;
 * d_eog: device [n_eog].  Asynchronous on the handle's stream. */
int nls_generate_step(nls_sampler* s, const float* d_logits, const double* d_u, int32_t* d_out,
                      const int32_t* d_eog, int32_t n_eog, int32_t* d_done);
/* Drops every row's history (a fresh newSampler keeps none). */
int nls_clear_history(nls_sampler* s);

/*
 * sample (sampler.nim:59-121), batched and asynchronous.
 *   d_logits  device [batch x vocab] fp32, row-major; read only, never modified
 *   d_u       device [batch] float64 uniforms in [0,1) standing for each row's
 *             rand(1.0) (:117); NULL draws from each row's own RNG, advancing
 *             it only for rows with temperature > 0, as the reference does
 *   d_out     device [batch] int32 sampled ids
 *   dbg       optional inspection output (NULL for none)
 */
int nls_sample(nls_sampler* s, const float* d_logits, const double* d_u, int32_t* d_out,
               const nls_debug* dbg);

/* Blocking convenience for host-resident logits (a CPU model's output):
 * samples h_logits [batch x vocab] with the rows' own RNGs and returns the
 * ids in h_out [batch] -- `s.sample(logits)` of sampler.nim:59 for a CPU
 * model.  The first call allocates a pinned host staging area (hipHostMalloc)
 * held by the handle; each call copies the logits there, and up to 8 MiB of
 * logits the kernels read them from it directly (larger batches go to device
 * memory first); the kernels write the ids back there, and one stream
 * synchronisation ends the call. */
int nls_sample_host(nls_sampler* s, const float* h_logits, int64_t* h_out);

/* No counterpart in the reference: nls_sample_host for callers that cannot
 * allocate (a serving loop or harness that forbids hipMalloc after set-up).
 * It allocates nothing, on the device or the host: the logits and ids are
 * staged in a 16 MiB device array of the library (one per GPU, set up by
 * nls_create on the device current there, held until the process ends), so
 * batch x vocab x 4 bytes (+ 4 bytes per row) must fit 16 MiB, else
 * NLS_ERR_UNSUPPORTED.  Same results as nls_sample_host.  Every call on one
 * GPU shares that array: calls that overlap on one GPU (other threads, other
 * handles' streams) race and must be serialised by the caller. */
int nls_sample_host_noalloc(nls_sampler* s, const float* h_logits, int64_t* h_out);

int nls_synchronize(nls_sampler* s);

/* The first n values of rand(1.0) after initRand(seed) (Nim std/random). */
int nls_rng_uniforms(int64_t seed, int64_t n, double* out);
/* Reads back row `row`'s RNG state (two 64-bit words), e.g. to checkpoint. */
int nls_get_rng_state(nls_sampler* s, int32_t row, uint64_t* a0, uint64_t* a1);
int nls_set_rng_state(nls_sampler* s, int32_t row, uint64_t a0, uint64_t a1);

/* topTokens (src/nimllm/sampler.nim:123-130): for each of `rows` rows of
 * d_logits [rows x vocab] (device, row-major), softmaxInPlace over the whole row
 * (:51-57: maximum, exp(l - max), fp32 sum in index order, division), then the
 * first m = min(n, vocab) entries of the stable sort by probability, descending
 * (equal probabilities keep ascending ids).  Row r's ids and probabilities go
 * to d_ids[r * n + j] and d_probs[r * n + j], j < m.  Asynchronous on `stream`.
 * m <= 0 or rows == 0 does nothing; m > 2048 is NLS_ERR_INVALID_ARGUMENT.
 * Rows holding NaN (or +inf with other values) have NaN probabilities, whose
 * order the reference's comparator leaves undefined: ids 0.. m-1 are returned. */
int nls_top_tokens(const float* d_logits, int32_t rows, int64_t vocab, int32_t n, int32_t* d_ids,
                   float* d_probs, void* stream);

/* argmax (src/nimllm/sampler.nim:45-49) of each of `rows` rows of d_logits
 * [rows x vocab] (device, row-major): d_out[r] = the first index of the
 * row's greatest value.  As in the reference, a NaN is never taken, a NaN at
 * index 0 answers 0, and vocab == 0 answers 0 for every row.  Bit-exact (an
 * index).  Asynchronous on `stream`; vocab >= 2^29 is
 * NLS_ERR_INVALID_ARGUMENT. */
int nls_argmax(const float* d_logits, int32_t rows, int64_t vocab, int32_t* d_out, void* stream);

/* perplexity's per-position term (src/nimllm/model.nim:578-583): for each of
 * `rows` rows of d_logits [rows x vocab] (device, row-major) and its target id
 * d_targets[r] in [0, vocab), d_out[r] = -(float64(l[t] - mx) - ln(s)), with mx
 * the float32 maximum of the row (NaN entries skipped, as Nim's max keeps mx)
 * and s the float64 sum of exp(float64(l - mx)), the subtraction in float32.
 * The sum runs in a fixed tree order on the device, not the reference's index
 * order, so d_out matches the reference within rounding (relative 1e-12), not
 * bit for bit.  Asynchronous on `stream`; targets outside [0, vocab) give NaN. */
int nls_row_nll(const float* d_logits, int32_t rows, int64_t vocab, const int32_t* d_targets,
                double* d_out, void* stream);

/* softmaxInPlace (src/nimllm/sampler.nim:51-57) on each of `rows` rows of
 * d_logits [rows x vocab] (device, row-major): d_out[r * vocab + i] =
 * exp(l_i - mx) / s, with mx the row's float32 maximum (NaN entries skipped, as
 * Nim's max keeps mx), exp correctly rounded (the sampler's exp) and s the
 * fp32 sum of the exponentials added one at a time in index order -- bit for
 * bit the reference's values under that exp.  d_out may equal d_logits (the
 * reference's in-place form).  Asynchronous on `stream`. */
int nls_softmax_rows(const float* d_logits, int32_t rows, int64_t vocab, float* d_out, void* stream);

/* logProb's per-token term (nimllm-doc-en.md:1700-1707: `var p = logits;
 * softmaxInPlace(p); result += ln(p[id].float)`): for each of `rows` rows and
 * its target id d_targets[r], d_prob[r] = p[target] as float32 (bit for bit,
 * as nls_softmax_rows computes it) and d_logp[r] = ln(float64(d_prob[r])) (the
 * device's float64 log, within 1 ulp of the C library's).  Summing d_logp over
 * a continuation's positions gives logProb.  Targets outside [0, vocab) give
 * NaN.  Asynchronous on `stream`. */
int nls_log_prob(const float* d_logits, int32_t rows, int64_t vocab, const int32_t* d_targets, float* d_prob,
                 double* d_logp, void* stream);

/* Correctly rounded exp on fp32 inputs, on the device: d_out[i] = exp(d_in[i]). */
int nls_expf_device(const float* d_in, float* d_out, int64_t n, void* stream);

/* Measurement hook (no counterpart in the reference): when set, the next
 * nls_sample records hipEvent_t `start` immediately before and `stop`
 * immediately after its streaming kernel (the one full read of the logits), on
 * the handle's stream, then clears the hook.  Pass NULLs to clear it. */
int nls_profile_next(nls_sampler* s, void* start_event, void* stop_event);
/* The same around the next call's whole-row kernel (full-sort rows), when the
 * call launches one. */
int nls_profile_next_generic(nls_sampler* s, void* start_event, void* stop_event);

/* Introspection (no counterpart in the reference): how nls_sample runs this
 * handle's batch, for byte accounting in measurements. */
typedef struct nls_plan {
  int32_t stream_threads;  /* workgroup size of the streaming kernel             */
  int32_t slices;          /* streaming workgroups per row                       */
  int32_t generic_launch;  /* 1: a second kernel serves the full-sort rows       */
  int32_t streamed_rows;   /* rows the streaming kernel runs to the end          */
  int64_t first_unit_bytes;/* logits a non-streamed row's workgroup requests before it leaves */
  int32_t k64;             /* 1: the streaming kernel is k64_kernel (1024 threads, k <= 64) */
  int32_t walk_split;      /* 1: the full-sort rows' walks over their groups run in a launch of their own,
                              one wave per row (more full-sort rows than CUs)    */
  int32_t floor_slices;    /* > 0: every row is a full sort, split over this many workgroups that keep the
                              values near the row maximum (rows x slices <= 2 x CUs); the second kernel
                              takes the rows they leave */
} nls_plan;
/* row_streamed: NULL or host [batch], 1 where the streaming kernel runs the row. */
int nls_get_plan(const nls_sampler* s, nls_plan* out, int32_t* row_streamed);

const char* nls_status_string(int status);
/* Last HIP error text seen by this thread ("" if none). */
const char* nls_last_error(void);

#ifdef __cplusplus
}
#endif
#endif
