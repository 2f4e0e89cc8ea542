// nls_api.cpp -- host side of the C ABI in include/nimllm_sampler.h.
//
// Owns the per-handle device state (row parameters, bias tables, history
// rings, RNG states, scratch) and orders every launch on the handle's stream.
// Mirrors src/nimllm/sampler.nim: newSampler (:37-39), accept (:41-43),
// sample (:59-121), the presets (:28-35) and std/random's initRand.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <new>
#include <random>
#include <string>
#include <vector>

#include "../../include/nimllm_sampler.h"
#include "../../include/nimllm_lmhead.h"
#include "nls_internal.h"

using namespace nls;

namespace {

thread_local std::string g_last_error;

int hip_fail(hipError_t e, const char* what) {
  g_last_error = std::string(what) + ": " + hipGetErrorString(e);
  return e == hipErrorOutOfMemory ? NLS_ERR_OUT_OF_MEMORY : NLS_ERR_HIP;
}

#define NLS_HIP(call)                                   \
  do {                                                  \
    hipError_t e_ = (call);                             \
    if (e_ != hipSuccess) return hip_fail(e_, #call);   \
  } while (0)

// Nim std/random: initRand(seed) -- seed 0 -> int32.high, a0 = seed shr 16,
// a1 = seed and 0xffff, jump (skipRandomNumbers), then one discarded `next`.
struct NimRand {
  uint64_t a0, a1;
};
inline uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
uint64_t nim_next(NimRand& r) {
  const uint64_t s0 = r.a0;
  uint64_t s1 = r.a1;
  const uint64_t res = s0 + s1;
  s1 ^= s0;
  r.a0 = rotl(s0, 55) ^ s1 ^ (s1 << 14);
  r.a1 = rotl(s1, 36);
  return res;
}
NimRand nim_init_rand(int64_t seed) {
  const int64_t s = seed != 0 ? seed : 2147483647LL;
  NimRand r{(uint64_t)(s >> 16), (uint64_t)(s & 0xffff)};
  const uint64_t jump[2] = {0xbeac0467eba5facbULL, 0xd86b048b86aa9922ULL};
  uint64_t j0 = 0, j1 = 0;
  for (uint64_t w : jump)
    for (int b = 0; b < 64; ++b) {
      if (w & (1ULL << b)) {
        j0 ^= r.a0;
        j1 ^= r.a1;
      }
      (void)nim_next(r);
    }
  r.a0 = j0;
  r.a1 = j1;
  (void)nim_next(r);
  return r;
}
double nim_rand_unit(NimRand& r) {
  const uint64_t x = nim_next(r);
  const uint64_t bits = (0x3FFULL << 52) | (x >> 12);
  double f;
  std::memcpy(&f, &bits, sizeof f);
  return f - 1.0;
}

// Staging of nls_sample_host_noalloc: the logits, then the ids, of one call.
// A file-scope device array, so that the entry point allocates nothing; every
// GPU the library runs on holds its own copy (16 MiB) until the process ends.
// In host code `scratch` names a host-side stand-in, never the device memory:
// its device address is taken once per device (scratch_device) and only that
// address is used.
constexpr size_t kNoAllocBytes = size_t{16} << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocBytes];
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on device `dev` (which must be current).
int scratch_device(int dev, void** out) {
  *out = nullptr;
  if (dev < 0 || dev >= kMaxDevices) {
    g_last_error = "device ordinal beyond the scratch table";
    return NLS_ERR_UNSUPPORTED;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (!p) {
      g_last_error = "hipGetSymbolAddress(scratch) returned no address";
      return NLS_ERR_HIP;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return NLS_OK;
}

template <typename T>
int dalloc(T** p, size_t n) {
  *p = nullptr;
  if (n == 0) return NLS_OK;
  NLS_HIP(hipMalloc(reinterpret_cast<void**>(p), n * sizeof(T)));
  return NLS_OK;
}
template <typename T>
void dfree(T*& p) {
  if (p) (void)hipFree(p);
  p = nullptr;
}

}  // namespace

struct nls_sampler {
  int B = 0;
  int64_t V = 0;
  int device = 0;        // the device current at nls_create
  void* scratch = nullptr;  // that device's address of `scratch`
  hipStream_t stream = nullptr;
  int max_bias = 0;
  int bstride = 0;  // > 0: bias lists at a fixed stride (row b at b * bstride)

  std::vector<RowParams> h_rp;
  std::vector<int64_t> h_len;     // accepted ids per row (an upper bound while !len_exact)
  bool len_exact = true;          // false after nls_accept_device, whose rows may skip
  std::vector<int> need_window;   // repeat_last_n (>0) or -1 (whole history), 0 if unused
  int hcap = 0;

  // streaming-kernel plan
  LaunchPlan plan{};
  int S = 1, L = 0, xcd_map = 0;
  int ccap = 0, nwords = 0, pcap = 0, mcap = 0, kcap = 0, offA = 0, pc = 0;
  int parity = 0;  // which generic counter this call uses
  // the split launches' counters of each parity may hold counts: a call that
  // splits leaves them in its parity's set, a whole-row launch zeroes the
  // other parity's, a call served inline by the streaming kernel leaves both
  bool split_dirty[2] = {false, false};
  // set when a call failed after some of its kernels may have run: the
  // counters it would have handed on are cleared before the next call
  bool counters_dirty = false;
  int hbits = 0;   // k64_kernel's hash table: 2^hbits slots

  RowParams* rp = nullptr;
  int32_t* bias_ids = nullptr;
  float* bias_vals = nullptr;
  int32_t* hist = nullptr;
  int64_t* hist_len = nullptr;
  uint64_t* part_cand = nullptr;
  SliceInfo* part_info = nullptr;
  uint32_t* arrive = nullptr;
  uint64_t* rng = nullptr;
  int32_t* generic_list = nullptr;
  int32_t* generic_count = nullptr;  // [8]: handed-on, claim, fallback and walk counts (each by call parity)
  int32_t* fb_list = nullptr;        // [B] the rows the grouped launch leaves to the whole-row launch
  double* fb_u = nullptr;            // [B] their uniforms, when drawn there
  // the grouped rows' walks in a launch of their own (many full-sort rows per CU)
  bool walk_split = false;
  float* gt_e = nullptr;      // [B * kGrpHashCap]
  uint32_t* gt_c = nullptr;   // [B * kGrpHashCap]
  uint32_t* gt_k = nullptr;   // [B * kGrpHashCap]
  int32_t* gt_n = nullptr;    // [B]
  int32_t* w_list = nullptr;  // [B]
  uint32_t* p3_rec = nullptr; // [B]
  uint32_t* p3_key = nullptr; // [B]
  int64_t* p3_t = nullptr;    // [B]
  // floor_kernel's slice records (a batch of full sorts only, no more rows than CUs)
  uint64_t* floor_part = nullptr;  // [B][S][kFloorKeep]
  int32_t* floor_n = nullptr;      // [B][S]
  uint32_t* floor_max = nullptr;   // [B][S]
  int32_t* all_rows = nullptr;       // no streaming rows: 0 .. B-1, then B (the count), then a spare
  // k64_kernel with full-sort rows in the batch: the streamed rows (its
  // grid) and the others (the whole-row kernel's fixed list)
  int32_t* k64_list = nullptr;
  int32_t* full_list = nullptr;
  int n_k64_list = 0, n_full_list = 0;
  uint32_t* done = nullptr;          // workgroups finished (whole-row rows served inline)
  int gen_inline = 0;
  uint32_t* gen_scratch = nullptr;
  int64_t gen_vpad = 0;
  int gen_scratch_blocks = 0;  // whole-row workgroups gen_scratch holds
  int ncu = 256;
  int32_t* stage_ids = nullptr;  // staged ids, then one append count per staged row
  size_t stage_cap = 0;
  std::vector<int32_t> h_stage;
  float* tmp_logits = nullptr;
  int32_t* tmp_out = nullptr;
  // nls_sample_host's pinned staging (hipHostMalloc, set up by its first
  // call): the logits and, 256 bytes on, the int32 ids; host_stage_dev is the
  // same memory as the device sees it
  unsigned char* host_stage = nullptr;
  unsigned char* host_stage_dev = nullptr;
  hipEvent_t prof_start = nullptr;
  hipEvent_t prof_stop = nullptr;
  hipEvent_t prof_gstart = nullptr;
  hipEvent_t prof_gstop = nullptr;

  ~nls_sampler() {
    dfree(rp);
    dfree(bias_ids);
    dfree(bias_vals);
    dfree(hist);
    dfree(hist_len);
    dfree(part_cand);
    dfree(part_info);
    dfree(arrive);
    dfree(rng);
    dfree(generic_list);
    dfree(generic_count);
    dfree(fb_list);
    dfree(fb_u);
    dfree(gt_e);
    dfree(gt_c);
    dfree(gt_k);
    dfree(gt_n);
    dfree(w_list);
    dfree(p3_rec);
    dfree(p3_key);
    dfree(p3_t);
    dfree(floor_part);
    dfree(floor_n);
    dfree(floor_max);
    dfree(all_rows);
    dfree(k64_list);
    dfree(full_list);
    dfree(done);
    dfree(gen_scratch);
    dfree(stage_ids);
    dfree(tmp_logits);
    dfree(tmp_out);
    if (host_stage) (void)hipHostFree(host_stage);
  }

  // True when a row the streaming kernel runs may patch more distinct ids
  // (history window + bias entries) than its LDS table holds: such a row is
  // handed on to the whole-row path, which then gets a launch of its own
  // across the CUs rather than the streaming kernel's last workgroup.
  bool window_may_overflow() const {
    const int64_t cap = plan.k64 ? (int64_t)((1 << hbits) - (1 << hbits) / 4) : (int64_t)pcap;
    for (int b = 0; b < B; ++b) {
      const RowParams& r = h_rp[b];
      if (!r.fast) continue;
      int64_t w = 0;
      if (need_window[b] != 0) w = need_window[b] > 0 ? std::min<int64_t>(need_window[b], h_len[b]) : h_len[b];
      if (w + r.bias_cnt > cap) return true;
    }
    return false;
  }

  // Grows the history ring so that every row's window fits after `extra`
  // more ids are appended to row `row` (every row when row < 0).  Re-lays the
  // ring out on the host.
  int ensure_history(int row, int64_t extra) {
    int64_t need = 0;
    for (int b = 0; b < B; ++b) {
      if (need_window[b] == 0) continue;
      const int64_t len = h_len[b] + ((row < 0 || row == b) ? extra : 0);
      const int64_t w = need_window[b] > 0 ? std::min<int64_t>(need_window[b], len) : len;
      need = std::max(need, w);
    }
    if (need <= hcap && hist) return NLS_OK;
    if (hist && !len_exact) {
      // rows that skipped a device accept: the device lengths are the true ones
      NLS_HIP(hipMemcpyAsync(h_len.data(), hist_len, sizeof(int64_t) * B, hipMemcpyDeviceToHost, stream));
      NLS_HIP(hipStreamSynchronize(stream));
      len_exact = true;
      return ensure_history(row, extra);
    }
    int64_t ncap = std::max<int64_t>(hcap, 16);
    while (ncap < need) ncap *= 2;
    if (ncap > (1 << 24)) {
      g_last_error = "history window beyond 2^24 ids";
      return NLS_ERR_UNSUPPORTED;
    }
    int32_t* nh = nullptr;
    int rc = dalloc(&nh, (size_t)B * ncap);
    if (rc) return rc;
    if (hist) {
      std::vector<int32_t> old((size_t)B * hcap), neu((size_t)B * ncap, -1);
      NLS_HIP(hipMemcpyAsync(old.data(), hist, old.size() * 4, hipMemcpyDeviceToHost, stream));
      NLS_HIP(hipStreamSynchronize(stream));
      for (int b = 0; b < B; ++b) {
        const int64_t len = h_len[b];
        const int64_t keep = std::min<int64_t>(len, hcap);
        for (int64_t j = len - keep; j < len; ++j)
          neu[(size_t)b * ncap + (size_t)(j % ncap)] = old[(size_t)b * hcap + (size_t)(j % hcap)];
      }
      NLS_HIP(hipMemcpyAsync(nh, neu.data(), neu.size() * 4, hipMemcpyHostToDevice, stream));
      NLS_HIP(hipStreamSynchronize(stream));
    }
    dfree(hist);
    hist = nh;
    hcap = (int)ncap;
    return NLS_OK;
  }
};

namespace {

int next_pow2_i(int64_t n) {
  int p = 1;
  while (p < n) p <<= 1;
  return p;
}

int env_int(const char* name, int dflt) {
  const char* v = std::getenv(name);
  return (v && *v) ? std::atoi(v) : dflt;
}

// Streaming-kernel geometry for a batch: workgroup size, slices per row, LDS
// layout, and the largest k the streaming kernel takes (larger k rows go to
// the whole-row kernel).
struct Geometry {
  int nt, S, L, ccap, nwords, pcap, mcap, kcap, offA, pc, q;
  bool wave;
  size_t lds;
};

Geometry plan_geometry(int B, int64_t V, int kmax, int ncu, int max_patch) {
  Geometry g{};
  // Top-k rows past the wave path (k > 64) on a batch of at least two rows
  // per CU: 512-thread workgroups whose LDS leaves room for two per CU, so
  // that one row's selection and tail run while the other row streams.
  if (kmax > kWaveTopK && B >= 2 * ncu && max_patch >= 0 && env_int("NLS_STREAM_NT", 512) == 512) {
    Geometry d{};
    d.nt = 512;
    d.S = 1;
    d.L = (int)((V + 3) / 4 * 4);
    d.pc = 0;
    d.wave = false;
    d.ccap = next_pow2_i(std::max<int64_t>(1024, 2LL * kmax));
    d.nwords = (int)((V + 31) / 32);
    d.mcap = next_pow2_i(std::max(2 * kmax, 2));
    d.kcap = kmax;
    d.q = 1;
    while (d.q < 8 && (int64_t)d.q * d.nt < 2LL * kmax) d.q <<= 1;
    const size_t cand = (size_t)2 * d.ccap * 8;
    const size_t head = (size_t)d.nwords * 4 + (((size_t)d.nwords * 2 + 3) & ~(size_t)3);
    const size_t tail = (size_t)d.mcap * 8 + (size_t)d.kcap * 12;
    const size_t target = kDualStreamLds;
    d.offA = (int)cand;
    if (cand + head < target) d.pcap = (int)std::min<size_t>(65535, (target - cand - head) / 16);
    d.lds = cand + std::max(head + (size_t)d.pcap * 16, tail);
    if (d.lds <= target && d.pcap >= std::max(max_patch, 1)) return d;
  }
  // 256-thread workgroups, >= 4 per CU: rows are split into S slices until the
  // grid holds about 4 workgroups per CU, keeping >= 2 tiles per slice.
  // a whole row per 1024-thread workgroup once the batch fills the chip, or
  // when a row is small enough that one workgroup streams it faster than the
  // slices of a split row exchange their candidates (V = 32000, B = 1: 18.9
  // against 23.9 us per call); otherwise rows are split over 256-thread
  // workgroups
  g.nt = env_int("NLS_STREAM_NT", (B >= ncu || V <= kSmallRowV) ? 1024 : 256) == 1024 ? 1024 : 256;
  const int64_t te = (int64_t)g.nt * kStreamVec4 * 4;
  const int want = g.nt == 1024 ? 1 : std::max(1, (4 * ncu + B - 1) / B);
  g.S = std::max(1, env_int("NLS_STREAM_S", want));
  g.S = (int)std::min<int64_t>({(int64_t)g.S, std::max<int64_t>(1, V / (2 * te)), (int64_t)kMaxSlices});
  g.S = std::max(g.S, 1);
  int64_t L = (V + g.S - 1) / g.S;
  L = (L + 3) / 4 * 4;
  g.S = (int)((V + L - 1) / L);
  g.L = (int)L;
  const int k = std::max(kmax, 1);
  g.pc = g.S > 1 ? (2 * k + 64 + 7) / 8 * 8 : 0;
  g.wave = kmax <= kWaveTopK;
  g.ccap = next_pow2_i(std::max<int64_t>({1024, 4LL * k, ((int64_t)g.S * g.pc + 1) / 2}));
  if (g.wave) g.ccap = std::max(g.ccap, g.nt / 64 * kWaveCap);  // one buffer region per wave
  if (g.S > 1) g.pc = std::max(g.pc, (2 * g.ccap / g.S) / 8 * 8);
  g.nwords = (int)((L + 31) / 32);
  g.mcap = next_pow2_i(std::max(2 * k, 2));
  g.kcap = k;
  g.q = 1;
  while (g.q < 8 && (int64_t)g.q * g.nt < 2LL * k) g.q <<= 1;
  const size_t cand = (size_t)2 * g.ccap * 8;
  const size_t head = (size_t)g.nwords * 4 + (((size_t)g.nwords * 2 + 3) & ~(size_t)3);
  const size_t tail = (size_t)g.mcap * 8 + (size_t)g.kcap * 12;
  g.offA = (int)cand;
  // room for 4 workgroups per CU (160 KB of LDS), more when k or V need it
  const size_t target = (size_t)(g.nt == 1024 ? 140 : 31) * 1024;
  const size_t min_lds = cand + std::max(head + (size_t)256 * 16, tail);
  const size_t lds = std::min(std::max(target, min_lds), nls::max_dynamic_lds());
  g.pcap = 0;  // 16 bytes per patched id: final value, bias, flags, id
  if (cand + head < lds) g.pcap = (int)std::min<size_t>(65535, (lds - cand - head) / 16);
  g.lds = cand + std::max(head + (size_t)g.pcap * 16, tail);
  return g;
}

}  // namespace

extern "C" {

nls_params nls_default_sampling(void) {
  nls_params p;
  std::memset(&p, 0, sizeof p);
  p.temperature = 0.7;
  p.top_k = 40;
  p.top_p = 0.95;
  p.min_p = 0.05;
  p.repeat_penalty = 1.1;
  p.repeat_last_n = 64;
  p.seed = -1;
  return p;
}

nls_params nls_greedy_sampling(void) {
  nls_params p;
  std::memset(&p, 0, sizeof p);
  p.temperature = 0.0;
  p.top_k = 0;
  p.top_p = 1.0;
  p.repeat_penalty = 1.0;
  p.seed = 0;
  return p;
}

const char* nls_status_string(int status) {
  switch (status) {
    case NLS_OK: return "ok";
    case NLS_ERR_INVALID_ARGUMENT: return "invalid argument";
    case NLS_ERR_EMPTY_VOCAB: return "empty vocabulary";
    case NLS_ERR_HIP: return "HIP runtime error";
    case NLS_ERR_OUT_OF_MEMORY: return "out of device memory";
    case NLS_ERR_NO_DEVICE: return "no usable device";
    case NLS_ERR_UNSUPPORTED: return "unsupported size";
    default: return "unknown status";
  }
}

const char* nls_last_error(void) { return g_last_error.c_str(); }

int nls_rng_uniforms(int64_t seed, int64_t n, double* out) {
  if (n < 0 || (n > 0 && !out)) return NLS_ERR_INVALID_ARGUMENT;
  NimRand r = nim_init_rand(seed);
  for (int64_t i = 0; i < n; ++i) out[i] = nim_rand_unit(r);
  return NLS_OK;
}

int nls_create(const nls_params* per_row, int32_t batch, int64_t vocab, void* stream,
               nls_sampler** out) {
  if (!out) return NLS_ERR_INVALID_ARGUMENT;
  *out = nullptr;
  if (!per_row || batch < 1) return NLS_ERR_INVALID_ARGUMENT;
  if (vocab <= 0) return NLS_ERR_EMPTY_VOCAB;
  if (vocab >= (1LL << 31) - 16) {
    g_last_error = "vocab beyond 2^31";
    return NLS_ERR_UNSUPPORTED;
  }
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev < 1) {
    g_last_error = "no HIP device";
    return NLS_ERR_NO_DEVICE;
  }
  nls_sampler* s = new (std::nothrow) nls_sampler();
  if (!s) return NLS_ERR_OUT_OF_MEMORY;
  s->B = batch;
  s->V = vocab;
  s->stream = reinterpret_cast<hipStream_t>(stream);
  const int B = batch;
  const int V = (int)vocab;
  s->h_rp.resize(B);
  s->h_len.assign(B, 0);
  s->need_window.assign(B, 0);

  // bias tables: per row, in-range ids, last value wins, sorted by id
  std::vector<int32_t> bid;
  std::vector<float> bval;
  std::vector<NimRand> rng_h(B);
  std::random_device rd;
  int kmax = 0;
  int max_patch = 0;  // patched ids a row can need (window + bias); -1: unbounded window
  for (int b = 0; b < B; ++b) {
    const nls_params& p = per_row[b];
    if (p.logit_bias_count < 0 || (p.logit_bias_count > 0 &&
                                   (!p.logit_bias_ids || !p.logit_bias_values))) {
      delete s;
      return NLS_ERR_INVALID_ARGUMENT;
    }
    std::map<int64_t, double> table;
    for (int64_t j = 0; j < p.logit_bias_count; ++j) table[p.logit_bias_ids[j]] = p.logit_bias_values[j];
    RowParams& r = s->h_rp[b];
    std::memset(&r, 0, sizeof r);
    r.bias_off = (int32_t)bid.size();
    for (const auto& kv : table) {
      if (kv.first < 0 || kv.first >= vocab) continue;  // sampler.nim:76
      bid.push_back((int32_t)kv.first);
      bval.push_back((float)kv.second);
    }
    r.bias_cnt = (int32_t)bid.size() - r.bias_off;
    s->max_bias = std::max(s->max_bias, (int)r.bias_cnt);
    r.rp32 = (float)p.repeat_penalty;
    r.minP32 = (float)p.min_p;
    r.pen_active = (p.repeat_penalty != 1.0 || p.presence_penalty != 0 || p.frequency_penalty != 0);
    r.rp_active = p.repeat_penalty != 1.0;
    r.topp_active = (p.top_p > 0 && p.top_p < 1);
    r.minp_active = p.min_p > 0;
    r.topP = p.top_p;
    r.freq = p.frequency_penalty;
    r.pres = p.presence_penalty;
    r.repeat_last_n = p.repeat_last_n;
    if (p.temperature <= 0) {
      r.mode = kModeGreedy;
      r.invT = 1.0f;
      r.k = V;
    } else {
      r.invT = (float)(1.0 / p.temperature);
      const int64_t k = p.top_k > 0 ? std::min<int64_t>(p.top_k, vocab) : vocab;
      r.k = (int32_t)k;
      r.mode = k < vocab ? kModeTopK : kModeFull;
      if (r.mode == kModeTopK && k <= kMaxTopKFast) kmax = std::max(kmax, (int)k);
    }
    if (r.pen_active) s->need_window[b] = p.repeat_last_n > 0 ? (int)std::min<int64_t>(p.repeat_last_n, 1 << 24) : -1;
    if (max_patch >= 0) {
      if (r.pen_active && p.repeat_last_n <= 0)
        max_patch = -1;
      else
        max_patch = std::max(max_patch, (r.pen_active ? (int)std::min<int64_t>(p.repeat_last_n, 1 << 24) : 0) +
                                            (int)r.bias_cnt);
    }
    int64_t seed = p.seed;
    if (seed < 0) {
      const uint64_t t = (uint64_t)std::chrono::high_resolution_clock::now().time_since_epoch().count();
      seed = (int64_t)((((uint64_t)rd() << 32) ^ rd() ^ t) & 0x7fffffffffffffffULL);
    }
    rng_h[b] = nim_init_rand(seed);
  }
  // streaming geometry: the largest k whose buffers fit in LDS
  int dev = 0, ncu = 0;
  (void)hipGetDevice(&dev);
  s->device = dev;
  {
    // the no-allocation entry point's staging on this device, set up here
    const int rc0 = scratch_device(dev, &s->scratch);
    if (rc0) {
      delete s;
      return rc0;
    }
  }
  if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || ncu < 1)
    ncu = 256;
  int kfast = kmax;
  Geometry g = plan_geometry(B, vocab, kfast, ncu, max_patch);
  while (kfast > 0 && (g.lds > max_dynamic_lds() || (g.nt != 512 && g.pcap < 256))) {
    kfast = kfast * 7 / 8;
    g = plan_geometry(B, vocab, kfast, ncu, max_patch);
  }
  // (false only for vocabularies far beyond 2^19; the slice's byte size must
  // also fit the 32-bit range of the kernel's buffer loads)
  const bool stream_ok = g.lds <= max_dynamic_lds() && g.pcap >= 1 && g.L < (1 << 28);
  if (!stream_ok) g.lds = 0;                    // every row then goes to the whole-row kernel
  bool any_full = false;
  for (int b = 0; b < B; ++b) {
    RowParams& r = s->h_rp[b];
    r.fast = stream_ok && (r.mode == kModeGreedy || (r.mode == kModeTopK && r.k <= kfast)) ? 1 : 0;
    any_full |= !r.fast;
  }
  s->S = g.S;
  s->L = g.L;
  s->xcd_map = (g.S > 1 && B % 8 == 0) ? 1 : 0;
  s->ccap = g.ccap;
  s->nwords = g.nwords;
  s->pcap = g.pcap;
  s->mcap = g.mcap;
  s->kcap = g.kcap;
  s->offA = g.offA;
  s->pc = g.pc;
  s->plan.nt = g.nt;
  s->plan.q = g.q;
  s->plan.wave = g.wave;
  s->plan.lds = g.lds;
  // Greedy and top-k <= 64 rows streamed whole by 1024-thread workgroups run
  // k64_kernel, its patch hash table as large as the LDS allows.
  s->plan.k64 = false;
  s->plan.k64_rows = kK64RowsAny;
  s->hbits = 0;
  if (stream_ok && g.wave && g.nt == 1024 && g.S == 1 && env_int("NLS_K64", 1)) {
    int hb = 0;
    for (int b = 8; b <= 12; ++b)
      if (k64_lds_bytes(vocab, b) <= kK64MaxDynLds) hb = b;
    if (hb > 0) {
      s->plan.k64 = true;
      s->hbits = hb;
      s->plan.lds = k64_lds_bytes(vocab, hb);
      // the instance for the kinds of streamed rows present
      bool any_greedy = false, any_topk = false;
      for (int b = 0; b < B; ++b) {
        if (!s->h_rp[b].fast) continue;
        any_greedy |= s->h_rp[b].mode == kModeGreedy;
        any_topk |= s->h_rp[b].mode == kModeTopK;
      }
      if (any_greedy != any_topk) s->plan.k64_rows = any_greedy ? kK64RowsGreedy : kK64RowsTopK;
    }
  }
  // Without full-sort rows the whole-row kernel only serves the rare row the
  // streaming kernel hands on: one workgroup keeps that launch cheap.
  bool any_fast = false;
  for (int b = 0; b < B; ++b) any_fast |= s->h_rp[b].fast != 0;
  // A batch without streaming rows (full sorts only) runs the whole-row
  // kernel alone over a fixed list of every row.
  s->plan.no_stream = !any_fast;
  // A batch of full sorts only whose row slices all fit the GPU at once (two
  // workgroups per CU): each row is split over slices (floor_kernel), and the
  // whole-row kernel takes the rows that cannot be finished from the values
  // near their maximum.  Past one round of slices the grouped path, one row
  // per CU, is faster (the slices' serial merge latency repeats each round).
  s->plan.floor_slices = 0;
  if (s->plan.no_stream && env_int("NLS_FLOOR", 1)) {
    bool all_full = true;
    for (int b = 0; b < B; ++b) all_full &= s->h_rp[b].mode == kModeFull;
    const int64_t S = (vocab + kFloorSlice - 1) / kFloorSlice;
    if (all_full && S <= kFloorMaxSlices && (int64_t)B * S <= 2 * (int64_t)ncu) s->plan.floor_slices = (int)S;
  }
  s->plan.gen_blocks = any_full ? std::min(B, 256) : 1;
  s->plan.gen_lds = group_lds_bytes(vocab);
  // ... and then its last workgroup serves that row itself, saving a launch
  s->gen_inline = any_full ? 0 : 1;

  int rc = NLS_OK;
  auto fail = [&](int code) {
    delete s;
    return code;
  };
  {
    const hipError_t e = set_kernel_attributes();
    if (e != hipSuccess) return fail(hip_fail(e, "hipFuncSetAttribute"));
  }
  // Bias lists of at most one workgroup's width go to a fixed stride, so the
  // streaming kernel can request them before it has read the row constants.
  if (s->max_bias > 0 && s->max_bias <= 256 && (int64_t)B * s->max_bias <= (1 << 24)) {
    const int st = s->max_bias;
    std::vector<int32_t> sid((size_t)B * st, -1);
    std::vector<float> sval((size_t)B * st, 0.0f);
    for (int b = 0; b < B; ++b) {
      RowParams& r = s->h_rp[b];
      for (int j = 0; j < r.bias_cnt; ++j) {
        sid[(size_t)b * st + j] = bid[(size_t)r.bias_off + j];
        sval[(size_t)b * st + j] = bval[(size_t)r.bias_off + j];
      }
      r.bias_off = b * st;
    }
    bid.swap(sid);
    bval.swap(sval);
    s->bstride = st;
  }
  if ((rc = dalloc(&s->rp, B))) return fail(rc);
  if ((rc = dalloc(&s->bias_ids, std::max<size_t>(bid.size(), 1)))) return fail(rc);
  if ((rc = dalloc(&s->bias_vals, std::max<size_t>(bval.size(), 1)))) return fail(rc);
  if ((rc = dalloc(&s->hist_len, B))) return fail(rc);
  if (s->S > 1) {
    if ((rc = dalloc(&s->part_cand, (size_t)B * s->S * s->pc))) return fail(rc);
    if ((rc = dalloc(&s->part_info, (size_t)B * s->S))) return fail(rc);
  }
  if ((rc = dalloc(&s->arrive, B))) return fail(rc);
  if ((rc = dalloc(&s->rng, (size_t)2 * B))) return fail(rc);
  if ((rc = dalloc(&s->generic_list, B))) return fail(rc);
  if ((rc = dalloc(&s->generic_count, 8))) return fail(rc);  // the launches' counters (by call parity)
  if (s->plan.gen_lds > 0) {
    if ((rc = dalloc(&s->fb_list, B))) return fail(rc);
    if ((rc = dalloc(&s->fb_u, B))) return fail(rc);
    // Many full-sort rows per CU: their walks (single-wave serial work) run
    // side by side in a launch of their own instead of one after another on
    // each CU, so the groups are stored between the launches.
    int n_full = 0;
    for (int b = 0; b < B; ++b) n_full += s->h_rp[b].mode == kModeFull ? 1 : 0;
    if (n_full > ncu && env_int("NLS_WALK_SPLIT", 1)) {
      const size_t cells = (size_t)B * kGrpHashCap;
      if ((rc = dalloc(&s->gt_e, cells))) return fail(rc);
      if ((rc = dalloc(&s->gt_c, cells))) return fail(rc);
      if ((rc = dalloc(&s->gt_k, cells))) return fail(rc);
      if ((rc = dalloc(&s->gt_n, B))) return fail(rc);
      if ((rc = dalloc(&s->w_list, B))) return fail(rc);
      if ((rc = dalloc(&s->p3_rec, B))) return fail(rc);
      if ((rc = dalloc(&s->p3_key, B))) return fail(rc);
      if ((rc = dalloc(&s->p3_t, B))) return fail(rc);
      s->walk_split = true;
      s->plan.walk_blocks = std::min((B + kWalkRows - 1) / kWalkRows, 2 * ncu);  // two workgroups per CU
      s->plan.walk_lds = walk_member_lds_bytes(vocab);
    }
  }
  if (s->plan.floor_slices > 0) {
    const size_t parts = (size_t)B * s->plan.floor_slices;
    if ((rc = dalloc(&s->floor_part, parts * kFloorKeep))) return fail(rc);
    if ((rc = dalloc(&s->floor_n, parts))) return fail(rc);
    if ((rc = dalloc(&s->floor_max, parts))) return fail(rc);
  }
  if (s->plan.no_stream) {
    std::vector<int32_t> rows((size_t)B + 2);
    for (int b = 0; b < B; ++b) rows[b] = b;
    rows[B] = B;
    rows[B + 1] = 0;
    if ((rc = dalloc(&s->all_rows, rows.size()))) return fail(rc);
    const hipError_t e0 = hipMemcpy(s->all_rows, rows.data(), rows.size() * 4, hipMemcpyHostToDevice);
    if (e0 != hipSuccess) return fail(hip_fail(e0, "upload row list"));
  }
  if (s->plan.k64 && any_full && any_fast) {
    // Rows that are not streamed would only hand themselves on from a
    // workgroup of their own; with random kinds that leaves some CUs many
    // more streamed rows than others.  The grid takes the streamed rows
    // alone, and the whole-row kernel the others from a fixed list.
    std::vector<int32_t> fast, full;
    for (int b = 0; b < B; ++b) (s->h_rp[b].fast ? fast : full).push_back(b);
    if ((rc = dalloc(&s->k64_list, fast.size()))) return fail(rc);
    if ((rc = dalloc(&s->full_list, full.size()))) return fail(rc);
    hipError_t e0 = hipMemcpy(s->k64_list, fast.data(), fast.size() * 4, hipMemcpyHostToDevice);
    if (e0 == hipSuccess) e0 = hipMemcpy(s->full_list, full.data(), full.size() * 4, hipMemcpyHostToDevice);
    if (e0 != hipSuccess) return fail(hip_fail(e0, "upload row lists"));
    s->n_k64_list = (int)fast.size();
    s->n_full_list = (int)full.size();
  }
  if ((rc = dalloc(&s->done, 1))) return fail(rc);
  int64_t vpad = 1;
  while (vpad < vocab) vpad <<= 1;
  s->gen_vpad = vpad;
  if ((rc = dalloc(&s->gen_scratch, (size_t)s->plan.gen_blocks * vpad * 5))) return fail(rc);
  s->gen_scratch_blocks = s->plan.gen_blocks;
  s->ncu = ncu;
  if ((rc = s->ensure_history(-1, 0))) return fail(rc);

  hipStream_t st = s->stream;
  auto up = [&](void* dst, const void* src, size_t bytes) {
    return hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, st);
  };
  hipError_t e;
  if ((e = up(s->rp, s->h_rp.data(), sizeof(RowParams) * B)) != hipSuccess)
    return fail(hip_fail(e, "upload params"));
  if (!bid.empty()) {
    if ((e = up(s->bias_ids, bid.data(), bid.size() * 4)) != hipSuccess)
      return fail(hip_fail(e, "upload bias"));
    if ((e = up(s->bias_vals, bval.data(), bval.size() * 4)) != hipSuccess)
      return fail(hip_fail(e, "upload bias"));
  }
  if ((e = up(s->hist_len, s->h_len.data(), sizeof(int64_t) * B)) != hipSuccess)
    return fail(hip_fail(e, "upload history"));
  if ((e = up(s->rng, rng_h.data(), sizeof(NimRand) * B)) != hipSuccess)
    return fail(hip_fail(e, "upload rng"));
  if ((e = hipMemsetAsync(s->arrive, 0, sizeof(uint32_t) * B, st)) != hipSuccess)
    return fail(hip_fail(e, "clear counters"));
  if ((e = hipMemsetAsync(s->done, 0, sizeof(uint32_t), st)) != hipSuccess)
    return fail(hip_fail(e, "clear counters"));
  if ((e = hipMemsetAsync(s->generic_count, 0, sizeof(int32_t) * 8, st)) != hipSuccess)
    return fail(hip_fail(e, "clear counters"));
  if ((e = hipStreamSynchronize(st)) != hipSuccess) return fail(hip_fail(e, "sync"));
  *out = s;
  return NLS_OK;
}

int nls_destroy(nls_sampler* s) {
  if (!s) return NLS_ERR_INVALID_ARGUMENT;
  (void)hipStreamSynchronize(s->stream);
  delete s;
  return NLS_OK;
}

int nls_set_stream(nls_sampler* s, void* stream) {
  if (!s) return NLS_ERR_INVALID_ARGUMENT;
  s->stream = reinterpret_cast<hipStream_t>(stream);
  return NLS_OK;
}

int32_t nls_batch(const nls_sampler* s) { return s ? s->B : 0; }
int64_t nls_vocab(const nls_sampler* s) { return s ? s->V : 0; }

static int accept_impl(nls_sampler* s, int row, const int64_t* ids, int32_t count) {
  if (!s || count < 0 || (count > 0 && !ids)) return NLS_ERR_INVALID_ARGUMENT;
  if (row >= s->B) return NLS_ERR_INVALID_ARGUMENT;
  if (count == 0) return NLS_OK;
  const int rows = row >= 0 ? 1 : s->B;
  // Stage each row's appended ids (NLS_ACCEPT_SKIP entries dropped) at
  // [r * count, ...), then the per-row counts after all rows.
  const size_t n = (size_t)rows * count;
  s->h_stage.assign(n + rows, -1);
  std::vector<int64_t> add(rows, 0);
  for (int r = 0; r < rows; ++r) {
    int c = 0;
    for (int j = 0; j < count; ++j) {
      const int64_t id = ids[(size_t)r * count + j];
      if (id == NLS_ACCEPT_SKIP) continue;
      s->h_stage[(size_t)r * count + c++] = (id >= 0 && id < s->V) ? (int32_t)id : -1;  // out of range: skipped later
    }
    s->h_stage[n + r] = c;
    add[r] = c;
  }
  int64_t most = 0;
  for (int r = 0; r < rows; ++r) most = std::max(most, add[r]);
  if (most == 0) return NLS_OK;
  int rc = s->ensure_history(row, most);
  if (rc) return rc;
  if (n + rows > s->stage_cap) {
    dfree(s->stage_ids);
    rc = dalloc(&s->stage_ids, n + rows);
    if (rc) return rc;
    s->stage_cap = n + rows;
  }
  NLS_HIP(hipMemcpyAsync(s->stage_ids, s->h_stage.data(), (n + rows) * 4, hipMemcpyHostToDevice,
                         s->stream));
  NLS_HIP(launch_accept_host(s->stage_ids, s->stage_ids + n, s->B, count, s->hist, s->hist_len,
                             s->hcap, row, s->stream));
  NLS_HIP(hipStreamSynchronize(s->stream));
  if (row >= 0)
    s->h_len[row] += add[0];
  else
    for (int b = 0; b < s->B; ++b) s->h_len[b] += add[b];
  return NLS_OK;
}

int nls_accept(nls_sampler* s, const int64_t* ids, int32_t count) {
  return accept_impl(s, -1, ids, count);
}

int nls_accept_row(nls_sampler* s, int32_t row, const int64_t* ids, int32_t count) {
  if (row < 0) return NLS_ERR_INVALID_ARGUMENT;
  return accept_impl(s, row, ids, count);
}

int nls_accept_device(nls_sampler* s, const int32_t* d_ids) {
  if (!s || !d_ids) return NLS_ERR_INVALID_ARGUMENT;
  int rc = s->ensure_history(-1, 1);
  if (rc) return rc;
  NLS_HIP(launch_accept_device(d_ids, s->B, s->V, s->hist, s->hist_len, s->hcap, s->stream));
  // a row may skip (NLS_ACCEPT_SKIP32): the host lengths become upper bounds
  for (int b = 0; b < s->B; ++b) s->h_len[b] += 1;
  s->len_exact = false;
  return NLS_OK;
}

int nls_clear_history(nls_sampler* s) {
  if (!s) return NLS_ERR_INVALID_ARGUMENT;
  std::fill(s->h_len.begin(), s->h_len.end(), 0);
  s->len_exact = true;
  NLS_HIP(hipMemcpyAsync(s->hist_len, s->h_len.data(), sizeof(int64_t) * s->B,
                         hipMemcpyHostToDevice, s->stream));
  NLS_HIP(hipStreamSynchronize(s->stream));
  return NLS_OK;
}

namespace {
// One nls_sample call; may_alloc = false for the no-allocation entry point
// (which then leaves handed-on rows to the streaming kernel's last workgroup).
int sample_impl(nls_sampler* s, const float* d_logits, const double* d_u, int32_t* d_out,
                const nls_debug* dbg, bool may_alloc, const int32_t* d_done = nullptr) {
  if (!s || !d_logits || !d_out) return NLS_ERR_INVALID_ARGUMENT;
  if (dbg && dbg->cap < 0) return NLS_ERR_INVALID_ARGUMENT;
  DebugPtrs dp;
  std::memset(&dp, 0, sizeof dp);
  if (dbg) {
    dp.n = dbg->n;
    dp.ncand = dbg->ncand;
    dp.cand_ids = dbg->cand_ids;
    dp.cand_probs = dbg->cand_probs;
    dp.total = dbg->total;
    dp.path = dbg->path;
    dp.cap = dbg->cap;
  }
  if (s->counters_dirty) {
    NLS_HIP(launch_clear_counters(s->arrive, s->B, s->done, s->generic_count, s->stream));
    s->parity = 0;
    s->counters_dirty = false;
    s->split_dirty[0] = s->split_dirty[1] = false;
  }
  int32_t* cnt_now = s->generic_count + s->parity;
  int32_t* cnt_next = s->generic_count + (s->parity ^ 1);
  StreamArgs a;
  std::memset(&a, 0, sizeof a);
  a.logits = d_logits;
  a.V = s->V;
  a.B = s->B;
  a.S = s->S;
  a.L = s->L;
  a.xcd_map = s->xcd_map;
  a.rp = s->rp;
  a.hist = s->hist;
  a.hist_len = s->hist_len;
  a.hcap = s->hcap;
  a.bias_ids = s->bias_ids;
  a.bias_vals = s->bias_vals;
  a.bstride = s->bstride;
  a.ccap = s->ccap;
  a.nwords = s->nwords;
  a.pcap = s->pcap;
  a.mcap = s->mcap;
  a.kcap = s->kcap;
  a.offA = s->offA;
  a.part_cand = s->part_cand;
  a.part_info = s->part_info;
  a.arrive = s->arrive;
  a.pc = s->pc;
  a.d_u = d_u;
  a.rng = s->rng;
  a.out = d_out;
  a.generic_list = s->generic_list;
  a.generic_count = cnt_now;
  a.dbg = dp;
  GenericArgs ga;
  std::memset(&ga, 0, sizeof ga);
  ga.logits = d_logits;
  ga.V = s->V;
  ga.rp = s->rp;
  ga.hist = s->hist;
  ga.hist_len = s->hist_len;
  ga.hcap = s->hcap;
  ga.bias_ids = s->bias_ids;
  ga.bias_vals = s->bias_vals;
  ga.generic_list = s->generic_list;
  ga.generic_count = cnt_now;
  ga.next_count = cnt_next;
  ga.list_cap = s->B;
  if (!s->gen_inline && !s->plan.no_stream) {
    // every call of this sampler launches the whole-row kernel, which zeroes
    // the next call's claim counter
    ga.claim = s->generic_count + 2 + s->parity;
    ga.next_claim = s->generic_count + 2 + (s->parity ^ 1);
  }
  ga.scratch = s->gen_scratch;
  ga.vpad = s->gen_vpad;
  ga.d_u = d_u;
  ga.rng = s->rng;
  ga.out = d_out;
  ga.dbg = dp;
  ga.grouped = s->plan.gen_lds > 0 ? 1 : 0;
  // every call zeroes the other parity's counters of the split launches
  // (whichever of its kernels runs), so calls of either form can follow
  if (s->fb_list) ga.fb_next = s->generic_count + 4 + (s->parity ^ 1);
  if (s->walk_split) {
    ga.w_next = s->generic_count + 6 + (s->parity ^ 1);
  }
  // (after floor_kernel the whole-row launch usually finds no row: one launch)
  if (ga.grouped && s->fb_list && !dp.cand_ids && !dp.cand_probs && s->plan.floor_slices == 0) {
    // the grouped rows in a launch of their own, then the rows it leaves
    // (candidate lists are written by the whole-row sort, so a call asking
    // for them keeps the one launch, where a grouped row is sorted as well)
    ga.fb_list = s->fb_list;
    ga.fb_count = s->generic_count + 4 + s->parity;
    ga.fb_u = s->fb_u;
    if (s->walk_split) {
      ga.walk_split = 1;
      ga.gt_e = s->gt_e;
      ga.gt_c = s->gt_c;
      ga.gt_k = s->gt_k;
      ga.gt_n = s->gt_n;
      ga.w_list = s->w_list;
      ga.w_count = s->generic_count + 6 + s->parity;
      ga.p3_rec = s->p3_rec;
      ga.p3_key = s->p3_key;
      ga.p3_t = s->p3_t;
    }
  }
  LaunchPlan lp = s->plan;
  a.gen_inline = s->gen_inline;
  if (a.gen_inline && s->window_may_overflow()) {
    const int want = std::min(s->B, s->ncu);
    if (s->gen_scratch_blocks < want && may_alloc) {
      uint32_t* ns = nullptr;
      const int rc = dalloc(&ns, (size_t)want * s->gen_vpad * 5);
      if (rc) return rc;
      NLS_HIP(hipStreamSynchronize(s->stream));  // the old scratch may still be in use
      dfree(s->gen_scratch);
      s->gen_scratch = ns;
      s->gen_scratch_blocks = want;
      ga.scratch = ns;
    }
    if (s->gen_scratch_blocks >= want) {
      a.gen_inline = 0;
      lp.gen_blocks = want;
    }
  }
  a.done = s->done;
  a.hbits = s->hbits;
  a.row_done = d_done;
  ga.row_done = d_done;
  FloorArgs fa;
  std::memset(&fa, 0, sizeof fa);
  if (lp.floor_slices > 0) {
    // every row through floor_kernel; the whole-row launch takes the rows it lists
    fa.logits = d_logits;
    fa.V = s->V;
    fa.B = s->B;
    fa.S = lp.floor_slices;
    fa.rp = s->rp;
    fa.hist = s->hist;
    fa.hist_len = s->hist_len;
    fa.hcap = s->hcap;
    fa.bias_ids = s->bias_ids;
    fa.bias_vals = s->bias_vals;
    fa.bstride = s->bstride;
    fa.d_u = d_u;
    fa.rng = s->rng;
    fa.out = d_out;
    fa.dbg = dp;
    fa.row_done = d_done;
    fa.generic_list = s->generic_list;
    fa.generic_count = cnt_now;
    fa.part = s->floor_part;
    fa.part_n = s->floor_n;
    fa.part_max = s->floor_max;
    fa.arrive = s->arrive;
    a.gen_inline = 0;
  } else if (lp.no_stream) {
    // every row, a constant count (the spare slot takes the kernel's reset of
    // the next call's counter)
    ga.generic_list = s->all_rows;
    ga.generic_count = s->all_rows + s->B;
    ga.next_count = s->all_rows + s->B + 1;
    a.gen_inline = 0;
  }
  if (s->k64_list && !lp.no_stream) {
    a.row_list = s->k64_list;
    a.n_list = s->n_k64_list;
    ga.fixed_list = s->full_list;
    ga.n_fixed = s->n_full_list;
  }
  a.ga = ga;
  lp.vec4 = (s->V % 4 == 0) && ((reinterpret_cast<uintptr_t>(d_logits) & 15) == 0);
  hipEvent_t e0 = s->prof_start, e1 = s->prof_stop, g0 = s->prof_gstart, g1 = s->prof_gstop;
  s->prof_start = s->prof_stop = s->prof_gstart = s->prof_gstop = nullptr;
  // A call that splits the whole-row launches counts in its parity's split
  // counters; counts a split call two back left there (the call between was
  // served inline, so nothing zeroed them) are cleared first.
  const bool whole_row = !a.gen_inline;
  const bool splits = whole_row && ga.fb_list != nullptr;
  if (splits && s->split_dirty[s->parity]) {
    NLS_HIP(launch_clear_counters(s->arrive, s->B, s->done, s->generic_count, s->stream));
    s->split_dirty[0] = s->split_dirty[1] = false;
  }
  const hipError_t le = launch_sample(a, ga, fa, lp, s->stream, e0, e1, g0, g1);
  if (le != hipSuccess) {
    // a kernel of this call may have run and left its counters for the next
    s->counters_dirty = true;
    return hip_fail(le, "launch_sample");
  }
  if (whole_row) s->split_dirty[s->parity ^ 1] = false;  // zeroed by the whole-row launches
  if (splits) s->split_dirty[s->parity] = true;
  s->parity ^= 1;
  return NLS_OK;
}
}  // namespace

int nls_sample(nls_sampler* s, const float* d_logits, const double* d_u, int32_t* d_out,
               const nls_debug* dbg) {
  return sample_impl(s, d_logits, d_u, d_out, dbg, true);
}

int nls_generate_step(nls_sampler* s, const float* d_logits, const double* d_u, int32_t* d_out,
                      const int32_t* d_eog, int32_t n_eog, int32_t* d_done) {
  if (!s || !d_logits || !d_out || !d_done || n_eog < 0 || (n_eog > 0 && !d_eog)) return NLS_ERR_INVALID_ARGUMENT;
  int rc = s->ensure_history(-1, 1);
  if (rc) return rc;
  rc = sample_impl(s, d_logits, d_u, d_out, nullptr, true, d_done);
  if (rc) return rc;
  NLS_HIP(launch_generate_step(d_out, s->B, s->V, d_eog, n_eog, d_done, s->hist, s->hist_len, s->hcap, s->stream));
  // rows that finished (or had finished) append nothing: the host lengths
  // become upper bounds
  for (int b = 0; b < s->B; ++b) s->h_len[b] += 1;
  s->len_exact = false;
  return NLS_OK;
}

int nls_profile_next(nls_sampler* s, void* start_event, void* stop_event) {
  if (!s || (!start_event) != (!stop_event)) return NLS_ERR_INVALID_ARGUMENT;
  s->prof_start = reinterpret_cast<hipEvent_t>(start_event);
  s->prof_stop = reinterpret_cast<hipEvent_t>(stop_event);
  return NLS_OK;
}

int nls_profile_next_generic(nls_sampler* s, void* start_event, void* stop_event) {
  if (!s || (!start_event) != (!stop_event)) return NLS_ERR_INVALID_ARGUMENT;
  s->prof_gstart = reinterpret_cast<hipEvent_t>(start_event);
  s->prof_gstop = reinterpret_cast<hipEvent_t>(stop_event);
  return NLS_OK;
}

int nls_get_plan(const nls_sampler* s, nls_plan* out, int32_t* row_streamed) {
  if (!s || !out) return NLS_ERR_INVALID_ARGUMENT;
  std::memset(out, 0, sizeof *out);
  out->stream_threads = s->plan.lds > 0 ? s->plan.nt : 0;
  out->slices = s->S;
  out->generic_launch = s->gen_inline ? 0 : 1;
  out->k64 = s->plan.k64 ? 1 : 0;
  out->walk_split = s->walk_split ? 1 : 0;
  out->floor_slices = s->plan.floor_slices;
  // a workgroup requests its first unit (kStreamVec4 float4 per thread)
  // before it reads the row's constants
  out->first_unit_bytes = (s->plan.lds > 0 && !s->plan.no_stream)
                              ? std::min<int64_t>((int64_t)s->S * s->plan.nt * kStreamVec4 * 16, s->V * 4)
                              : 0;
  for (int b = 0; b < s->B; ++b) {
    const int f = s->h_rp[b].fast ? 1 : 0;
    out->streamed_rows += f;
    if (row_streamed) row_streamed[b] = f;
  }
  return NLS_OK;
}

// Up to this many bytes of logits, nls_sample_host's kernels read them
// straight from the pinned staging (one transfer fewer in a call's chain of
// latencies); larger batches are copied to device memory first.
constexpr size_t kHostDirectBytes = size_t{8} << 20;

int nls_sample_host(nls_sampler* s, const float* h_logits, int64_t* h_out) {
  if (!s || !h_logits || !h_out) return NLS_ERR_INVALID_ARGUMENT;
  const size_t n = (size_t)s->B * s->V;
  const size_t ids_off = (n * 4 + 255) & ~(size_t)255;
  int rc;
  if (!s->host_stage) {
    void* h = nullptr;
    void* d = nullptr;
    NLS_HIP(hipHostMalloc(&h, ids_off + (size_t)s->B * 4, hipHostMallocDefault));
    const hipError_t e = hipHostGetDevicePointer(&d, h, 0);
    if (e != hipSuccess) {
      (void)hipHostFree(h);
      return hip_fail(e, "hipHostGetDevicePointer");
    }
    s->host_stage = static_cast<unsigned char*>(h);
    s->host_stage_dev = static_cast<unsigned char*>(d);
  }
  // the previous call ended with a synchronisation: the staging is free
  std::memcpy(s->host_stage, h_logits, n * 4);
  const float* d_logits = reinterpret_cast<const float*>(s->host_stage_dev);
  if (n * 4 > kHostDirectBytes) {
    if (!s->tmp_logits && (rc = dalloc(&s->tmp_logits, n))) return rc;
    NLS_HIP(hipMemcpyAsync(s->tmp_logits, s->host_stage, n * 4, hipMemcpyHostToDevice, s->stream));
    d_logits = s->tmp_logits;
  }
  // the ids are written by the kernel into the pinned staging
  rc = nls_sample(s, d_logits, nullptr, reinterpret_cast<int32_t*>(s->host_stage_dev + ids_off), nullptr);
  if (rc) {
    // a kernel of the failed call may still read the staging
    (void)hipStreamSynchronize(s->stream);
    return rc;
  }
  NLS_HIP(hipStreamSynchronize(s->stream));
  for (int b = 0; b < s->B; ++b) {
    int32_t v;
    std::memcpy(&v, s->host_stage + ids_off + (size_t)4 * b, sizeof v);
    h_out[b] = v;
  }
  return NLS_OK;
}

int nls_sample_host_noalloc(nls_sampler* s, const float* h_logits, int64_t* h_out) {
  if (!s || !h_logits || !h_out) return NLS_ERR_INVALID_ARGUMENT;
  const size_t n = (size_t)s->B * (size_t)s->V;
  const size_t ids_off = (n * 4 + 255) & ~(size_t)255;
  if (ids_off + (size_t)s->B * 4 > kNoAllocBytes) {
    g_last_error = "nls_sample_host_noalloc: batch x vocab x 4 bytes (+ the ids) exceeds its " +
                   std::to_string(kNoAllocBytes >> 20) + " MiB staging; use nls_sample_host";
    return NLS_ERR_UNSUPPORTED;
  }
  if (!s->scratch) {
    g_last_error = "nls_sample_host_noalloc: no staging address for the handle's device";
    return NLS_ERR_HIP;
  }
  unsigned char* base = static_cast<unsigned char*>(s->scratch);
  float* d_logits = reinterpret_cast<float*>(base);
  int32_t* d_out = reinterpret_cast<int32_t*>(base + ids_off);
  NLS_HIP(hipMemcpyAsync(d_logits, h_logits, n * 4, hipMemcpyHostToDevice, s->stream));
  const int rc = sample_impl(s, d_logits, nullptr, d_out, nullptr, false);
  if (rc) return rc;
  // the int32 ids land in the first half of h_out's bytes and are widened in
  // place, from the last one down (no host buffer either; each narrow id is
  // read as bytes before its slot's wide store can overlap it)
  unsigned char* bytes = reinterpret_cast<unsigned char*>(h_out);
  NLS_HIP(hipMemcpyAsync(bytes, d_out, (size_t)s->B * 4, hipMemcpyDeviceToHost, s->stream));
  NLS_HIP(hipStreamSynchronize(s->stream));
  for (int b = s->B - 1; b >= 0; --b) {
    int32_t v;
    std::memcpy(&v, bytes + (size_t)4 * b, sizeof v);
    h_out[b] = v;
  }
  return NLS_OK;
}

int nls_synchronize(nls_sampler* s) {
  if (!s) return NLS_ERR_INVALID_ARGUMENT;
  NLS_HIP(hipStreamSynchronize(s->stream));
  return NLS_OK;
}

int nls_get_rng_state(nls_sampler* s, int32_t row, uint64_t* a0, uint64_t* a1) {
  if (!s || row < 0 || row >= s->B || !a0 || !a1) return NLS_ERR_INVALID_ARGUMENT;
  uint64_t st[2];
  NLS_HIP(hipMemcpyAsync(st, s->rng + 2 * row, 16, hipMemcpyDeviceToHost, s->stream));
  NLS_HIP(hipStreamSynchronize(s->stream));
  *a0 = st[0];
  *a1 = st[1];
  return NLS_OK;
}

int nls_set_rng_state(nls_sampler* s, int32_t row, uint64_t a0, uint64_t a1) {
  if (!s || row < 0 || row >= s->B) return NLS_ERR_INVALID_ARGUMENT;
  uint64_t st[2] = {a0, a1};
  NLS_HIP(hipMemcpyAsync(s->rng + 2 * row, st, 16, hipMemcpyHostToDevice, s->stream));
  NLS_HIP(hipStreamSynchronize(s->stream));
  return NLS_OK;
}

int nls_top_tokens(const float* d_logits, int32_t rows, int64_t vocab, int32_t n, int32_t* d_ids,
                   float* d_probs, void* stream) {
  // (the kernel addresses a row in bytes with 32-bit offsets)
  if (rows < 0 || vocab < 0 || vocab >= (int64_t{1} << 29)) return NLS_ERR_INVALID_ARGUMENT;
  const int64_t m = std::min<int64_t>(n, vocab);  // topTokens returns min(n, len) entries (:130)
  if (rows == 0 || m <= 0) return NLS_OK;
  if (m > nls::kTopMaxN || !d_logits || !d_ids || !d_probs) return NLS_ERR_INVALID_ARGUMENT;
  NLS_HIP(launch_top_tokens(d_logits, rows, vocab, n, d_ids, d_probs,
                            reinterpret_cast<hipStream_t>(stream)));
  return NLS_OK;
}

int nls_row_nll(const float* d_logits, int32_t rows, int64_t vocab, const int32_t* d_targets,
                double* d_out, void* stream) {
  // (the kernel addresses a row in bytes with 32-bit offsets)
  if (rows < 0 || vocab < 0 || vocab >= (int64_t{1} << 29)) return NLS_ERR_INVALID_ARGUMENT;
  if (rows == 0) return NLS_OK;
  if (vocab == 0) return NLS_ERR_EMPTY_VOCAB;
  if (!d_logits || !d_targets || !d_out) return NLS_ERR_INVALID_ARGUMENT;
  NLS_HIP(launch_row_nll(d_logits, rows, vocab, d_targets, d_out, reinterpret_cast<hipStream_t>(stream)));
  return NLS_OK;
}

int nls_argmax(const float* d_logits, int32_t rows, int64_t vocab, int32_t* d_out, void* stream) {
  // (the kernel addresses a row in bytes with 32-bit offsets)
  if (rows < 0 || vocab < 0 || vocab >= (int64_t{1} << 29)) return NLS_ERR_INVALID_ARGUMENT;
  if (rows == 0) return NLS_OK;
  if (!d_out || (vocab > 0 && !d_logits)) return NLS_ERR_INVALID_ARGUMENT;
  NLS_HIP(launch_argmax(d_logits, rows, vocab, d_out, reinterpret_cast<hipStream_t>(stream)));
  return NLS_OK;
}

int nls_softmax_rows(const float* d_logits, int32_t rows, int64_t vocab, float* d_out, void* stream) {
  // (the kernel addresses a row in bytes with 32-bit offsets)
  if (rows < 0 || vocab < 0 || vocab >= (int64_t{1} << 29)) return NLS_ERR_INVALID_ARGUMENT;
  if (rows == 0) return NLS_OK;
  if (vocab == 0) return NLS_ERR_EMPTY_VOCAB;
  if (!d_logits || !d_out) return NLS_ERR_INVALID_ARGUMENT;
  NLS_HIP(launch_softmax_rows(d_logits, rows, vocab, d_out, reinterpret_cast<hipStream_t>(stream)));
  return NLS_OK;
}

int nls_log_prob(const float* d_logits, int32_t rows, int64_t vocab, const int32_t* d_targets, float* d_prob,
                 double* d_logp, void* stream) {
  if (rows < 0 || vocab < 0 || vocab >= (int64_t{1} << 29)) return NLS_ERR_INVALID_ARGUMENT;
  if (rows == 0) return NLS_OK;
  if (vocab == 0) return NLS_ERR_EMPTY_VOCAB;
  if (!d_logits || !d_targets || !d_prob || !d_logp) return NLS_ERR_INVALID_ARGUMENT;
  NLS_HIP(launch_log_prob(d_logits, rows, vocab, d_targets, d_prob, d_logp,
                          reinterpret_cast<hipStream_t>(stream)));
  return NLS_OK;
}

int nls_expf_device(const float* d_in, float* d_out, int64_t n, void* stream) {
  if (n < 0 || (n > 0 && (!d_in || !d_out))) return NLS_ERR_INVALID_ARGUMENT;
  NLS_HIP(launch_expf(d_in, d_out, n, reinterpret_cast<hipStream_t>(stream)));
  return NLS_OK;
}

}  // extern "C"

// ---------------------------------------------------------------- LM head

namespace {

// blockSize / typeSize (quant.nim:38-63) of the types the reference reads
int lm_block_size(int t) {
  switch (t) {
    case 0: case 1: case 30: return 1;
    case 2: case 3: case 6: case 7: case 8: return 32;
    case 10: case 11: case 12: case 13: case 14: case 15: return 256;
    default: return 0;
  }
}
int lm_type_bytes(int t) {
  switch (t) {
    case 0: return 4;
    case 1: case 30: return 2;
    case 2: return 18;
    case 3: return 20;
    case 6: return 22;
    case 7: return 24;
    case 8: return 34;
    case 10: return 84;
    case 11: return 110;
    case 12: return 144;
    case 13: return 176;
    case 14: return 210;
    case 15: return 292;
    default: return 0;
  }
}
size_t align256(size_t n) { return (n + 255) & ~size_t{255}; }

// model.nim:184-185
bool lm_uses_act(int type, int64_t cols, int nb, bool exact) {
  const int bl = lm_act_block_len(type);
  return !exact && bl > 0 && cols % bl == 0 && (nb <= 4 || type != 8);
}

// workspace: [act qs][act d][lora tmp], each 256-byte aligned
struct LmLayout {
  size_t qs = 0, d = 0, tmp = 0, total = 0;
};
LmLayout lm_layout(int type, int64_t cols, int nb, int rank, bool exact) {
  LmLayout L;
  if (lm_uses_act(type, cols, nb, exact)) {
    const int64_t n = (int64_t)nb * cols;
    L.d = align256((size_t)n);
    L.tmp = L.d + align256(sizeof(float) * (size_t)(n / lm_act_block_len(type)));
  }
  L.total = L.tmp + (rank > 0 ? align256(sizeof(float) * (size_t)nb * (size_t)rank) : 0);
  return L;
}

}  // namespace

extern "C" {

int64_t nls_lm_head_row_bytes(int32_t type, int64_t cols) {
  if (!lm_type_supported(type) || cols <= 0 || cols % lm_block_size(type) != 0) return -1;
  return cols / lm_block_size(type) * lm_type_bytes(type);
}

size_t nls_lm_head_workspace(int32_t type, int64_t cols, int32_t nb, int32_t lora_rank, int32_t exact) {
  if (!lm_type_supported(type) || cols <= 0 || nb < 0 || lora_rank < 0) return 0;
  if (cols % lm_block_size(type) != 0) return 0;
  return lm_layout(type, cols, nb, lora_rank, exact != 0).total;
}

int32_t nls_lm_head(const void* d_weight, int32_t type, int64_t rows, int64_t cols, const float* d_x, int32_t nb,
                    float* d_y, int32_t exact, const nls_lora* lora, void* d_work, size_t work_bytes,
                    void* stream) {
  if (!lm_type_supported(type) || rows < 0 || cols <= 0 || nb < 0) return NLS_ERR_INVALID_ARGUMENT;
  // rowBytes raises for a row that is not whole blocks (quant.nim:65-70)
  if (cols % lm_block_size(type) != 0 || cols >= (int64_t{1} << 28) || rows >= (int64_t{1} << 40))
    return NLS_ERR_INVALID_ARGUMENT;
  if (rows == 0 || nb == 0) return NLS_OK;
  if (!d_weight || !d_x || !d_y) return NLS_ERR_INVALID_ARGUMENT;
  if ((reinterpret_cast<uintptr_t>(d_weight) & 15) || (reinterpret_cast<uintptr_t>(d_x) & 15) ||
      (reinterpret_cast<uintptr_t>(d_y) & 3))
    return NLS_ERR_INVALID_ARGUMENT;
  const int rank = lora ? lora->rank : 0;
  if (rank < 0 || (rank > 0 && (!lora->d_a || !lora->d_b))) return NLS_ERR_INVALID_ARGUMENT;
  const bool ex = exact != 0;
  const LmLayout L = lm_layout(type, cols, nb, rank, ex);
  if (L.total > 0 && (!d_work || work_bytes < L.total || (reinterpret_cast<uintptr_t>(d_work) & 255)))
    return NLS_ERR_INVALID_ARGUMENT;
  LmHeadCall c{};
  c.w = d_weight;
  c.type = type;
  c.rows = rows;
  c.cols = cols;
  c.row_bytes = cols / lm_block_size(type) * lm_type_bytes(type);
  c.x = d_x;
  c.nb = nb;
  c.y = d_y;
  c.use_act = lm_uses_act(type, cols, nb, ex);
  if (c.use_act && cols / lm_act_block_len(type) > kLmMaxIntBlocks) {
    g_last_error = "nls_lm_head: more than 1024 blocks per row on the int8 path";
    return NLS_ERR_UNSUPPORTED;
  }
  char* wk = static_cast<char*>(d_work);
  c.act_qs = c.use_act ? reinterpret_cast<int8_t*>(wk + L.qs) : nullptr;
  c.act_d = c.use_act ? reinterpret_cast<float*>(wk + L.d) : nullptr;
  c.lora_rank = rank;
  if (rank > 0) {
    c.lora_a = lora->d_a;
    c.lora_b = lora->d_b;
    c.lora_scale = lora->scale;
    c.lora_tmp = reinterpret_cast<float*>(wk + L.tmp);
  }
  NLS_HIP(launch_lm_head(c, reinterpret_cast<hipStream_t>(stream)));
  return NLS_OK;
}

}  // extern "C"
