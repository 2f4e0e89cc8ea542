// nls_kernels.hip -- gfx950 kernels outside the sampler's two main kernels,
// and the launchers nls_api.cpp calls.
//
// nls_sample runs stream_kernel (nls_stream_*.hip: one translation unit per
// workgroup size and load width) and, when full-sort rows are present,
// generic_kernel (nls_generic.hip); both are defined in nls_device.h.  This
// file holds topTokens (top_tokens_kernel), perplexity's per-position term
// (row_nll_kernel), the history-ring appends and the exp test hook.
//
// All fp32/fp64 arithmetic follows the reference's order; this file is built
// with -ffp-contract=off so no multiply-add is fused.
#include "nls_device.h"
#include "nls_launch.h"
#include "nls_seqsum.h"

namespace nls {

// ---------------------------------------------------------------------------
// 3. top_tokens_kernel -- topTokens (sampler.nim:123-130)
// ---------------------------------------------------------------------------
// One workgroup per row: softmaxInPlace (:51-57) over the whole row and the
// first m = min(n, V) entries of the stable sort by probability (:127-128).
// Two reads of the row when m <= 1024:
//   1. each thread's largest logit: their maximum is mx (:52-53; Nim's
//      max(mx, v) keeps mx for a NaN v, as fmaxf does), and the m-th largest
//      of them bounds the row's m-th largest logit from below (they are m
//      distinct elements);
//   2. exp(l - mx) (correctly rounded) chunk by chunk into LDS, summed in
//      index order exactly as one-at-a-time fp32 adds would (nls_seqsum.h),
//      while the elements at or above the bound are listed.
// The probability is non-decreasing in the logit (l - mx, the exp and the
// division by s each are), so the m-th largest probability is p(L) of the m-th
// largest logit L, found among the listed ones, and the entries whose
// probability reaches p(L) are those whose logit is at least l_lo, the lowest
// float with p(l_lo) == p(L) (a bisection on the float's bits).  When l_lo is
// at or above the bound they are all listed: taken with their probabilities,
// sorted by (probability desc, index asc), the first m written.  (Equal
// probabilities can come from different logits: the exp and the division
// round, so the order cannot be taken from the logits.)
// Otherwise (m > 1024, a full list, l_lo below the bound, s not a number) the
// row is read again: the entries at or above l_lo found by an exact radix
// select on the logits, or -- when they are many, or s is NaN -- an exact
// radix select on the probabilities themselves and, among the entries equal
// to the m-th, the lowest indices (a second select on the index), as the
// stable sort keeps them.
// A row holding NaN, or +inf with anything else, has NaN probabilities; the
// reference's comparator is no order on NaN, so such rows are outside the
// parity claim (this kernel then returns the first indices).
namespace {
constexpr int kTopPer = 8;                      // logits per thread and chunk of the sum
constexpr int kTopCh = kTopThreads * kTopPer;   // 8192 exponentials in LDS
constexpr int kTopList = 2048;                  // logits listed at or above the bound
}  // namespace

template <int NT>
__global__ __launch_bounds__(NT) void top_tokens_kernel(const float* __restrict__ logits, int64_t V,
                                                        int n, int32_t* __restrict__ ids,
                                                        float* __restrict__ probs) {
  constexpr int NW = NT / kWave;
  static_assert((size_t)kTopCh * sizeof(float) >= (size_t)kTopMaxN * 2 * sizeof(uint64_t),
                "the members (and the fallback's candidates) reuse the exponentials' buffer");
  static_assert(NT == kTopThreads && kTopPer % 4 == 0, "chunk layout");
  __shared__ __align__(16) float ebuf[kTopCh];
  __shared__ uint64_t list[kTopList];
  __shared__ uint32_t hist[kSelWords];
  __shared__ int smem[NW + 4];
  __shared__ float s_part[NW];
  __shared__ int s_cnt;
  __shared__ SeqSumShared sh;
  __shared__ double s_pow2[kExpfPow2Count];  // the exponential's table
  const int row = (int)blockIdx.x;
  const int tid = (int)threadIdx.x;
  const int lane = lane_id();
  const int wv = tid >> 6;
  const int nV = (int)V;  // V < 2^29 (checked by the host)
  const float* __restrict__ x = logits + (int64_t)row * V;
  const __amdgpu_buffer_rsrc_t xr = slice_rsrc(x, nV);
  const int m = (int)min((int64_t)n, V);  // 1 <= m <= kTopMaxN (checked by the host)
  for (int q = tid; q < kSelWords; q += NT) hist[q] = 0u;
  // 16-byte loads when every row start is 16-byte aligned; element of slot q
  // of this thread in the chunk at c0: float4 group tid + (q / 4) * NT, or
  // element tid + q * NT
  const bool vec = (nV % 4 == 0) && ((reinterpret_cast<uintptr_t>(logits) & 15) == 0);
  auto elem = [&](int c0, int q) -> int {
    return vec ? c0 + 4 * (tid + (q >> 2) * NT) + (q & 3) : c0 + tid + q * NT;
  };
  auto load = [&](int c0, float (&v)[kTopPer]) __attribute__((always_inline)) {
    if (vec) {
#pragma unroll
      for (int g = 0; g < kTopPer / 4; ++g) {
        const int e0 = c0 + 4 * (tid + g * NT);
        const f32x4 t = __builtin_bit_cast(
            f32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, e0 < nV ? e0 * 4 : 0x7ffffff0, 0, 0));
        v[4 * g] = t.x;
        v[4 * g + 1] = t.y;
        v[4 * g + 2] = t.z;
        v[4 * g + 3] = t.w;
      }
    } else {
#pragma unroll
      for (int q = 0; q < kTopPer; ++q) {
        const int e = c0 + tid + q * NT;
        v[q] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(xr, e < nV ? e * 4 : 0x7ffffff0, 0, 0));
      }
    }
  };
  // fn(i, l, in) over the row for the fallback's passes, eight requests per
  // thread in flight at a time (past the row they read 0 with in == false);
  // every lane makes the same number of calls
  constexpr int kScanU = 8;
  auto row_scan = [&](auto fn) __attribute__((always_inline)) {
    for (int i0 = 0; i0 < nV; i0 += NT * kScanU) {
      float l[kScanU];
#pragma unroll
      for (int u = 0; u < kScanU; ++u) {
        const int i = i0 + u * NT + tid;
        l[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                             xr, i < nV ? i * 4 : 0x7ffffff0, 0, 0));
      }
#pragma unroll
      for (int u = 0; u < kScanU; ++u) {
        const int i = i0 + u * NT + tid;
        fn(i, l[u], i < nV);
      }
    }
  };

  // (1) mx and each thread's largest logit key (the next chunk requested
  // before the current one is reduced)
  float mx = -__builtin_inff();
  uint32_t tk = 0u;
  {
    float a[kTopPer], b[kTopPer];
    load(0, a);
    // (after the first chunk's requests; the barrier after this pass orders it)
    if (tid < kExpfPow2Count) s_pow2[tid] = kExpfPow2J64[tid];
    for (int c0 = 0; c0 < nV; c0 += kTopCh) {
      const bool more = c0 + kTopCh < nV;
      if (more) load(c0 + kTopCh, b);
#pragma unroll
      for (int q = 0; q < kTopPer; ++q)
        if (elem(c0, q) < nV) {
          mx = __builtin_fmaxf(mx, a[q]);
          tk = max(tk, f2key(a[q]));
        }
      if (more) {
#pragma unroll
        for (int q = 0; q < kTopPer; ++q) a[q] = b[q];
      }
    }
  }
  for (int o = kWave / 2; o > 0; o >>= 1) mx = __builtin_fmaxf(mx, __shfl_xor(mx, o));
  if (lane == 0) s_part[wv] = mx;
  __syncthreads();
  mx = s_part[0];
  for (int w = 1; w < NW; ++w) mx = __builtin_fmaxf(mx, s_part[w]);
  // the bound: the m-th largest thread maximum, when at least m threads hold
  // an element (else every element is listed)
  uint32_t t0 = 0u;
  const int holders = vec ? min(NT, (nV + 3) / 4) : min(NT, nV);
  if (m <= holders) {
    const SelectResult b0 = block_select<NT>([&](auto fn) { fn(tk, tid < holders); }, m, -1, hist, smem);
    t0 = b0.tau;
  }
  seq_sum_init(sh);
  if (tid == 0) s_cnt = 0;
  __syncthreads();

  // (2) s = e_0 + e_1 + ... in index order (:54-56), listing the logits >= t0
  float s = 0.0f;
  {
    int J = 1, nwin = 0;
    float v[kTopPer];
    load(0, v);
    for (int c0 = 0; c0 < nV; c0 += kTopCh) {
#pragma unroll
      for (int q = 0; q < kTopPer; ++q) {
        const int e = elem(c0, q);
        if (e < nV) {
          ebuf[e - c0] = expf_cr_t(v[q] - mx, s_pow2);
          const uint32_t k = f2key(v[q]);
          if (m <= NT && k >= t0) {
            const int slot = atomicAdd(&s_cnt, 1);
            if (slot < kTopList) list[slot] = ((uint64_t)k << 32) | (uint32_t)e;
          }
        }
      }
      __syncthreads();
      if (c0 + kTopCh < nV) load(c0 + kTopCh, v);
      s = seq_sum_block<NT>(ebuf, min(kTopCh, nV - c0), s, J, nwin, c0, sh);  // ends with a barrier
    }
  }
  const int nl = s_cnt;
  // probs[i] /= s (:57)
  auto prob_of = [&](float l) -> float { return expf_cr_t(l - mx, s_pow2) / s; };
  auto pkey = [&](float l) -> uint32_t { return f2key(prob_of(l)); };

  uint64_t* mem = reinterpret_cast<uint64_t*>(ebuf);
  constexpr int kCand = (int)(sizeof(ebuf) / (sizeof(uint64_t)));
  auto emit = [&](int cnt) {  // mem[0..cnt): key << 32 | ~index; the first m, sorted, out
    const int np = next_pow2(cnt);
    for (int i = cnt + tid; i < np; i += NT) mem[i] = 0ull;  // below every real key
    __syncthreads();
    bitonic_sort_u64<NT>(mem, np, true);
    __syncthreads();
    for (int j = tid; j < m; j += NT) {
      const uint64_t e = mem[j];
      ids[(int64_t)row * n + j] = (int32_t)(0xffffffffu - (uint32_t)e);
      probs[(int64_t)row * n + j] = key2f((uint32_t)(e >> 32));
    }
  };
  // the lowest key in [key(-inf), key(L)] whose probability reaches p(L)
  auto lowest_key = [&](uint32_t kL) -> uint32_t {
    const float pm = prob_of(key2f(kL));
    uint32_t lo = f2key(-__builtin_inff()), hi = kL;
    while (lo < hi) {
      const uint32_t mid = lo + (hi - lo) / 2;
      if (prob_of(key2f(mid)) >= pm)
        hi = mid;
      else
        lo = mid + 1;
    }
    return hi;
  };
  if (s == s && m <= NT && nl <= kTopList) {  // uniform
    // L among the listed logits (it is one of them: L >= t0)
    const SelectResult sl = block_select<NT>(
        [&](auto fn) {
          for (int i0 = 0; i0 < kTopList; i0 += NT) {
            const int i = i0 + tid;
            const bool in = i < nl;
            fn(in ? (uint32_t)(list[i] >> 32) : 0u, in);
          }
        },
        m, -1, hist, smem);
    if (tid == 0) {
      smem[NW] = (int)lowest_key(sl.tau);
      s_cnt = 0;
    }
    __syncthreads();
    const uint32_t klo = (uint32_t)smem[NW];
    if (klo >= t0) {  // uniform: every entry at or above l_lo is listed
      for (int i = tid; i < nl; i += NT) {
        const uint64_t le = list[i];
        const uint32_t k = (uint32_t)(le >> 32);
        if (k >= klo) {
          const int slot = atomicAdd(&s_cnt, 1);
          mem[slot] = ((uint64_t)f2key(prob_of(key2f(k))) << 32) | (0xffffffffu - (uint32_t)le);
        }
      }
      __syncthreads();
      emit(s_cnt);
      return;
    }
    __syncthreads();
  }
  // (3) the fallback.  With s a number: the entries whose logit reaches
  // l_lo, found by a select over the whole row, gathered and sorted when they
  // fit.
  if (s == s) {  // uniform
    const SelectResult sl = block_select<NT>(
        [&](auto fn) { row_scan([&](int, float l, bool in) { fn(in ? f2key(l) : 0u, in); }); }, m, -1,
        hist, smem);
    if (tid == 0) {
      smem[NW] = (int)lowest_key(sl.tau);
      s_cnt = 0;
    }
    __syncthreads();
    const uint32_t klo = (uint32_t)smem[NW];
    row_scan([&](int i, float l, bool in) {
      if (in && f2key(l) >= klo) {
        const int slot = atomicAdd(&s_cnt, 1);
        if (slot < kCand) mem[slot] = ((uint64_t)f2key(prob_of(l)) << 32) | (0xffffffffu - (uint32_t)i);
      }
    });
    __syncthreads();
    const int nc = s_cnt;
    if (nc <= kCand) {  // uniform
      emit(nc);
      return;
    }
    __syncthreads();
  }
  // (3') the m-th largest probability key T
  const SelectResult sr = block_select<NT>(
      [&](auto fn) { row_scan([&](int, float l, bool in) { fn(in ? pkey(l) : 0u, in); }); }, m, -1,
      hist, smem);
  const uint32_t T = sr.tau;
  // (4) ties at T: the stable sort keeps the lowest indices; the (m - gt)-th
  // lowest index among them is the last one kept
  uint32_t imax = 0xffffffffu;
  if (sr.ge > m) {
    __syncthreads();
    const SelectResult st = block_select<NT>(
        [&](auto fn) {
          row_scan([&](int i, float l, bool in) {
            const bool tie = in && pkey(l) == T;
            fn(tie ? 0xffffffffu - (uint32_t)i : 0u, tie);
          });
        },
        m - sr.gt, -1, hist, smem);
    imax = 0xffffffffu - st.tau;
  }
  // (5) the members, sorted by (key desc, index asc): key << 32 | ~index
  if (tid == 0) s_cnt = 0;
  __syncthreads();
  row_scan([&](int i, float l, bool in) {
    const uint32_t k = pkey(l);
    if (in && (k > T || (k == T && (uint32_t)i <= imax))) {
      const int slot = atomicAdd(&s_cnt, 1);
      if (slot < kTopMaxN) mem[slot] = ((uint64_t)k << 32) | (0xffffffffu - (uint32_t)i);
    }
  });
  __syncthreads();
  emit(min(s_cnt, kTopMaxN));  // == m
}

// ---------------------------------------------------------------------------
// small helpers
// ---------------------------------------------------------------------------
// ---------------------------------------------------------------------------
// 4. row_nll_kernel -- perplexity's per-position term (model.nim:578-583)
// ---------------------------------------------------------------------------
// One workgroup per row, two passes over it (16-byte loads, 64 KB in flight
// per workgroup): the float32 maximum (Nim's max(mx, v) keeps mx for a
// NaN v, as fmaxf does), then s = sum of exp(float64(l - mx)) in float64 --
// each thread over its own elements in index order, then a fixed tree over
// the threads -- and -(float64(l[t] - mx) - ln(s)).  The reference adds in
// index order; the tree differs from it only by float64 rounding.  The exp is
// the table-driven one of nls_exp64.h (within a few ulps of the library's).
template <int NT>
__global__ __launch_bounds__(NT) void row_nll_kernel(const float* __restrict__ logits, int64_t V,
                                                     const int32_t* __restrict__ targets,
                                                     double* __restrict__ out) {
  constexpr int NW = NT / kWave;
  constexpr int U = 8;  // loads in flight per thread
  __shared__ float s_mx[NW];
  __shared__ double s_ps[NW];
  __shared__ double s_t[kExp64Table];
  const int row = (int)blockIdx.x;
  const int tid = (int)threadIdx.x;
  const int lane = lane_id();
  const int wv = tid >> 6;
  const float* __restrict__ x = logits + (int64_t)row * V;
  const __amdgpu_buffer_rsrc_t xr = slice_rsrc(x, (int)V);  // V < 2^29 (checked by the host)
  // fn(l, in) over the row: with 16-byte loads (V % 4 == 0, aligned rows),
  // four per thread in flight (64 KB per workgroup); otherwise 4-byte loads,
  // eight per thread.  Past the row the loads read 0 with in == false.
  const bool vec = (V % 4 == 0) && ((reinterpret_cast<uintptr_t>(x) & 15) == 0);
  auto scan = [&](auto fn) __attribute__((always_inline)) {
    if (vec) {
      const int V4 = (int)(V >> 2);
      for (int b = tid; b < V4; b += NT * 4) {
        f32x4 q[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int i4 = b + u * NT;
          q[u] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                               xr, i4 < V4 ? i4 * 16 : 0x7ffffff0, 0, 0));
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const bool in = b + u * NT < V4;
          fn(q[u].x, in);
          fn(q[u].y, in);
          fn(q[u].z, in);
          fn(q[u].w, in);
        }
      }
      return;
    }
    for (int i0 = 0; i0 < (int)V; i0 += NT * U) {
      float l[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = i0 + u * NT + tid;
        l[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                             xr, i < (int)V ? i * 4 : 0x7ffffff0, 0, 0));
      }
#pragma unroll
      for (int u = 0; u < U; ++u) fn(l[u], i0 + u * NT + tid < (int)V);
    }
  };
  if (tid < kExp64Table) s_t[tid] = exp64_table_entry(tid);
  float mx = -__builtin_inff();
  scan([&](float l, bool in) { mx = in ? __builtin_fmaxf(mx, l) : mx; });
  for (int o = kWave / 2; o > 0; o >>= 1) mx = __builtin_fmaxf(mx, __shfl_xor(mx, o));
  if (lane == 0) s_mx[wv] = mx;
  __syncthreads();
  mx = s_mx[0];
  for (int w = 1; w < NW; ++w) mx = __builtin_fmaxf(mx, s_mx[w]);
  double ps = 0.0;
  scan([&](float l, bool in) {
    if (in) ps += exp64((double)(l - mx), s_t);  // table-driven (nls_exp64.h)
  });
  for (int o = kWave / 2; o > 0; o >>= 1) ps += __shfl_xor(ps, o);
  if (lane == 0) s_ps[wv] = ps;
  __syncthreads();
  if (tid == 0) {
    double s = s_ps[0];
    for (int w = 1; w < NW; ++w) s += s_ps[w];
    const int t = targets[row];
    out[row] = (t >= 0 && (int64_t)t < V) ? -((double)(x[t] - mx) - log(s)) : __builtin_nan("");
  }
}

// argmax (src/nimllm/sampler.nim:45-49) of each row (one workgroup per row):
// `best` moves to i only when l[i] > l[best], so the answer is the first
// index of the greatest value, a NaN is never taken, a NaN at index 0 keeps
// the answer 0, and an empty row answers 0.  Each thread keeps the first of
// its largest values (its elements arrive in index order); the threads'
// (value, index) pairs then reduce by larger value, then smaller index.
template <int NT>
__global__ __launch_bounds__(NT) void argmax_rows_kernel(const float* __restrict__ logits, int64_t V,
                                                         int32_t* __restrict__ out) {
  constexpr int NW = NT / kWave;
  constexpr int kNone = 0x7fffffff;
  __shared__ float s_v[NW];
  __shared__ int s_i[NW];
  const int row = (int)blockIdx.x;
  const int tid = (int)threadIdx.x;
  const int lane = lane_id();
  const int wv = tid >> 6;
  if (V == 0) {
    if (tid == 0) out[row] = 0;
    return;
  }
  const float* __restrict__ x = logits + (int64_t)row * V;
  const __amdgpu_buffer_rsrc_t xr = slice_rsrc(x, (int)V);  // V < 2^29 (checked by the host)
  float bv = -__builtin_inff();
  int bi = kNone;
  auto take = [&](float l, int i, bool in) __attribute__((always_inline)) {
    if (in && (l > bv || (l == bv && i < bi))) {
      bv = l;
      bi = i;
    }
  };
  const bool vec = (V % 4 == 0) && ((reinterpret_cast<uintptr_t>(x) & 15) == 0);
  if (vec) {
    const int V4 = (int)(V >> 2);
    for (int b = tid; b < V4; b += NT * 4) {
      f32x4 q[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i4 = b + u * NT;
        q[u] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                             xr, i4 < V4 ? i4 * 16 : 0x7ffffff0, 0, 0));
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i4 = b + u * NT;
        const bool in = i4 < V4;
        take(q[u].x, 4 * i4, in);
        take(q[u].y, 4 * i4 + 1, in);
        take(q[u].z, 4 * i4 + 2, in);
        take(q[u].w, 4 * i4 + 3, in);
      }
    }
  } else {
    constexpr int U = 8;
    for (int i0 = 0; i0 < (int)V; i0 += NT * U) {
      float l[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = i0 + u * NT + tid;
        l[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                             xr, i < (int)V ? i * 4 : 0x7ffffff0, 0, 0));
      }
#pragma unroll
      for (int u = 0; u < U; ++u) take(l[u], i0 + u * NT + tid, i0 + u * NT + tid < (int)V);
    }
  }
  for (int o = kWave / 2; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const int oi = __shfl_xor(bi, o);
    if (ov > bv || (ov == bv && oi < bi)) {
      bv = ov;
      bi = oi;
    }
  }
  if (lane == 0) {
    s_v[wv] = bv;
    s_i[wv] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < NW; ++w)
      if (s_v[w] > bv || (s_v[w] == bv && s_i[w] < bi)) {
        bv = s_v[w];
        bi = s_i[w];
      }
    const float x0 = x[0];
    out[row] = (x0 != x0 || bi == kNone) ? 0 : bi;
  }
}

// ids: [rows x count] staged ids (skipped entries already removed), row b
// appending its first cnt[b] of them.
__global__ void accept_host_kernel(const int32_t* __restrict__ ids, const int32_t* __restrict__ cnt,
                                   int count, int32_t* __restrict__ hist,
                                   int64_t* __restrict__ hist_len, int hcap, int row_only) {
  const int b = row_only >= 0 ? row_only : (int)blockIdx.x;
  const int r = row_only >= 0 ? 0 : b;  // the staged row
  const int64_t len = hist_len[b];
  const int32_t* src = ids + (int64_t)r * count;
  const int n = cnt[r];
  // Only the last hcap ids survive in the ring; writing just those keeps
  // every slot single-writer when n > hcap.
  const int first = n > hcap ? n - hcap : 0;
  for (int j = first + (int)threadIdx.x; j < n; j += blockDim.x)
    hist[(int64_t)b * hcap + (int)((len + j) % hcap)] = src[j];
  __syncthreads();
  if (threadIdx.x == 0) hist_len[b] = len + n;
}

__global__ void accept_device_kernel(const int32_t* __restrict__ ids, int B, int64_t V,
                                     int32_t* __restrict__ hist, int64_t* __restrict__ hist_len,
                                     int hcap) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  int32_t id = ids[b];
  if (id == INT32_MIN) return;  // the row accepts nothing this step
  const int64_t len = hist_len[b];
  if (id < 0 || id >= V) id = -1;
  hist[(int64_t)b * hcap + (int)(len % hcap)] = id;
  hist_len[b] = len + 1;
}

// One step of batched generation after nls_sample (chat.nim:204-208 per
// row): a row not yet done whose id is an end-of-generation id finishes (the
// id is not accepted); the others accept their id into the history ring
// (out-of-range ids take a -1 slot, as accept_device_kernel stores them).
__global__ void generate_step_kernel(const int32_t* __restrict__ out, int B, int64_t V,
                                     const int32_t* __restrict__ eog, int n_eog, int32_t* __restrict__ row_done,
                                     int32_t* __restrict__ hist, int64_t* __restrict__ hist_len, int hcap) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B || row_done[b] != 0) return;
  int32_t id = out[b];
  for (int j = 0; j < n_eog; ++j)
    if (eog[j] == id) {
      row_done[b] = 1;
      return;
    }
  const int64_t len = hist_len[b];
  if (id < 0 || id >= V) id = -1;
  hist[(int64_t)b * hcap + (int)(len % hcap)] = id;
  hist_len[b] = len + 1;
}

// Both device evaluations of the exponential: y[i] = exp(x[i]) when they
// agree, else a NaN with the payload 0xdead (so a checksum over every input
// covers both).
__global__ void expf_kernel(const float* __restrict__ x, float* __restrict__ y, int64_t n) {
  __shared__ double pow2[kExpfPow2Count];
  if (threadIdx.x < kExpfPow2Count) pow2[threadIdx.x] = kExpfPow2J64[threadIdx.x];
  __syncthreads();
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    const float a = expf_cr(x[i]);
    const float b = expf_cr_t(x[i], pow2);
    y[i] = __float_as_uint(a) == __float_as_uint(b) ? a : __uint_as_float(0x7fc0deadu);
  }
}

// ---------------------------------------------------------------------------
// launchers (called from nls_api.cpp)
// ---------------------------------------------------------------------------
static hipError_t launch_stream(const StreamArgs& a, const LaunchPlan& p, hipStream_t s) {
  if (p.nt == 512) return p.vec4 ? launch_stream_variant<512, true>(a, p, s) : launch_stream_variant<512, false>(a, p, s);
  if (p.nt == 1024)
    return p.vec4 ? launch_stream_variant<1024, true>(a, p, s) : launch_stream_variant<1024, false>(a, p, s);
  return p.vec4 ? launch_stream_variant<256, true>(a, p, s) : launch_stream_variant<256, false>(a, p, s);
}

hipError_t launch_sample(const StreamArgs& sa, const GenericArgs& ga, const FloorArgs& fa, const LaunchPlan& lp,
                         hipStream_t s, hipEvent_t ev_start, hipEvent_t ev_stop, hipEvent_t gev_start,
                         hipEvent_t gev_stop) {
  hipError_t e;
  if (lp.floor_slices > 0) {
    if (ev_start && (e = hipEventRecord(ev_start, s)) != hipSuccess) return e;
    if ((e = launch_floor(fa, lp, lp.vec4, s)) != hipSuccess) return e;
    if (ev_stop && (e = hipEventRecord(ev_stop, s)) != hipSuccess) return e;
  } else if (!lp.no_stream) {
    if (ev_start && (e = hipEventRecord(ev_start, s)) != hipSuccess) return e;
    if ((e = lp.k64 ? launch_k64(sa, lp, s) : launch_stream(sa, lp, s)) != hipSuccess) return e;
    if (ev_stop && (e = hipEventRecord(ev_stop, s)) != hipSuccess) return e;
  }
  if (!sa.gen_inline) {
    if (gev_start && (e = hipEventRecord(gev_start, s)) != hipSuccess) return e;
    if ((e = launch_generic(ga, lp, s)) != hipSuccess) return e;
    if (gev_stop && (e = hipEventRecord(gev_stop, s)) != hipSuccess) return e;
  }
  return hipGetLastError();
}

hipError_t launch_accept_host(const int32_t* d_ids, const int32_t* d_cnt, int B, int count,
                              int32_t* hist, int64_t* hist_len, int hcap, int row_only, hipStream_t s) {
  hipLaunchKernelGGL(accept_host_kernel, dim3(row_only >= 0 ? 1 : B), dim3(256), 0, s, d_ids, d_cnt,
                     count, hist, hist_len, hcap, row_only);
  return hipGetLastError();
}

// Zeroes a handle's per-call counters: the S > 1 arrival counts, the
// finished-workgroup count and the eight counters of the whole-row launches.
__global__ void clear_counters_kernel(uint32_t* arrive, int B, uint32_t* done, int32_t* gcount) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < B) arrive[i] = 0u;
  if (i == 0) *done = 0u;
  if (i < 8) gcount[i] = 0;
}

hipError_t launch_clear_counters(uint32_t* arrive, int B, uint32_t* done, int32_t* gcount, hipStream_t s) {
  const int n = B > 8 ? B : 8;
  hipLaunchKernelGGL(clear_counters_kernel, dim3((n + 255) / 256), dim3(256), 0, s, arrive, B, done, gcount);
  return hipGetLastError();
}

hipError_t launch_generate_step(const int32_t* d_out, int B, int64_t V, const int32_t* eog, int n_eog,
                                int32_t* row_done, int32_t* hist, int64_t* hist_len, int hcap, hipStream_t s) {
  hipLaunchKernelGGL(generate_step_kernel, dim3((B + 255) / 256), dim3(256), 0, s, d_out, B, V, eog, n_eog,
                     row_done, hist, hist_len, hcap);
  return hipGetLastError();
}

hipError_t launch_accept_device(const int32_t* d_ids, int B, int64_t V, int32_t* hist,
                                int64_t* hist_len, int hcap, hipStream_t s) {
  hipLaunchKernelGGL(accept_device_kernel, dim3((B + 255) / 256), dim3(256), 0, s, d_ids, B, V,
                     hist, hist_len, hcap);
  return hipGetLastError();
}

size_t max_dynamic_lds() { return 143 * 1024; }  // 160 KB of LDS less the largest static part

hipError_t set_kernel_attributes() {
  hipError_t e;
  if ((e = set_generic_attributes()) != hipSuccess) return e;
  if ((e = set_floor_attributes()) != hipSuccess) return e;
  if ((e = set_k64_attributes()) != hipSuccess) return e;
  if ((e = set_stream_attributes<512, true>()) != hipSuccess) return e;
  if ((e = set_stream_attributes<512, false>()) != hipSuccess) return e;
  if ((e = set_stream_attributes<256, true>()) != hipSuccess) return e;
  if ((e = set_stream_attributes<256, false>()) != hipSuccess) return e;
  if ((e = set_stream_attributes<1024, true>()) != hipSuccess) return e;
  return set_stream_attributes<1024, false>();
}

hipError_t launch_top_tokens(const float* logits, int rows, int64_t V, int n, int32_t* ids,
                             float* probs, hipStream_t s) {
  hipLaunchKernelGGL(top_tokens_kernel<kTopThreads>, dim3(rows), dim3(kTopThreads), 0, s, logits, V, n,
                     ids, probs);
  return hipGetLastError();
}

hipError_t launch_row_nll(const float* logits, int rows, int64_t V, const int32_t* targets, double* out,
                          hipStream_t s) {
  hipLaunchKernelGGL(row_nll_kernel<1024>, dim3(rows), dim3(1024), 0, s, logits, V, targets, out);
  return hipGetLastError();
}

hipError_t launch_argmax(const float* logits, int rows, int64_t V, int32_t* out, hipStream_t s) {
  if (V < 32768)
    hipLaunchKernelGGL(argmax_rows_kernel<256>, dim3(rows), dim3(256), 0, s, logits, V, out);
  else
    hipLaunchKernelGGL(argmax_rows_kernel<1024>, dim3(rows), dim3(1024), 0, s, logits, V, out);
  return hipGetLastError();
}

hipError_t launch_expf(const float* x, float* y, int64_t n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(expf_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, y, n);
  return hipGetLastError();
}

}  // namespace nls
