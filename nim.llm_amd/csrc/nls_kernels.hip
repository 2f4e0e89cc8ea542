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

namespace nls {

// ---------------------------------------------------------------------------
// 3. top_tokens_kernel -- topTokens (sampler.nim:123-130)
// ---------------------------------------------------------------------------
// One workgroup per row: softmaxInPlace (:51-57) over the whole row -- the
// maximum, exp(l - mx), the fp32 sum in index order, the division -- and the
// first n entries of the stable sort by probability (:127-128).  The
// probabilities are recomputed from the logits wherever they are needed, so
// the row is read a few times and only the n results are written.
//   * The sum runs in index order, one add at a time, in lane 0 of wave 0,
//     while the other waves compute the next chunk's exponentials into LDS.
//   * The n-th largest logit L comes from an exact radix select on the logits'
//     keys; the entries whose probability reaches p(L) are those with a logit
//     at or above the lowest float whose probability equals p(L) (a bisection
//     on the float's bits).  They are few: gathered with their probabilities,
//     sorted by (probability desc, index asc) in LDS, the first n kept.
//     (Equal probabilities can come from different logits: the exp and the
//     division round, so the order cannot be taken from the logits.)
//   * Rows where that set is large (or s is NaN) select on the probabilities
//     themselves: an exact radix select of the n-th largest probability T, and
//     among the entries equal to T the lowest indices (a second select on the
//     index), as the stable sort keeps them.
// A row holding NaN, or +inf with anything else, has NaN probabilities; the
// reference's comparator is no order on NaN, so such rows are outside the
// parity claim (this kernel then returns the first indices).
template <int NT>
__global__ __launch_bounds__(NT) void top_tokens_kernel(const float* __restrict__ logits, int64_t V,
                                                        int n, int32_t* __restrict__ ids,
                                                        float* __restrict__ probs) {
  constexpr int NW = NT / kWave;
  static_assert((size_t)kTopChunk * 2 * sizeof(float) >= (size_t)kTopMaxN * sizeof(uint64_t),
                "the members reuse the chunk buffers");
  __shared__ __align__(16) float ebuf[2][kTopChunk];
  __shared__ uint32_t hist[kSelWords];
  __shared__ int smem[NW + 4];
  __shared__ float s_part[NW];
  __shared__ float s_sum;
  __shared__ int s_cnt;
  const int row = (int)blockIdx.x;
  const int tid = (int)threadIdx.x;
  const int lane = lane_id();
  const int wv = tid >> 6;
  const float* __restrict__ x = logits + (int64_t)row * V;
  const __amdgpu_buffer_rsrc_t xr = slice_rsrc(x, (int)V);  // V < 2^29 (checked by the host)
  const int m = (int)min((int64_t)n, V);  // 1 <= m <= kTopMaxN (checked by the host)
  for (int q = tid; q < kSelWords; q += NT) hist[q] = 0u;
  // fn(i, l, in) over the row, eight requests per thread in flight at a time
  // (past the row they read 0 with in == false); every lane makes the same
  // number of calls
  constexpr int kScanU = 8;
  auto row_scan = [&](auto fn) __attribute__((always_inline)) {
    for (int i0 = 0; i0 < (int)V; i0 += NT * kScanU) {
      float l[kScanU];
#pragma unroll
      for (int u = 0; u < kScanU; ++u) {
        const int i = i0 + u * NT + tid;
        l[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                             xr, i < (int)V ? i * 4 : 0x7ffffff0, 0, 0));
      }
#pragma unroll
      for (int u = 0; u < kScanU; ++u) {
        const int i = i0 + u * NT + tid;
        fn(i, l[u], i < (int)V);
      }
    }
  };

  // (1) mx (:53): nim's max(mx, v) takes v when mx <= v, so NaN is never
  // taken; the float maximum of the rest (its sign of zero changes no l - mx)
  float mx = -__builtin_inff();
  row_scan([&](int, float l, bool in) { mx = in ? __builtin_fmaxf(mx, l) : mx; });
  for (int o = kWave / 2; o > 0; o >>= 1) mx = __builtin_fmaxf(mx, __shfl_xor(mx, o));
  if (lane == 0) s_part[wv] = mx;
  __syncthreads();
  mx = s_part[0];
  for (int w = 1; w < NW; ++w) mx = __builtin_fmaxf(mx, s_part[w]);

  // (2) s = e_0 + e_1 + ... in index order (:54-56): chunk c is computed by
  // waves 1.. into ebuf[c & 1] while lane 0 of wave 0 adds chunk c - 1
  const int64_t nch = (V + kTopChunk - 1) / kTopChunk;
  float s = 0.0f;
  for (int64_t c = 0; c <= nch; ++c) {
    if (wv != 0 && c < nch) {
      // every producer thread's loads go out together (past the row they read 0)
      constexpr int PP = (kTopChunk + NT - kWave - 1) / (NT - kWave);
      const int c0 = (int)(c * kTopChunk);
      float* eb = ebuf[c & 1];
      float lv[PP];
#pragma unroll
      for (int q = 0; q < PP; ++q) {
        const int j = tid - kWave + q * (NT - kWave);
        lv[q] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                              xr, j < kTopChunk ? (c0 + j) * 4 : 0x7ffffff0, 0, 0));
      }
#pragma unroll
      for (int q = 0; q < PP; ++q) {
        const int j = tid - kWave + q * (NT - kWave);
        if (j < kTopChunk) eb[j] = c0 + j < V ? expf_cr(lv[q] - mx) : 0.0f;
      }
    }
    if (wv == 0 && c > 0 && lane == 0) {
      // the whole chunk: entries past the row are +0, which leave s unchanged
      const f32x4* e4 = reinterpret_cast<const f32x4*>(ebuf[(c - 1) & 1]);
      // blocks of 16; the reads of the block two ahead are issued before the
      // adds of the current one (the barrier keeps the compiler from sinking
      // them), so the adds never wait for the LDS
      constexpr int nb = kTopChunk / 16;
      constexpr int kLast = nb - 1;
      f32x4 a[4], b[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        a[q] = e4[q];
        b[q] = e4[4 + q];
      }
#pragma unroll 8
      for (int blk = 0; blk < nb; ++blk) {
        const int nx = min(blk + 2, kLast) * 4;
        f32x4 t[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) t[q] = e4[nx + q];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          s = s + a[q].x;
          s = s + a[q].y;
          s = s + a[q].z;
          s = s + a[q].w;
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          a[q] = b[q];
          b[q] = t[q];
        }
      }
    }
    __syncthreads();
  }
  if (tid == 0) s_sum = s;
  __syncthreads();
  s = s_sum;
  // probs[i] /= s (:57)
  auto pkey = [&](float l) -> uint32_t { return f2key(expf_cr(l - mx) / s); };

  uint64_t* mem = reinterpret_cast<uint64_t*>(&ebuf[0][0]);
  constexpr int kCand = (int)(sizeof(ebuf) / sizeof(uint64_t));
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
  // (3) The probability is non-decreasing in the logit (l - mx, the exp and
  // the division by s each are), so the m-th largest probability is p(L) of
  // the m-th largest logit L, and the entries whose probability reaches it are
  // exactly those whose logit is at least l_lo, the lowest float with
  // p(l_lo) == p(L).  With s a number (no NaN or +inf in the row) those few
  // are gathered with their probabilities and sorted.  Rows where they are
  // many fall through to the selection on the probabilities below.
  auto prob_of = [&](float l) -> float { return expf_cr(l - mx) / s; };
  if (s == s) {  // uniform
    const SelectResult sl = block_select<NT>(
        [&](auto fn) { row_scan([&](int, float l, bool in) { fn(in ? f2key(l) : 0u, in); }); }, m, -1,
        hist, smem);
    if (tid == 0) {
      // the lowest key in [key(-inf), key(L)] whose probability reaches p(L)
      const float pm = prob_of(key2f(sl.tau));
      uint32_t lo = f2key(-__builtin_inff()), hi = sl.tau;
      while (lo < hi) {
        const uint32_t mid = lo + (hi - lo) / 2;
        if (prob_of(key2f(mid)) >= pm)
          hi = mid;
        else
          lo = mid + 1;
      }
      smem[NW] = (int)hi;
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

__global__ void expf_kernel(const float* __restrict__ x, float* __restrict__ y, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = expf_cr(x[i]);
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

hipError_t launch_sample(const StreamArgs& sa, const GenericArgs& ga, const LaunchPlan& lp,
                         hipStream_t s, hipEvent_t ev_start, hipEvent_t ev_stop, hipEvent_t gev_start,
                         hipEvent_t gev_stop) {
  hipError_t e;
  if (ev_start && (e = hipEventRecord(ev_start, s)) != hipSuccess) return e;
  if ((e = lp.k64 ? launch_k64(sa, lp, s) : launch_stream(sa, lp, s)) != hipSuccess) return e;
  if (ev_stop && (e = hipEventRecord(ev_stop, s)) != hipSuccess) return e;
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

hipError_t launch_expf(const float* x, float* y, int64_t n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(expf_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, y, n);
  return hipGetLastError();
}

}  // namespace nls
