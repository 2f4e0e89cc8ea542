// nls_kernels.hip -- gfx950 kernels of the batched token sampler.
//
// Pipeline for one nls_sample call over B rows of V fp32 logits:
//   1. prep_kernel     (B workgroups)  history window + logit bias -> sorted patch
//                       list per row (penalties S2 and bias S3, sampler.nim:64-76)
//   2. chunk_kernel    (B x ceil(V/16384) workgroups)  the single HBM pass: each
//                       workgroup streams a 64 KB chunk into registers, applies
//                       the patches and temperature (:80-81), reduces max/argmax,
//                       and for top-k rows keeps every value that can still be
//                       among the row's k best (superset, exact).
//   3. merge_kernel    (B workgroups)  greedy rows: argmax (:77-78); top-k rows:
//                       the exact heap membership/order (:85-95), softmax (:98-100),
//                       top-p (:103-108), min-p (:110-114) and the draw (:115-121).
//   4. generic_kernel  whole-row kernel for full-sort rows (:96-97) and for any
//                       top-k row whose candidate set overflowed the fast path.
//
// All fp32/fp64 arithmetic follows the reference's order; this file is built
// with -ffp-contract=off so no multiply-add is fused.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "nls_expf.h"
#include "nls_internal.h"
#include "nls_primitives.h"

namespace nls {

// Apply one patch to the original logit: penalties first (:71-74), then bias (:76).
__device__ __forceinline__ float apply_patch(float v, const Patch& p, const RowParams& P) {
  if (p.flags & kPatchPen) {
    if (P.rp_active) v = (v > 0.0f) ? (v / P.rp32) : (v * P.rp32);
    v = v - p.pen;
  }
  if (p.flags & kPatchBias) v = v + p.bias;
  return v;
}

// ---------------------------------------------------------------------------
// 1. prep: sorted patch list per row
// ---------------------------------------------------------------------------
// Entries: history id -> (id << 32); bias j -> (id << 32) | 0x80000000 | j;
// out-of-range history ids -> all-ones (dropped, sampler.nim:70).  After an
// ascending sort, a run of equal ids holds that id's history occurrences
// followed by its bias entry.
template <int NT>
__device__ void prep_row(uint64_t* a, int npow, int n_hist, int n, const RowParams& P, int row,
                         int64_t V, const int32_t* __restrict__ hist, int64_t len, int hcap,
                         const int32_t* __restrict__ bias_ids, const float* __restrict__ bias_vals,
                         Patch* __restrict__ out, int32_t* __restrict__ out_cnt, int* smem) {
  for (int i = threadIdx.x; i < npow; i += NT) {
    uint64_t e = ~0ull;
    if (i < n_hist) {
      const int64_t j = len - n_hist + i;
      const int id = hist[(int64_t)row * hcap + (int)(j % hcap)];
      if (id >= 0 && id < V) e = (uint64_t)(uint32_t)id << 32;
    } else if (i < n) {
      const int b = i - n_hist;
      e = ((uint64_t)(uint32_t)bias_ids[P.bias_off + b] << 32) | 0x80000000ull | (uint64_t)b;
    }
    a[i] = e;
  }
  __syncthreads();
  bitonic_sort_u64<NT>(a, npow, false);
  // valid entries form a prefix; count them
  int nv_local = 0;
  for (int i = threadIdx.x; i < npow; i += NT) nv_local += (a[i] != ~0ull);
  const int nv = block_sum<NT>(nv_local, smem);
  // runs: thread t owns the contiguous slice [lo, hi)
  const int per = (nv + NT - 1) / NT;
  const int lo = min(nv, (int)threadIdx.x * per), hi = min(nv, lo + per);
  int starts = 0;
  for (int i = lo; i < hi; ++i)
    starts += (i == 0 || (a[i] >> 32) != (a[i - 1] >> 32));
  int total;
  int pos = block_excl_scan<NT>(starts, smem, total);
  for (int i = lo; i < hi; ++i) {
    const uint64_t id = a[i] >> 32;
    if (!(i == 0 || id != (a[i - 1] >> 32))) continue;
    // run end: first entry with a larger id (binary search)
    int l = i + 1, r = nv;
    while (l < r) {
      const int m = (l + r) >> 1;
      if ((a[m] >> 32) == id)
        l = m + 1;
      else
        r = m;
    }
    const int end = l - 1;
    const bool has_bias = (a[end] & 0x80000000ull) != 0;
    const int cnt = (end - i + 1) - (has_bias ? 1 : 0);
    Patch p;
    p.id = (int32_t)id;
    p.flags = (cnt > 0 ? kPatchPen : 0) | (has_bias ? kPatchBias : 0);
    p.pen = 0.0f;
    if (cnt > 0) {
      const double pen = (double)cnt * P.freq + P.pres;  // float64, one rounding (:74)
      p.pen = (float)pen;
    }
    p.bias = has_bias ? bias_vals[P.bias_off + (int)(a[end] & 0x7fffffffull)] : 0.0f;
    out[pos++] = p;
  }
  if (threadIdx.x == 0) out_cnt[row] = total;
}

__global__ __launch_bounds__(256) void prep_kernel(
    const RowParams* __restrict__ rp, int64_t V, const int32_t* __restrict__ hist,
    const int64_t* __restrict__ hist_len, int hcap, const int32_t* __restrict__ bias_ids,
    const float* __restrict__ bias_vals, Patch* __restrict__ patches,
    int32_t* __restrict__ patch_cnt, int pcap, uint64_t* __restrict__ gscratch,
    int64_t gscratch_stride, int32_t* __restrict__ generic_count) {
  constexpr int NT = 256;
  __shared__ uint64_t sbuf[kPrepSortLds];
  __shared__ int smem[NT / kWave + 4];
  const int row = blockIdx.x;
  if (row == 0 && threadIdx.x == 0) *generic_count = 0;
  const RowParams P = rp[row];
  const int64_t len = hist_len[row];
  int n_hist = 0;
  if (len > 0 && P.pen_active)
    n_hist = (int)((P.repeat_last_n > 0) ? (P.repeat_last_n < len ? P.repeat_last_n : len) : len);
  const int n = n_hist + P.bias_cnt;
  if (n == 0) {
    if (threadIdx.x == 0) patch_cnt[row] = 0;
    return;
  }
  const int npow = next_pow2(n);
  Patch* out = patches + (int64_t)row * pcap;
  if (npow <= kPrepSortLds) {
    prep_row<NT>(sbuf, npow, n_hist, n, P, row, V, hist, len, hcap, bias_ids, bias_vals, out,
                 patch_cnt, smem);
  } else {
    prep_row<NT>(gscratch + (int64_t)row * gscratch_stride, npow, n_hist, n, P, row, V, hist,
                 len, hcap, bias_ids, bias_vals, out, patch_cnt, smem);
  }
}

// ---------------------------------------------------------------------------
// 2. chunk pass (the only full read of the logits)
// ---------------------------------------------------------------------------
// Lower bound for the chunk's k-th largest: the k-th largest of the threads'
// top-Q values (those are k real chunk elements), so every element that can be
// among the row's k best is >= it.
template <int Q>
__device__ __forceinline__ void topq_insert(uint32_t (&t)[Q], uint32_t key) {
  if (key > t[Q - 1]) {
    t[Q - 1] = key;
#pragma unroll
    for (int s = Q - 1; s > 0; --s) {
      if (t[s] > t[s - 1]) {
        const uint32_t x = t[s];
        t[s] = t[s - 1];
        t[s - 1] = x;
      }
    }
  }
}

constexpr int kPatchRound = 512;
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int NV4, int Q, bool VEC>
__global__ __launch_bounds__(kChunkThreads) void chunk_kernel(
    const float* __restrict__ logits, int64_t V, int nchunks, const RowParams* __restrict__ rp,
    const Patch* __restrict__ patches, const int32_t* __restrict__ patch_cnt, int pcap,
    ChunkStat* __restrict__ stats, uint64_t* __restrict__ cand, int ccap) {
  constexpr int NT = kChunkThreads;
  constexpr int NE = NV4 * 4;
  constexpr int CH = NT * NE;
  __shared__ uint32_t bitmap[CH / 32];
  __shared__ Patch plist[kPatchRound];
  __shared__ uint32_t hist[256];
  __shared__ int smem[NT / kWave + 4];
  __shared__ float red_v[NT / kWave];
  __shared__ int red_i[NT / kWave];
  __shared__ int prange[2];

  const int row = blockIdx.x / nchunks;
  const int c = blockIdx.x - row * nchunks;
  const RowParams P = rp[row];
  const int c0 = c * CH;
  const int clen = (int)((V - c0) < CH ? (V - c0) : CH);
  const float* __restrict__ src = logits + (int64_t)row * V + c0;
  const int tid = threadIdx.x;

  float v[NE];
#pragma unroll
  for (int j = 0; j < NV4; ++j) {
    const int o = (j * NT + tid) * 4;
    if (VEC && o + 4 <= clen) {
      const f32x4 t = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(src + o));
      v[4 * j + 0] = t.x;
      v[4 * j + 1] = t.y;
      v[4 * j + 2] = t.z;
      v[4 * j + 3] = t.w;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[4 * j + e] = (o + e < clen) ? src[o + e] : 0.0f;
    }
  }

  // ---- patches (penalties + bias) for ids in [c0, c0 + clen) ----
  const int pn = patch_cnt[row];
  if (pn > 0) {
    const Patch* __restrict__ pl = patches + (int64_t)row * pcap;
    if (tid < 2) {
      const int target = c0 + (tid ? clen : 0);
      int l = 0, r = pn;
      while (l < r) {
        const int m = (l + r) >> 1;
        if (pl[m].id < target)
          l = m + 1;
        else
          r = m;
      }
      prange[tid] = l;
    }
    __syncthreads();
    const int pa = prange[0], pb = prange[1];
    for (int base = pa; base < pb; base += kPatchRound) {
      const int cnt = min(kPatchRound, pb - base);
      for (int q = tid; q < CH / 32; q += NT) bitmap[q] = 0u;
      for (int q = tid; q < cnt; q += NT) plist[q] = pl[base + q];
      __syncthreads();
      for (int q = tid; q < cnt; q += NT) {
        const int off = plist[q].id - c0;
        atomicOr(&bitmap[off >> 5], 1u << (off & 31));
      }
      __syncthreads();
#pragma unroll
      for (int j = 0; j < NV4; ++j) {
        const int o = (j * NT + tid) * 4;
        const uint32_t bits4 = (bitmap[o >> 5] >> (o & 31)) & 15u;
        if (bits4) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if ((bits4 >> e) & 1u) {
              const int id = c0 + o + e;
              int l = 0, r = cnt - 1;
              while (l < r) {
                const int m = (l + r) >> 1;
                if (plist[m].id < id)
                  l = m + 1;
                else
                  r = m;
              }
              v[4 * j + e] = apply_patch(v[4 * j + e], plist[l], P);
            }
          }
        }
      }
      __syncthreads();
    }
  }

  // ---- temperature (:80-81) ----
  if (P.mode != kModeGreedy) {
    const float invT = P.invT;
#pragma unroll
    for (int q = 0; q < NE; ++q) v[q] = v[q] * invT;
  }

  // ---- max / first argmax ----
  {
    float bv = -__builtin_inff();
    int bi = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < NV4; ++j) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int o = (j * NT + tid) * 4 + e;
        if (o < clen) argmax_merge(bv, bi, v[4 * j + e], c0 + o);
      }
    }
    wave_argmax(bv, bi);
    if (lane_id() == 0) {
      red_v[tid >> 6] = bv;
      red_i[tid >> 6] = bi;
    }
    __syncthreads();
    if (tid == 0) {
      float fv = red_v[0];
      int fi = red_i[0];
      for (int w = 1; w < NT / kWave; ++w) argmax_merge(fv, fi, red_v[w], red_i[w]);
      ChunkStat& s = stats[blockIdx.x];
      s.vmax = fv;
      s.amax = fi;
      s.ncand = 0;
      s.flags = 0;
    }
  }
  if (P.mode != kModeTopK || !P.fast) return;

  // ---- top-k candidates: every value >= LB, LB <= the chunk's k-th largest ----
  const int k = P.k;
  uint32_t lb = 0u;
  if (clen > k && k <= NT * Q) {
    uint32_t tops[Q];
#pragma unroll
    for (int q = 0; q < Q; ++q) tops[q] = 0u;
#pragma unroll
    for (int j = 0; j < NV4; ++j) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int o = (j * NT + tid) * 4 + e;
        if (o < clen) topq_insert<Q>(tops, f2key(v[4 * j + e]));
      }
    }
    lb = block_radix_select<NT>(
        [&](auto fn) {
#pragma unroll
          for (int q = 0; q < Q; ++q) fn(tops[q]);
        },
        k, hist, smem);
  }
  int mine = 0;
#pragma unroll
  for (int j = 0; j < NV4; ++j) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int o = (j * NT + tid) * 4 + e;
      mine += (o < clen && f2key(v[4 * j + e]) >= lb);
    }
  }
  int total;
  int pos = block_excl_scan<NT>(mine, smem, total);
  if (total > ccap) {
    if (tid == 0) {
      stats[blockIdx.x].ncand = total;
      stats[blockIdx.x].flags = kChunkOverflow;
    }
    return;
  }
  uint64_t* __restrict__ dst = cand + (int64_t)blockIdx.x * ccap;
#pragma unroll
  for (int j = 0; j < NV4; ++j) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int o = (j * NT + tid) * 4 + e;
      if (o < clen) {
        const uint32_t key = f2key(v[4 * j + e]);
        if (key >= lb) dst[pos++] = ((uint64_t)key << 32) | (uint32_t)(c0 + o);
      }
    }
  }
  if (tid == 0) stats[blockIdx.x].ncand = total;
}

// ---------------------------------------------------------------------------
// Shared tail: softmax over candidates in reference order, top-p, min-p, draw.
// `val` holds the candidates' final fp32 values (non-increasing), `ids` their
// token ids; `e` is scratch of the same length.  Sequential sums run in wave 0
// in candidate order, exactly as sampler.nim:51-57,103-121 accumulate.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float lane_f(float x, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l));
}

struct TailOut {
  int id;
  int n;
  float total;
};

template <int NT, typename VPtr, typename IPtr, typename EPtr>
__device__ TailOut softmax_cutoff_draw(VPtr val, IPtr ids, EPtr e, int ncand, const RowParams& P,
                                       double u, int* smem) {
  const float mx = val[0];  // candidates are in non-increasing order
  for (int i = threadIdx.x; i < ncand; i += NT) e[i] = expf_cr(val[i] - mx);
  __syncthreads();
  __shared__ float s_sum;
  __shared__ int s_n;
  __shared__ float s_total;
  __shared__ int s_pos;
  const int lane = lane_id();
  if (threadIdx.x < kWave) {
    // s = sum of e in order
    float s = 0.0f;
    for (int base = 0; base < ncand; base += kWave) {
      const float x = (base + lane < ncand) ? e[base + lane] : 0.0f;
      const int lim = min(kWave, ncand - base);
      for (int l = 0; l < lim; ++l) s += lane_f(x, l);
    }
    if (lane == 0) s_sum = s;
  }
  __syncthreads();
  const float s = s_sum;
  for (int i = threadIdx.x; i < ncand; i += NT) e[i] = e[i] / s;
  __syncthreads();
  if (threadIdx.x < kWave) {
    int n = ncand;
    if (P.topp_active) {
      float cum = 0.0f;
      bool done = false;
      for (int base = 0; base < ncand && !done; base += kWave) {
        const float x = (base + lane < ncand) ? e[base + lane] : 0.0f;
        const int lim = min(kWave, ncand - base);
        for (int l = 0; l < lim; ++l) {
          cum += lane_f(x, l);
          if ((double)cum >= P.topP) {
            n = base + l + 1;
            done = true;
            break;
          }
        }
      }
    }
    if (P.minp_active) {
      const float thr = e[0] * P.minP32;
      int m = 1;
      while (m < n && e[m] >= thr) ++m;
      n = m;
    }
    float total = 0.0f;
    for (int base = 0; base < n; base += kWave) {
      const float x = (base + lane < n) ? e[base + lane] : 0.0f;
      const int lim = min(kWave, n - base);
      for (int l = 0; l < lim; ++l) total += lane_f(x, l);
    }
    float r = (float)u * total;
    int pos = n - 1;
    bool found = false;
    for (int base = 0; base < n && !found; base += kWave) {
      const float x = (base + lane < n) ? e[base + lane] : 0.0f;
      const int lim = min(kWave, n - base);
      for (int l = 0; l < lim; ++l) {
        r = r - lane_f(x, l);
        if (r <= 0.0f) {
          pos = base + l;
          found = true;
          break;
        }
      }
    }
    if (lane == 0) {
      s_n = n;
      s_total = total;
      s_pos = pos;
    }
  }
  __syncthreads();
  TailOut t;
  t.n = s_n;
  t.total = s_total;
  t.id = ids[s_pos];
  return t;
}



template <int NT, typename EPtr, typename IPtr>
__device__ void write_debug(const DebugPtrs& dbg, int row, int path, int n, int ncand,
                            float total, IPtr ids, EPtr probs) {
  if (threadIdx.x == 0) {
    if (dbg.n) dbg.n[row] = n;
    if (dbg.ncand) dbg.ncand[row] = ncand;
    if (dbg.total) dbg.total[row] = total;
    if (dbg.path) dbg.path[row] = path;
  }
  const int m = min(n, dbg.cap);
  if (dbg.cand_ids)
    for (int i = threadIdx.x; i < m; i += NT) dbg.cand_ids[(int64_t)row * dbg.cap + i] = ids[i];
  if (dbg.cand_probs)
    for (int i = threadIdx.x; i < m; i += NT)
      dbg.cand_probs[(int64_t)row * dbg.cap + i] = probs[i];
}

__device__ __forceinline__ double row_uniform(const double* __restrict__ d_u, uint64_t* rng,
                                              int row) {
  if (d_u) return d_u[row];
  uint64_t st[2] = {rng[2 * row], rng[2 * row + 1]};
  const double u = nim_rand_unit(st);
  rng[2 * row] = st[0];
  rng[2 * row + 1] = st[1];
  return u;
}

// ---------------------------------------------------------------------------
// 3. merge: greedy rows and top-k rows
// ---------------------------------------------------------------------------
// Dynamic LDS: entries[ncap] u64 | members[mcap] u64 | vals[mcap] f32 |
//              ids[mcap] i32 | e[mcap] f32
template <int NT>
__global__ __launch_bounds__(NT) void merge_kernel(
    const RowParams* __restrict__ rp, int nchunks, const ChunkStat* __restrict__ stats,
    const uint64_t* __restrict__ cand, int ccap, int mcap, const double* __restrict__ d_u,
    uint64_t* __restrict__ rng, int32_t* __restrict__ out, float* __restrict__ row_max,
    int32_t* __restrict__ generic_list, int32_t* __restrict__ generic_count, DebugPtrs dbg) {
  extern __shared__ __align__(16) unsigned char dyn[];
  __shared__ uint32_t hist[256];
  __shared__ int smem[NT / kWave + 4];
  __shared__ int offs[kMaxChunks + 1];
  __shared__ int s_flag;
  const int row = blockIdx.x;
  const RowParams P = rp[row];
  const ChunkStat* st = stats + (int64_t)row * nchunks;

  if (P.mode == kModeGreedy) {
    if (threadIdx.x == 0) {
      float bv = st[0].vmax;
      int bi = st[0].amax;
      for (int c = 1; c < nchunks; ++c) argmax_merge(bv, bi, st[c].vmax, st[c].amax);
      out[row] = bi;
      if (dbg.n) dbg.n[row] = 0;
      if (dbg.ncand) dbg.ncand[row] = 0;
      if (dbg.total) dbg.total[row] = 0.0f;
      if (dbg.path) dbg.path[row] = 1;
    }
    return;
  }
  if (P.mode == kModeFull || !P.fast) {
    if (threadIdx.x == 0) {
      float bv = st[0].vmax;
      int bi = st[0].amax;
      for (int c = 1; c < nchunks; ++c) argmax_merge(bv, bi, st[c].vmax, st[c].amax);
      row_max[row] = bv;
      generic_list[atomicAdd(generic_count, 1)] = row;
    }
    return;
  }
  // ---- top-k row ----
  if (threadIdx.x == 0) {
    int acc = 0, flag = 0;
    for (int c = 0; c < nchunks; ++c) {
      offs[c] = acc;
      acc += st[c].ncand;
      flag |= st[c].flags;
    }
    offs[nchunks] = acc;
    s_flag = flag;
  }
  __syncthreads();
  const int N = offs[nchunks];
  if (s_flag || N > nchunks * ccap) {
    if (threadIdx.x == 0) generic_list[atomicAdd(generic_count, 1)] = row;
    return;
  }
  const int ncap = nchunks * ccap;
  uint64_t* ent = reinterpret_cast<uint64_t*>(dyn);
  uint64_t* mem = ent + ncap;
  float* vals = reinterpret_cast<float*>(mem + mcap);
  int32_t* ids = reinterpret_cast<int32_t*>(vals + mcap);
  float* ebuf = reinterpret_cast<float*>(ids + mcap);

  for (int c = 0; c < nchunks; ++c) {
    const int cnt = offs[c + 1] - offs[c];
    const uint64_t* srcc = cand + ((int64_t)row * nchunks + c) * ccap;
    for (int i = threadIdx.x; i < cnt; i += NT) ent[offs[c] + i] = srcc[i];
  }
  __syncthreads();
  const int k = P.k;
  const uint32_t T = block_radix_select<NT>(
      [&](auto fn) {
        for (int i = threadIdx.x; i < N; i += NT) fn((uint32_t)(ent[i] >> 32));
      },
      k, hist, smem);
  int gt_l = 0, ge_l = 0;
  for (int i = threadIdx.x; i < N; i += NT) {
    const uint32_t key = (uint32_t)(ent[i] >> 32);
    gt_l += key > T;
    ge_l += key >= T;
  }
  const int gt = block_sum<NT>(gt_l, smem);
  const int ge = block_sum<NT>(ge_l, smem);
  const int m = k - gt;  // ties at T to keep
  const int kpow = next_pow2(k);
  if (ge == k) {
    // no excess ties: the members are exactly the entries >= T
    int mine = 0;
    for (int i = threadIdx.x; i < N; i += NT) mine += ((uint32_t)(ent[i] >> 32) >= T);
    int tot;
    int pos = block_excl_scan<NT>(mine, smem, tot);
    for (int i = threadIdx.x; i < N; i += NT)
      if ((uint32_t)(ent[i] >> 32) >= T) mem[pos++] = ent[i];
  } else {
    // excess ties: heap rule (members = G + the m largest indices among ties
    // at or before p*, p* = index of the k-th entry >= T in index order)
    if (next_pow2(ge) > mcap) {
      if (threadIdx.x == 0) generic_list[atomicAdd(generic_count, 1)] = row;
      return;
    }
    const int gpow = next_pow2(ge);
    int mine = 0;
    for (int i = threadIdx.x; i < N; i += NT) mine += ((uint32_t)(ent[i] >> 32) >= T);
    int tot;
    int pos = block_excl_scan<NT>(mine, smem, tot);
    for (int i = threadIdx.x; i < N; i += NT) {
      const uint64_t x = ent[i];
      if ((uint32_t)(x >> 32) >= T) mem[pos++] = (x << 32) | (x >> 32);  // idx-major
    }
    for (int i = ge + threadIdx.x; i < gpow; i += NT) mem[i] = ~0ull;
    __syncthreads();
    bitonic_sort_u64<NT>(mem, gpow, false);
    // ties among the first k (index order); keep the last m of them
    int tl = 0;
    const int per = (k + NT - 1) / NT;
    const int lo = min(k, (int)threadIdx.x * per), hi = min(k, lo + per);
    for (int i = lo; i < hi; ++i) tl += ((uint32_t)mem[i] == T);
    int ntie;
    int trank = block_excl_scan<NT>(tl, smem, ntie);
    // members, written key-major into ent[] (free now): every entry with
    // key > T (any index) plus the selected ties
    int keep_l = 0;
    for (int i = threadIdx.x; i < ge; i += NT) keep_l += ((uint32_t)mem[i] > T);
    int gtot;
    int gpos = block_excl_scan<NT>(keep_l, smem, gtot);
    for (int i = threadIdx.x; i < ge; i += NT) {
      const uint64_t x = mem[i];
      if ((uint32_t)x > T) ent[gpos++] = (x << 32) | (x >> 32);
    }
    for (int i = lo; i < hi; ++i) {
      const uint64_t x = mem[i];
      if ((uint32_t)x == T) {
        if (trank >= ntie - m) ent[gtot + (trank - (ntie - m))] = (x << 32) | (x >> 32);
        ++trank;
      }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < k; i += NT) mem[i] = ent[i];
    __syncthreads();
  }
  for (int i = k + threadIdx.x; i < kpow; i += NT) mem[i] = 0ull;
  __syncthreads();
  // reference order: descending (value, index)
  bitonic_sort_u64<NT>(mem, kpow, true);
  for (int i = threadIdx.x; i < k; i += NT) {
    vals[i] = key2f((uint32_t)(mem[i] >> 32));
    ids[i] = (int32_t)(uint32_t)mem[i];
  }
  __syncthreads();
  __shared__ double s_u;
  if (threadIdx.x == 0) s_u = row_uniform(d_u, rng, row);
  __syncthreads();
  const TailOut t = softmax_cutoff_draw<NT>(vals, ids, ebuf, k, P, s_u, smem);
  if (threadIdx.x == 0) out[row] = t.id;
  write_debug<NT>(dbg, row, 2, t.n, k, t.total, ids, ebuf);
}

// ---------------------------------------------------------------------------
// 4. generic: whole-row stable radix sort, then the reference's tail
// ---------------------------------------------------------------------------
// Scratch per workgroup: keysA, idxA, keysB, idxB (uint32 each, vpad) and
// f32 work (vpad).  Keys are ~f2key(value): an ascending stable sort gives
// descending value with ascending index on ties (sampler.nim:97).
constexpr int kGenIPT = 8;

template <int NT>
__device__ void radix_sort_pass(const uint32_t* __restrict__ kin, const uint32_t* __restrict__ iin,
                                uint32_t* __restrict__ kout, uint32_t* __restrict__ iout, int n,
                                int shift, uint32_t* wcnt /*[NT/64][256]*/,
                                uint32_t* dbase /*[256]*/, uint32_t* drun /*[256]*/) {
  constexpr int NW = NT / kWave;
  constexpr int TILE = NT * kGenIPT;
  const int lane = lane_id();
  const int w = threadIdx.x >> 6;
  // digit histogram -> exclusive bases
  for (int d = threadIdx.x; d < 256; d += NT) {
    dbase[d] = 0u;
    drun[d] = 0u;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < n; i += NT) atomicAdd(&dbase[(kin[i] >> shift) & 255u], 1u);
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t acc = 0;
    for (int d = 0; d < 256; ++d) {
      const uint32_t c = dbase[d];
      dbase[d] = acc;
      acc += c;
    }
  }
  __syncthreads();
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int tbase = 0; tbase < n; tbase += TILE) {
    for (int q = threadIdx.x; q < NW * 256; q += NT) wcnt[q] = 0u;
    __syncthreads();
    uint32_t key[kGenIPT], idv[kGenIPT], rank[kGenIPT];
#pragma unroll
    for (int it = 0; it < kGenIPT; ++it) {
      const int i = tbase + (w * kGenIPT + it) * kWave + lane;
      const bool valid = i < n;
      key[it] = valid ? kin[i] : 0u;
      idv[it] = valid ? iin[i] : 0u;
      const uint32_t d = (key[it] >> shift) & 255u;
      uint64_t match = __ballot(valid);
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        const uint64_t bal = __ballot((d >> b) & 1u);
        match &= ((d >> b) & 1u) ? bal : ~bal;
      }
      rank[it] = 0u;
      if (valid) {
        const uint32_t before = wcnt[w * 256 + d];
        rank[it] = before + (uint32_t)__popcll(match & lt_mask);
        // the lowest lane of the group publishes the new count
        if ((match & lt_mask) == 0ull) wcnt[w * 256 + d] = before + (uint32_t)__popcll(match);
      }
    }
    __syncthreads();
    // per-(wave, digit) offsets within the tile, plus the digit's running total
    for (int d = threadIdx.x; d < 256; d += NT) {
      uint32_t acc = drun[d];
      for (int q = 0; q < NW; ++q) {
        const uint32_t c = wcnt[q * 256 + d];
        wcnt[q * 256 + d] = acc;
        acc += c;
      }
      drun[d] = acc;
    }
    __syncthreads();
#pragma unroll
    for (int it = 0; it < kGenIPT; ++it) {
      const int i = tbase + (w * kGenIPT + it) * kWave + lane;
      if (i < n) {
        const uint32_t d = (key[it] >> shift) & 255u;
        const uint32_t p = dbase[d] + wcnt[w * 256 + d] + rank[it];
        kout[p] = key[it];
        iout[p] = idv[it];
      }
    }
    __syncthreads();
  }
}

// lower/upper bound on an ascending uint32 array
__device__ __forceinline__ int lower_bound_u32(const uint32_t* a, int n, uint32_t x) {
  int l = 0, r = n;
  while (l < r) {
    const int m = (l + r) >> 1;
    if (a[m] < x)
      l = m + 1;
    else
      r = m;
  }
  return l;
}
__device__ __forceinline__ int upper_bound_u32(const uint32_t* a, int n, uint32_t x) {
  int l = 0, r = n;
  while (l < r) {
    const int m = (l + r) >> 1;
    if (a[m] <= x)
      l = m + 1;
    else
      r = m;
  }
  return l;
}

template <int NT>
__global__ __launch_bounds__(NT) void generic_kernel(
    const float* __restrict__ logits, int64_t V, const RowParams* __restrict__ rp,
    const Patch* __restrict__ patches, const int32_t* __restrict__ patch_cnt, int pcap,
    const int32_t* __restrict__ generic_list, const int32_t* __restrict__ generic_count,
    const float* __restrict__ row_max, const double* __restrict__ d_u, uint64_t* __restrict__ rng,
    int32_t* __restrict__ out, uint32_t* __restrict__ scratch, int64_t vpad, DebugPtrs dbg) {
  constexpr int NW = NT / kWave;
  __shared__ uint32_t wcnt[NW * 256];
  __shared__ uint32_t dbase[256];
  __shared__ uint32_t drun[256];
  __shared__ int smem[NT / kWave + 4];
  __shared__ double s_u;
  __shared__ float s_f;
  __shared__ int s_i[4];
  const int n = (int)V;
  uint32_t* kA = scratch + (int64_t)blockIdx.x * vpad * 5;
  uint32_t* iA = kA + vpad;
  uint32_t* kB = iA + vpad;
  uint32_t* iB = kB + vpad;
  float* work = reinterpret_cast<float*>(iB + vpad);
  const int count = *generic_count;
  const int lane = lane_id();
  (void)row_max;
  for (int li = blockIdx.x; li < count; li += gridDim.x) {
    const int row = generic_list[li];
    const RowParams P = rp[row];
    const float* __restrict__ src = logits + (int64_t)row * V;
    // final values -> keys (patches applied over the plain pass)
    for (int i = threadIdx.x; i < n; i += NT) {
      kA[i] = ~f2key(src[i] * P.invT);
      iA[i] = (uint32_t)i;
    }
    __syncthreads();
    const int pn = patch_cnt[row];
    const Patch* pl = patches + (int64_t)row * pcap;
    for (int q = threadIdx.x; q < pn; q += NT) {
      const Patch p = pl[q];
      kA[p.id] = ~f2key(apply_patch(src[p.id], p, P) * P.invT);
    }
    __syncthreads();
    radix_sort_pass<NT>(kA, iA, kB, iB, n, 0, wcnt, dbase, drun);
    radix_sort_pass<NT>(kB, iB, kA, iA, n, 8, wcnt, dbase, drun);
    radix_sort_pass<NT>(kA, iA, kB, iB, n, 16, wcnt, dbase, drun);
    radix_sort_pass<NT>(kB, iB, kA, iA, n, 24, wcnt, dbase, drun);
    // kA: ~key ascending (value descending, index ascending on ties)
    if (threadIdx.x == 0) s_u = row_uniform(d_u, rng, row);
    __syncthreads();
    if (P.mode == kModeFull) {
      // candidates = the whole sorted row; values into work, ids stay in iA
      for (int i = threadIdx.x; i < n; i += NT) work[i] = key2f(~kA[i]);
      __syncthreads();
      // reuse kB as the exp buffer
      const TailOut t = softmax_cutoff_draw<NT>(work, iA, reinterpret_cast<float*>(kB), n, P, s_u,
                                                smem);
      if (threadIdx.x == 0) out[row] = t.id;
      write_debug<NT>(dbg, row, 4, t.n, n, t.total, iA, reinterpret_cast<float*>(kB));
      __syncthreads();
      continue;
    }
    // ---- top-k row (k < V) by the heap rule ----
    const int k = P.k;
    const uint32_t Tn = kA[k - 1];  // ~key of the k-th largest
    const int g = lower_bound_u32(kA, n, Tn);
    const int tend = upper_bound_u32(kA, n, Tn);
    const int m = k - g;
    int take_lo, take_hi;  // selected ties: sorted positions [take_lo, take_hi)
    if (tend == k) {
      take_lo = g;
      take_hi = k;
    } else {
      // p*: the k-th element in index order among sorted[0, tend).  Sort G's
      // indices ascending (in kB), then merge-walk with the ties (iA[g..tend)).
      const int gp = next_pow2(g > 0 ? g : 1);
      uint64_t* gs = reinterpret_cast<uint64_t*>(kB);  // spans kB+iB
      for (int i = threadIdx.x; i < gp; i += NT) gs[i] = (i < g) ? (uint64_t)iA[i] : ~0ull;
      __syncthreads();
      bitonic_sort_u64<NT>(gs, gp, false);
      if (threadIdx.x == 0) {
        int a = 0, b = 0;  // a over G, b over ties
        int taken = 0;
        while (taken < k) {
          const uint64_t gi = (a < g) ? gs[a] : ~0ull;
          const uint64_t ti = (g + b < tend) ? (uint64_t)iA[g + b] : ~0ull;
          if (gi < ti)
            ++a;
          else
            ++b;
          ++taken;
        }
        s_i[0] = g + b - m;  // the last m ties taken
        s_i[1] = g + b;
      }
      __syncthreads();
      take_lo = s_i[0];
      take_hi = s_i[1];
      __syncthreads();
    }
    // reference order: value descending, index descending on ties.  Reverse
    // every run of equal values among G; the selected ties come last, reversed.
    for (int i = threadIdx.x; i < g; i += NT) {
      const uint32_t key = kA[i];
      const int a = lower_bound_u32(kA, g, key);
      const int b = upper_bound_u32(kA, g, key);
      const int o = a + (b - 1 - i);
      work[o] = key2f(~key);
      reinterpret_cast<int32_t*>(kB)[o] = (int32_t)iA[i];
    }
    for (int i = take_lo + threadIdx.x; i < take_hi; i += NT) {
      const int o = g + (take_hi - 1 - i);
      work[o] = key2f(~kA[i]);
      reinterpret_cast<int32_t*>(kB)[o] = (int32_t)iA[i];
    }
    __syncthreads();
    const TailOut t = softmax_cutoff_draw<NT>(work, reinterpret_cast<int32_t*>(kB),
                                              reinterpret_cast<float*>(iB), k, P, s_u, smem);
    if (threadIdx.x == 0) out[row] = t.id;
    write_debug<NT>(dbg, row, 4, t.n, k, t.total, reinterpret_cast<int32_t*>(kB),
                    reinterpret_cast<float*>(iB));
    __syncthreads();
    (void)lane;
    (void)s_f;
  }
}

// ---------------------------------------------------------------------------
// small helpers
// ---------------------------------------------------------------------------
__global__ void accept_host_kernel(const int32_t* __restrict__ ids, int B, int count,
                                   int32_t* __restrict__ hist, int64_t* __restrict__ hist_len,
                                   int hcap, int row_only) {
  const int b = row_only >= 0 ? row_only : (int)blockIdx.x;
  const int64_t len = hist_len[b];
  const int32_t* src = ids + (row_only >= 0 ? 0 : (int64_t)b * count);
  // Only the last hcap ids survive in the ring; writing just those keeps
  // every slot single-writer when count > hcap.
  const int first = count > hcap ? count - hcap : 0;
  for (int j = first + (int)threadIdx.x; j < count; j += blockDim.x)
    hist[(int64_t)b * hcap + (int)((len + j) % hcap)] = src[j];
  __syncthreads();
  if (threadIdx.x == 0) hist_len[b] = len + count;
  (void)B;
}

__global__ void accept_device_kernel(const int32_t* __restrict__ ids, int B, int64_t V,
                                     int32_t* __restrict__ hist, int64_t* __restrict__ hist_len,
                                     int hcap) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  const int64_t len = hist_len[b];
  int32_t id = ids[b];
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


template <int Q, bool VEC>
static hipError_t launch_chunk(const LaunchArgs& a, hipStream_t s) {
  hipLaunchKernelGGL((chunk_kernel<kChunkVec4, Q, VEC>), dim3(a.B * a.nchunks),
                     dim3(kChunkThreads), 0, s, a.logits, a.V, a.nchunks, a.rp, a.patches,
                     a.patch_cnt, a.pcap, a.stats, a.cand, a.ccap);
  return hipGetLastError();
}

hipError_t launch_sample(const LaunchArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(prep_kernel, dim3(a.B), dim3(256), 0, s, a.rp, a.V, a.hist, a.hist_len,
                     a.hcap, a.bias_ids, a.bias_vals, a.patches, a.patch_cnt, a.pcap,
                     a.prep_scratch, a.prep_stride, a.generic_count);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int q = a.qmax <= 1 ? 1 : a.qmax <= 2 ? 2 : a.qmax <= 4 ? 4 : 8;
  if (a.ev_start && (e = hipEventRecord(a.ev_start, s)) != hipSuccess) return e;
  if (a.vec4) {
    if (q == 1) e = launch_chunk<1, true>(a, s);
    else if (q == 2) e = launch_chunk<2, true>(a, s);
    else if (q == 4) e = launch_chunk<4, true>(a, s);
    else e = launch_chunk<8, true>(a, s);
  } else {
    if (q == 1) e = launch_chunk<1, false>(a, s);
    else if (q == 2) e = launch_chunk<2, false>(a, s);
    else if (q == 4) e = launch_chunk<4, false>(a, s);
    else e = launch_chunk<8, false>(a, s);
  }
  if (e != hipSuccess) return e;
  if (a.ev_stop && (e = hipEventRecord(a.ev_stop, s)) != hipSuccess) return e;
  hipLaunchKernelGGL(merge_kernel<kMergeThreads>, dim3(a.B), dim3(kMergeThreads), a.merge_lds, s,
                     a.rp, a.nchunks, a.stats, a.cand, a.ccap, a.mcap, a.d_u, a.rng, a.out,
                     a.row_max, a.generic_list, a.generic_count, a.dbg);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(generic_kernel<kGenericThreads>, dim3(a.gen_blocks), dim3(kGenericThreads),
                     0, s, a.logits, a.V, a.rp, a.patches, a.patch_cnt, a.pcap, a.generic_list,
                     a.generic_count, a.row_max, a.d_u, a.rng, a.out, a.gen_scratch, a.gen_vpad,
                     a.dbg);
  return hipGetLastError();
}

hipError_t launch_accept_host(const int32_t* d_ids, int B, int count, int32_t* hist,
                              int64_t* hist_len, int hcap, int row_only, hipStream_t s) {
  hipLaunchKernelGGL(accept_host_kernel, dim3(row_only >= 0 ? 1 : B), dim3(256), 0, s, d_ids, B,
                     count, hist, hist_len, hcap, row_only);
  return hipGetLastError();
}

hipError_t launch_accept_device(const int32_t* d_ids, int B, int64_t V, int32_t* hist,
                                int64_t* hist_len, int hcap, hipStream_t s) {
  hipLaunchKernelGGL(accept_device_kernel, dim3((B + 255) / 256), dim3(256), 0, s, d_ids, B, V,
                     hist, hist_len, hcap);
  return hipGetLastError();
}

hipError_t set_kernel_attributes() {
  return hipFuncSetAttribute(reinterpret_cast<const void*>(&merge_kernel<kMergeThreads>),
                             hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024 - 8192);
}

hipError_t launch_expf(const float* x, float* y, int64_t n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(expf_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, y, n);
  return hipGetLastError();
}

}  // namespace nls
