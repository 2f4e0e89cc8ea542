// nls_device.h -- device code of the batched token sampler's two kernels
// (gfx950); instantiated by nls_stream_*.hip and nls_generic.hip.
//
// One nls_sample call over B rows of V fp32 logits runs two kernels:
//   1. stream_kernel   (B x S workgroups; S slices per row)  the single HBM
//      pass.  A workgroup builds its slice's penalty/bias patch table in LDS
//      from the row's history window and logit bias (sampler.nim:64-76),
//      streams the slice tile by tile (occupancy hides HBM latency), applies patches
//      and temperature (:80-81), tracks the first argmax (:45-49, :77-78) and,
//      on top-k rows, keeps every value that can still be among the row's k
//      best in an LDS buffer behind a rising threshold.  The workgroup that
//      completes a row (the only one when S == 1) selects the heap-path
//      members in reference order (:85-95), then runs softmax (:98-100),
//      top-p (:103-108), min-p (:110-114) and the draw (:115-121).
//      Workgroups: one 1024-thread workgroup per row when the batch fills
//      the chip or the row is small; two 512-thread workgroups per CU for
//      large batches of top-k rows with k > 64; otherwise rows split over
//      256-thread slices.
//   2. generic_kernel  full-sort rows (:96-97) and rows the streaming kernel
//      hands on (candidate or patch overflow, a speculative threshold that
//      admitted fewer than k): the row's distinct values with their
//      multiplicities and the exact run closed forms of the sequential fp32
//      chains (grouped_row), or else a whole-row stable radix sort.
//
// All fp32/fp64 arithmetic follows the reference's order; this file is built
// with -ffp-contract=off so no multiply-add is fused.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "nls_exp64.h"
#include "nls_expf.h"
#include "nls_grouped.h"
#include "nls_internal.h"
#include "nls_primitives.h"

namespace nls {

// Phase timestamps (the `phases` build only: -DNLS_PHASE_STAMPS): per row,
// slot i of nls_phase_stamp holds the real-time counter (100 MHz) when the
// row's workgroup reached phase i (or, for NLS_STAMP_VALUE, a count);
// nls_wave_stamp holds each wave's end of stream.  Each unit has its own
// copy; the k64 unit's is read back (nls_phase_stamps).
#ifdef NLS_PHASE_STAMPS
constexpr int kStampRows = 4096;
static __device__ uint64_t nls_phase_stamp[kStampRows * 16];
static __device__ uint64_t nls_wave_stamp[kStampRows * 16];
static __device__ uint64_t nls_detail_stamp[kStampRows * 16];
static __device__ uint64_t nls_gen_stamp[kStampRows * 16];  // the grouped path's phases, per row
#define NLS_GSTAMP(row, i)                                                                       \
  do {                                                                                           \
    if (threadIdx.x == 0 && (row) < kStampRows)                                                 \
      nls_gen_stamp[(row) * 16 + (i)] = __builtin_amdgcn_s_memrealtime();                        \
  } while (0)
#define NLS_STAMP(row, i)                                                                        \
  do {                                                                                           \
    if (__lane_id() == 0 && (row) < kStampRows)                                                 \
      nls_phase_stamp[(row) * 16 + (i)] = __builtin_amdgcn_s_memrealtime();                      \
  } while (0)
#define NLS_STAMP_VALUE(row, i, v)                                                               \
  do {                                                                                           \
    if (__lane_id() == 0 && (row) < kStampRows) nls_phase_stamp[(row) * 16 + (i)] = (uint64_t)(v); \
  } while (0)
#define NLS_DETAIL_STAMP(row, i)                                                                 \
  do {                                                                                           \
    if (__lane_id() == 0 && (row) < kStampRows)                                                 \
      nls_detail_stamp[(row) * 16 + (i)] = __builtin_amdgcn_s_memrealtime();                     \
  } while (0)
#define NLS_DETAIL_CLOCK(row, i)                                                                 \
  do {                                                                                           \
    if (__lane_id() == 0 && (row) < kStampRows)                                                 \
      nls_detail_stamp[(row) * 16 + (i)] = __builtin_amdgcn_s_memtime();                         \
  } while (0)
#define NLS_WAVE_STAMP(row, w)                                                                   \
  do {                                                                                           \
    if (__lane_id() == 0 && (row) < kStampRows)                                                 \
      nls_wave_stamp[(row) * 16 + (w)] = __builtin_amdgcn_s_memrealtime();                       \
  } while (0)
#else
#define NLS_GSTAMP(row, i) \
  do {                     \
  } while (0)
#define NLS_STAMP(row, i) \
  do {                    \
  } while (0)
#define NLS_STAMP_VALUE(row, i, v) \
  do {                             \
  } while (0)
#define NLS_WAVE_STAMP(row, w) \
  do {                         \
  } while (0)
#define NLS_DETAIL_STAMP(row, i) \
  do {                           \
  } while (0)
#define NLS_DETAIL_CLOCK(row, i) \
  do {                           \
  } while (0)
#endif

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Penalties first (:71-74), then bias (:76), on the original logit.
__device__ __forceinline__ float apply_patch(float v, float pen, float bias, uint32_t flags,
                                             const RowParams& P) {
  if (flags & kPatchPen) {
    if (P.rp_active) v = (v > 0.0f) ? (v / P.rp32) : (v * P.rp32);
    v = v - pen;
  }
  if (flags & kPatchBias) v = v + bias;
  return v;
}

// Reads a row-uniform value through the constant address space, which lets
// the compiler use scalar loads: nothing in the kernel writes it.
template <typename T>
__device__ __forceinline__ T load_const(const T* p) {
  static_assert(sizeof(T) % 4 == 0, "whole words");
  typedef const __attribute__((address_space(4))) uint32_t ConstWord;
  const ConstWord* w = (const ConstWord*)p;
  uint32_t x[sizeof(T) / 4];
#pragma unroll
  for (size_t i = 0; i < sizeof(T) / 4; ++i) x[i] = w[i];
  return __builtin_bit_cast(T, x);
}

// Buffer resource over a slice of `len` floats: loads at or beyond `len`
// return 0 without touching memory, so tile loads need no per-lane branch (a
// divergent branch around a load makes the compiler wait for it on the spot).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t slice_rsrc(const float* src, int len) {
  constexpr int kRsrcWord3 = 0x00020000;  // gfx9 untyped 32-bit buffer
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(src), (short)0, len * 4, kRsrcWord3);
}

// Loads float4 group j of the unit at `toff` of a slice: thread `th` of the
// unit owns the groups at toff + j * GS + th * 4 (GS floats apart), so each
// wave's load covers 1 KB contiguously.  Elements at or beyond the slice read
// as 0 and are masked by the caller.  Loads are nontemporal: every logit is
// read once.
template <int GS, bool VEC>
__device__ __forceinline__ f32x4 load_group(__amdgpu_buffer_rsrc_t rs, int toff, int j, int th) {
  constexpr int kNT = 2;  // cache policy: nt
  const int b = (toff + j * GS + th * 4) * 4;
  if (VEC) {
    // VEC implies len % 4 == 0: a group is either whole or absent
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, b, 0, kNT));
  } else {
    f32x4 r;
    r.x = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, b + 0, 0, kNT));
    r.y = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, b + 4, 0, kNT));
    r.z = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, b + 8, 0, kNT));
    r.w = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, b + 12, 0, kNT));
    return r;
  }
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
  int nan_cand;  // kPathNaN when a candidate value is NaN, else 0
};

// Wave-level fp32 chain over x[0..cnt) in index order: acc = acc OP x[0] OP
// x[1] ... as a sequence of dependent adds (or subtractions), exactly the
// reference's sequential accumulation.  Past cnt the values read +0, which
// leave acc unchanged.  stop(value, i) asks whether the chain ends after
// element i with the running value `value`; the walk returns the first such
// i (cnt if none) and, in *at, the running value there.  `stop` must be
// monotone along the chain (once true it stays true, as for a running sum of
// non-negative terms against a bound, or a difference of them against 0):
// it is tested once per block of 64, and only the block where it first holds
// (or where the value turns NaN) is walked again keeping every lane's value.
// Lane l holds element b0 + l of a block and readlane broadcasts it, so a
// step is one readlane and one operation; blocks are fetched 8 ahead so that
// a walk over global scratch does not wait a round trip per block.
template <bool SUB, bool HAS_STOP, typename XPtr, typename Stop>
__device__ __forceinline__ int chain_walk(XPtr x, int cnt, float& acc, Stop stop, float* at = nullptr) {
  constexpr int PF = 8;
  const int lane = lane_id();
  for (int base = 0; base < cnt; base += kWave * PF) {
    float xs[PF];
#pragma unroll
    for (int u = 0; u < PF; ++u) {
      const int i = base + u * kWave + lane;
      xs[u] = x[min(i, cnt - 1)];
      xs[u] = i < cnt ? xs[u] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < PF; ++u) {
      const int b0 = base + u * kWave;
      if (b0 >= cnt) break;
      const float a0 = acc;
#pragma unroll
      for (int l = 0; l < kWave; ++l) acc = SUB ? acc - lane_f(xs[u], l) : acc + lane_f(xs[u], l);
      if (HAS_STOP && (acc != acc || stop(acc, min(b0 + kWave, cnt) - 1))) {
        float r = a0, mine = 0.0f;
#pragma unroll
        for (int l = 0; l < kWave; ++l) {
          r = SUB ? r - lane_f(xs[u], l) : r + lane_f(xs[u], l);
          if (lane == l) mine = r;
        }
        const uint64_t hit = __ballot(b0 + lane < cnt && stop(mine, b0 + lane));
        if (hit) {
          const int hl = __ffsll((unsigned long long)hit) - 1;
          if (at) *at = lane_f(mine, hl);
          return b0 + hl;
        }
      }
    }
  }
  return cnt;
}

// chain_walk's contract over an LDS array, with the running value held whole
// by every lane: each step is one dependent fp32 operation on a term that all
// lanes read from the same LDS address (a broadcast), so no lane-to-lane move
// sits in the chain and every branch is uniform.  Full blocks of 32 terms are
// read as eight 16-byte loads; a partial block at either end with 4-byte
// loads clamped into the array, padded with +0, which leaves the value (a sum
// of terms >= 0 from +0, or a difference of them) unchanged.  stop is tested
// once per block (it is monotone along the chain, or the value turned NaN),
// and the block where it holds is walked again step by step.  Every lane
// calls it.
template <bool SUB, bool HAS_STOP, typename Stop>
__device__ __forceinline__ int chain_lds(const float* x, int cnt, float& acc, Stop stop, float* at = nullptr) {
  constexpr int B = 32;      // terms per block
  constexpr int BQ = B / 4;  // 16-byte reads per block
  int res = cnt;
  float a = acc;
  if (cnt <= 0) return res;
  auto op = [](float s, float t) -> float { return SUB ? s - t : s + t; };
  auto uni = [](bool c) -> bool { return __builtin_amdgcn_readfirstlane((int)c) != 0; };
  // B steps over t (elements i0 ..); true when stop holds at one of them.
  // The block where it holds is walked again from its start, its terms read
  // from LDS once more (through an opaque index, so that neither the terms
  // nor the running values of the first walk stay in registers for it).
  auto run = [&](const float (&t)[B], int i0) -> bool {
    const float a0 = a;
#pragma unroll
    for (int j = 0; j < B; ++j) a = op(a, t[j]);
    if (HAS_STOP && uni(a != a || stop(a, i0 + B - 1))) {
      float r = a0;
      int o = i0;
      asm volatile("" : "+v"(r), "+s"(o));
#pragma unroll
      for (int j = 0; j < B; ++j) {
        r = op(r, o + j < cnt ? x[o + j] : 0.0f);
        if (uni(stop(r, i0 + j))) {
          res = i0 + j;
          if (at) *at = r;
          return true;
        }
      }
    }
    return false;
  };
  auto partial = [&](int i0, int m) -> bool {  // elements i0 .. i0 + m - 1 (m <= B)
    float t[B];
#pragma unroll
    for (int j = 0; j < B; ++j) t[j] = x[min(i0 + j, cnt - 1)];
#pragma unroll
    for (int j = 0; j < B; ++j) t[j] = j < m ? t[j] : 0.0f;
    return run(t, i0);
  };
  const int head = min(cnt, (int)((16u - ((uint32_t)(uintptr_t)x & 15u)) & 15u) >> 2);
  bool done = head > 0 && partial(0, head);
  const int nb = (cnt - head) / B;
  const float4* x4 = reinterpret_cast<const float4*>(x + head);
  for (int b = 0; b < nb && !done; ++b) {
    float t[B];
#pragma unroll
    for (int q = 0; q < BQ; ++q) {
      const float4 c = x4[b * BQ + q];
      t[4 * q + 0] = c.x;
      t[4 * q + 1] = c.y;
      t[4 * q + 2] = c.z;
      t[4 * q + 3] = c.w;
    }
    done = run(t, head + b * B);
  }
  const int i1 = head + nb * B;
  if (!done && i1 < cnt) partial(i1, cnt - i1);
  acc = a;
  return res;
}

// beyond (a workgroup-shared flag, or null): set when a step ran past the
// last candidate -- top-p not reached, min-p keeping every candidate, or the
// draw not ended -- so that a caller holding only the row's leading
// candidates can tell whether the rest of the row could have mattered.
template <int NT, bool E_LDS = false, typename VPtr, typename IPtr, typename EPtr>
__device__ __forceinline__ TailOut softmax_cutoff_draw(VPtr val, IPtr ids, EPtr e, int ncand, const RowParams& P,
                                       double u, int* smem, int* beyond = nullptr) {
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
    if constexpr (E_LDS)
      chain_lds<false, false>(e, ncand, s, [](float, int) { return false; });
    else
      chain_walk<false, false>(e, ncand, s, [](float, int) { return false; });
    if (lane == 0) s_sum = s;
  }
  __syncthreads();
  const float s = s_sum;
  for (int i = threadIdx.x; i < ncand; i += NT) e[i] = e[i] / s;
  __syncthreads();
  if (threadIdx.x < kWave) {
    int n = ncand;
    // the top-p running sum is the same fp32 sequence as the total over its
    // first n terms: when min-p keeps n, the total is the running sum there
    float cum_n = 0.0f;
    bool past = false;
    if (P.topp_active) {
      // the first i with (double)(e_0 + ... + e_i) >= topP
      float cum = 0.0f, at = 0.0f;
      auto reached = [&](float c, int) { return (double)c >= P.topP; };
      int stop;
      if constexpr (E_LDS)
        stop = chain_lds<false, true>(e, ncand, cum, reached, &at);
      else
        stop = chain_walk<false, true>(e, ncand, cum, reached, &at);
      if (stop < ncand) n = stop + 1;
      cum_n = stop < ncand ? at : cum;
      past = stop >= ncand;
    }
    const int n_topp = n;
    if (P.minp_active) {
      // m = the first index >= 1 whose probability is below thr (n if none)
      const float thr = e[0] * P.minP32;
      int m = n;
      for (int base = 1; base < n; base += kWave) {
        const int i = base + lane;
        const uint64_t fail = __ballot(i < n && !(e[min(i, n - 1)] >= thr));
        if (fail) {
          m = base + __ffsll((unsigned long long)fail) - 1;
          break;
        }
      }
      past |= m == ncand;
      n = m;
    }
    float total = 0.0f;
    if (P.topp_active && n == n_topp)
      total = cum_n;
    else if constexpr (E_LDS)
      chain_lds<false, false>(e, n, total, [](float, int) { return false; });
    else
      chain_walk<false, false>(e, n, total, [](float, int) { return false; });
    float r = (float)u * total;
    auto drawn = [](float rr, int) { return rr <= 0.0f; };
    int hit;
    if constexpr (E_LDS)
      hit = chain_lds<true, true>(e, n, r, drawn);
    else
      hit = chain_walk<true, true>(e, n, r, drawn);
    const int pos = hit < n ? hit : n - 1;
    past |= hit >= n && n == ncand;
    if (lane == 0) {
      s_n = n;
      s_total = total;
      s_pos = pos;
      if (beyond) *beyond = past ? 1 : 0;
    }
  }
  __syncthreads();
  TailOut t;
  t.n = s_n;
  t.total = s_total;
  t.id = ids[s_pos];
  // (NaN keys sort to the ends of the candidate order)
  const float last = val[ncand - 1];
  t.nan_cand = (mx != mx || last != last) ? kPathNaN : 0;
  return t;
}



template <int NT, typename EPtr, typename IPtr>
__device__ __forceinline__ void write_debug(const DebugPtrs& dbg, int row, int path, int n, int ncand,
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


// Agent-scope (device-wide coherent) relaxed stores and loads for the slice
// exchange between workgroups of one row.
template <typename T>
__device__ __forceinline__ void store_agent(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ T load_agent(const T* p) {
  return __hip_atomic_load(const_cast<T*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Lists `row` for the whole-row path; returns true (the caller's flag that it
// has published an entry).
__device__ __forceinline__ bool push_generic(int32_t* list, int32_t* count, int row) {
  store_agent(&list[atomicAdd(count, 1)], row);
  return true;
}


// ---------------------------------------------------------------------------
// Heap-path members (sampler.nim:85-95) from a candidate set
// ---------------------------------------------------------------------------
// ent[0..N): (key << 32 | id) entries holding every element of the row whose
// key is >= some threshold no larger than the row's k-th largest key, with
// N >= k and k < V.  Writes the k members, key-major and in no particular
// order, to mem[0..k).  Membership: T = k-th largest, G = {key > T},
// m = k - |G|, p* = index at which the running count of {key >= T} reaches
// k; members = G + the m largest indices among ties at T with index <= p*.
// Returns false (uniformly) when the tie set does not fit `mem`.
// `s_cnt` is an LDS counter set to 0 before the call.
template <int NT>
__device__ __forceinline__ bool topk_members(uint64_t* ent, int N, int k, uint64_t* mem, int mcap,
                                             uint32_t* hist, int* smem, int* s_cnt) {
  // fit = k: stop as soon as the items >= the current prefix are exactly k
  const SelectResult sr = block_select<NT>(
      [&](auto fn) {
        for (int i0 = 0; i0 < N; i0 += NT) {
          const int i = i0 + (int)threadIdx.x;
          const bool in = i < N;
          fn(in ? (uint32_t)(ent[i] >> 32) : 0u, in);
        }
      },
      k, k, hist, smem);
  const uint32_t T = sr.tau;
  const int gt = sr.gt, ge = sr.ge;
  if (ge == k) {
    // no excess ties: the members are exactly the entries >= T
    for (int i = threadIdx.x; i < N; i += NT) {
      const uint64_t x = ent[i];
      if ((uint32_t)(x >> 32) >= T) mem[atomicAdd(s_cnt, 1)] = x;
    }
    __syncthreads();
    return true;
  }
  // excess ties at the exact T (the select ran to the last digit)
  const int m = k - gt;
  const int gpow = next_pow2(ge);
  if (gpow > mcap) return false;
  int mine = 0;
  for (int i = threadIdx.x; i < N; i += NT) mine += ((uint32_t)(ent[i] >> 32) >= T);
  int tot;
  int pos = block_excl_scan<NT>(mine, smem, tot);
  for (int i = threadIdx.x; i < N; i += NT) {
    const uint64_t x = ent[i];
    if ((uint32_t)(x >> 32) >= T) mem[pos++] = (x << 32) | (x >> 32);  // index-major
  }
  for (int i = ge + threadIdx.x; i < gpow; i += NT) mem[i] = ~0ull;
  __syncthreads();
  bitonic_sort_u64<NT>(mem, gpow, false);
  // mem[0..k): the elements >= T with index <= p*; keep the last m ties
  int tl = 0;
  const int per = (k + NT - 1) / NT;
  const int lo = min(k, (int)threadIdx.x * per), hi = min(k, lo + per);
  for (int i = lo; i < hi; ++i) tl += ((uint32_t)mem[i] == T);
  int ntie;
  int trank = block_excl_scan<NT>(tl, smem, ntie);
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
  return true;
}

// The row's uniform (sampler.nim:117): the caller's value, or the next
// rand(1.0) of the row's own stream, whose advanced state is written back.
// `u_in`/`st` were read at kernel start by the calling lane.
__device__ __forceinline__ double take_uniform(const double* d_u, double u_in, uint64_t st0,
                                               uint64_t st1, uint64_t* rng, int row) {
  if (d_u) return u_in;
  uint64_t st[2] = {st0, st1};
  const double u = nim_rand_unit(st);
  rng[2 * row] = st[0];
  rng[2 * row + 1] = st[1];
  return u;
}

__device__ __forceinline__ float lane_fc(float x, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l));
}

// The reference's tail on one wave, for k <= 64 members (mem[0..k), any
// order): lane i holds candidate i after a descending (value, index) rank
// sort (sampler.nim:88-95), then softmax (:98-100, :51-57), top-p (:103-108),
// min-p (:110-114) and the draw (:115-121).  Every sequential fp32 sum runs
// in candidate order as an unrolled chain; the top-p running sum doubles as
// `total`, which the reference accumulates with the same operations.
__device__ __forceinline__ void wave_tail(uint64_t* mem, int k, const RowParams& P,
                                          double u_lane0, int row, int32_t* out,
                                          const DebugPtrs& dbg, int path = 2) {
  const int lane = lane_id();
  // rank sort: each member's position is the number of members above it
  // (entries are distinct (key, id) pairs; the zero padding ranks last)
  uint64_t x = (lane < k) ? mem[lane] : 0ull;
  {
    int rank = 0;
#pragma unroll 8
    for (int j = 0; j < k; ++j) rank += (mem[j] > x);  // one LDS broadcast per step
    if (lane < k) mem[rank] = x;  // the whole wave has read mem[] above
    x = (lane < k) ? mem[lane] : 0ull;
  }
  NLS_STAMP(row, 8);
  const bool valid = lane < k;
  const int id = (int)(uint32_t)x;
  const float v = key2f((uint32_t)(x >> 32));
  const float mx = lane_fc(v, 0);
  const float e = valid ? expf_cr(v - mx) : 0.0f;
  // s = e_0 + e_1 + ... in order
  // (unrolled over the wave: the zero tail past k leaves the sums unchanged)
  float ssum = 0.0f;
#pragma unroll
  for (int i = 0; i < kWave; ++i) ssum = ssum + lane_fc(e, i);
  const float p = valid ? e / ssum : 0.0f;
  NLS_STAMP(row, 9);
  float acc = 0.0f, cum = 0.0f;
#pragma unroll
  for (int i = 0; i < kWave; ++i) {
    acc = acc + lane_fc(p, i);
    if (lane == i) cum = acc;
  }
  int n = k;
  if (P.topp_active) {
    const uint64_t m = __ballot(valid && (double)cum >= P.topP);
    if (m) n = __ffsll((unsigned long long)m);
  }
  if (P.minp_active) {
    const float thr = lane_fc(p, 0) * P.minP32;
    const uint64_t m = __ballot(lane >= 1 && lane < n && !(p >= thr));
    if (m) n = __ffsll((unsigned long long)m) - 1;
  }
  const float total = lane_fc(cum, n - 1);
  NLS_STAMP(row, 10);
  const double u = __hiloint2double(__builtin_amdgcn_readlane(__double2hiint(u_lane0), 0),
                                    __builtin_amdgcn_readlane(__double2loint(u_lane0), 0));
  float r = (float)u * total;
  float rl = 0.0f;  // (lanes past n are not read)
#pragma unroll
  for (int i = 0; i < kWave; ++i) {
    r = r - lane_fc(p, i);
    if (lane == i) rl = r;
  }
  const uint64_t hit = __ballot(lane < n && rl <= 0.0f);
  const int pos = hit ? __ffsll((unsigned long long)hit) - 1 : n - 1;
  const int tok = __builtin_amdgcn_readlane(id, pos);
  const bool nan_c = dbg.path && __ballot(valid && v != v) != 0ull;  // a NaN candidate
  if (lane == 0) {
    out[row] = tok;
    if (dbg.n) dbg.n[row] = n;
    if (dbg.ncand) dbg.ncand[row] = k;
    if (dbg.total) dbg.total[row] = total;
    if (dbg.path) dbg.path[row] = path | (nan_c ? kPathNaN : 0);
  }
  if (lane < min(n, dbg.cap)) {
    if (dbg.cand_ids) dbg.cand_ids[(int64_t)row * dbg.cap + lane] = id;
    if (dbg.cand_probs) dbg.cand_probs[(int64_t)row * dbg.cap + lane] = p;
  }
}

// The next call's counters of the split whole-row launches, zeroed by every
// whole-row launch (a call whose rows the streaming kernel's last workgroup
// serves makes none: the host clears stale counts before a later call that
// splits).
__device__ __forceinline__ void zero_next_counters(const GenericArgs& g) {
  if (g.fb_next) store_agent(g.fb_next, 0);
  if (g.w_next) store_agent(g.w_next, 0);
}

template <int NT, bool GROUPED = false, bool CLAIM = false, bool ONLY = false>
__device__ __forceinline__ void generic_rows(const GenericArgs& a, int w0, int nw, int count, uint32_t* wcnt,
                                             uint32_t* dbase, uint32_t* drun, int* smem, double* s_u_p,
                                             int* s_i, float* s_rv, int* s_ri,
                                             unsigned char* glds = nullptr);

// LDS word of bin b of a 4096-bin histogram laid out for one wave's scan:
// bins form 64 ranges r of 64 consecutive bins j; the 4 bins 4q..4q+3 of
// range r sit at words (q * 64 + r) * 4 .. +3, so that the 64 lanes reading
// their ranges' bins 4q..4q+3 with one 16-byte load each cover 1 KB without
// bank conflicts.
__device__ __forceinline__ uint32_t hist4k_addr(uint32_t b) {
  const uint32_t r = b >> 6, j = b & 63u;
  return ((j >> 2) * 64u + r) * 4u + (j & 3u);
}

// One wave: the bin b of a 4096-bin histogram (hist4k_addr layout) where the
// count from the top bin down reaches `rank`, and the count in the bins
// above it.  Returns false when the whole histogram holds fewer.
__device__ __forceinline__ bool hist4k_rank(const uint32_t* hist, int rank, int& bin, int& above) {
  const int lane = lane_id();
  const int range = kWave - 1 - lane;  // lane l sums range 63 - l (largest first)
  int c = 0;
  const uint4* h4 = reinterpret_cast<const uint4*>(hist);
#pragma unroll
  for (int q = 0; q < kWave / 4; ++q) {
    const uint4 v = h4[q * kWave + range];
    c += (int)(v.x + v.y + v.z + v.w);
  }
  const int incl = wave_incl_scan(c);
  const uint64_t mk = __ballot(incl - c < rank && incl >= rank);
  if (!mk) return false;
  const int sl = __ffsll((unsigned long long)mk) - 1;
  const int ab = __builtin_amdgcn_readlane(incl - c, sl);
  const int r = kWave - 1 - sl;
  const int cb = (int)hist[hist4k_addr((uint32_t)(r * kWave + kWave - 1 - lane))];  // this lane's bin, from the top
  const int inc2 = wave_incl_scan(cb) + ab;
  const uint64_t m2 = __ballot(inc2 - cb < rank && inc2 >= rank);
  const int l2 = __ffsll((unsigned long long)m2) - 1;
  bin = r * kWave + (kWave - 1 - l2);
  above = __builtin_amdgcn_readlane(inc2 - cb, l2);
  return true;
}

// The rank-th largest of one key per thread (rank >= 1), to 24 bits: the
// returned key, with its low 8 bits zero, is at most that key, and every key
// at or above it agrees with that key in its top 24 bits.  Two 4096-bin
// histogram rounds (the top 12 bits, then the next 12 within the chosen bin)
// over h1 and h2 (4096 words each, LDS, free); every thread calls it.
template <int NT>
__device__ __forceinline__ uint32_t block_rank24(uint32_t key, int rank, uint32_t* h1, uint32_t* h2, int* smem) {
  constexpr int NW = NT / kWave;
  const int tid = threadIdx.x;
  uint4* z1 = reinterpret_cast<uint4*>(h1);
  uint4* z2 = reinterpret_cast<uint4*>(h2);
  const uint4 z = make_uint4(0u, 0u, 0u, 0u);
  for (int i = tid; i < 1024; i += NT) {
    z1[i] = z;
    z2[i] = z;
  }
  __syncthreads();
  atomicAdd(&h1[hist4k_addr(key >> 20)], 1u);
  __syncthreads();
  if (tid < kWave) {
    int b = 0, ab = 0;
    if (!hist4k_rank(h1, rank, b, ab)) b = 0, ab = 0;
    if (tid == 0) {
      smem[NW + 1] = b;
      smem[NW + 2] = ab;
    }
  }
  __syncthreads();
  const uint32_t b1 = (uint32_t)smem[NW + 1];
  const int r2 = rank - smem[NW + 2];
  if ((key >> 20) == b1) atomicAdd(&h2[hist4k_addr((key >> 8) & 4095u)], 1u);
  __syncthreads();
  if (tid < kWave) {
    int b = 0, ab = 0;
    if (!hist4k_rank(h2, r2, b, ab)) b = 0;
    if (tid == 0) smem[NW + 3] = b;
  }
  __syncthreads();
  return (b1 << 20) | ((uint32_t)smem[NW + 3] << 8);
}

// ---------------------------------------------------------------------------
// 1. stream_kernel
// ---------------------------------------------------------------------------
// Dynamic LDS: cand[2][ccap] u64 | region A.
// Region A up to the final selection: bitmap[nwords] u32 | wpre[nwords] u16
// (padded to 4 bytes) | pfin[pcap] f32 | pbias[pcap] f32 | pflag[pcap] u32 |
// pid[pcap] i32.  Afterwards it holds the tail: mem[mcap] u64 |
// vals[kcap] f32 | ids[kcap] i32 | e[kcap] f32.
//
// Penalties and bias touch few ids of a slice [lo, lo + len) (the patched
// ids).  Bit (id - lo) of `bitmap` marks them; patch p of a marked id sits
// at wpre[w] + popcount(bits of word w below it).  Their original logits are
// gathered up front and their final values (pfin) computed once, so the
// stream leaves them out -- only where a value would be kept or would raise
// the argmax does it test the bitmap -- and they rejoin the candidates (or
// the argmax) after the stream.
template <int NT, bool VEC, int Q, bool WAVE>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(NT <= 512 ? 4 : 2)))
void stream_kernel(const StreamArgs a) {
  constexpr int NW = NT / kWave;
  constexpr int NV4 = kStreamVec4;
  constexpr int NE = NV4 * 4;
  constexpr int TE = NT * NE;
  // Units of the stream.  The wave path works in chunks of kWave * NE floats,
  // one wave each: every wave takes the chunk of tile 0, then further chunks
  // in index order from a shared counter, so that waves which get their data
  // early take more and all finish together.  The block path works in tiles
  // of TE floats, all threads together.
  constexpr int UE = WAVE ? kWave * NE : TE;  // floats per unit
  constexpr int GS = WAVE ? kWave * 4 : NT * 4;  // floats between a thread's groups
  constexpr int PER = kWaveCap / kWave;  // wave path: buffer entries per lane
  constexpr int M0 = (kWave + NW - 1) / NW;  // wave path: offers per wave (NW * M0 >= 64 >= k)
  constexpr int kMidUnits = 3;  // wave path: units before every wave offers its buffer maxima
  extern __shared__ __align__(16) unsigned char lds[];
  __shared__ int smem[NW + 4];
  // block_select histogram; while streaming, the wave path's per-wave ones
  constexpr int kHistWords = kSelWords > NW * kWaveBins ? kSelWords : NW * kWaveBins;
  __shared__ uint32_t shist[kHistWords];
  __shared__ int s_wn[NW];
  __shared__ uint32_t s_wt[NW];
  __shared__ uint32_t s_tau;  // wave path: the highest published wave threshold
  __shared__ uint32_t s_top[kWave];  // wave path: the lane maxima of tile 0, then the buffer maxima
  __shared__ int s_tile_cnt[3];
  __shared__ int s_cnt;
  __shared__ int s_next;  // wave path: the next unclaimed chunk (after the first two of every wave)
  __shared__ float s_rv[NW];
  __shared__ int s_ri[NW];
  __shared__ int s_last;
  __shared__ uint32_t s_te;  // wave path: the lead wave's bound, then its verdict
  __shared__ uint32_t s_mid[kWave];  // wave path: every wave's largest buffer keys after its first units
  __shared__ int s_midn;             // wave path: the waves that have written theirs
  __shared__ double s_u;

  // The row's work; every exit of it leads to the final section below.
  bool pushed = false;  // thread 0: this workgroup listed a row for the whole-row path
  auto run = [&]() __attribute__((always_inline)) {
    int row, sl;
    if (a.xcd_map) {
      const int x = (int)(blockIdx.x & 7u), slot = (int)(blockIdx.x >> 3);
      row = (slot / a.S) * 8 + x;
      sl = slot - (slot / a.S) * a.S;
    } else {
      row = (int)blockIdx.x / a.S;
      sl = (int)blockIdx.x - row * a.S;
    }
    const int tid = threadIdx.x;
    const int lane = lane_id();
    const int wv = tid >> 6;
    if (wv == 0) NLS_STAMP(row, 0);
    // The row's history ring and bias entries are requested first: they do not
    // depend on the row constants, so they go out while those load, before any
    // tile traffic.  Thread tid reads ring slots h * NT + tid and bias entry
    // tid (the bias lists sit at a fixed stride); whether a slot lies in the
    // penalty window, or an entry in the row's list, is decided once the row
    // constants are in.  Requests past the ring or the list read 0 and are
    // dropped by index.
    constexpr int HPT = 8;  // ring slots per thread
    constexpr int kOutOfRange = 0x7ffffff0;
    // (the requests are unconditional: a resource of zero records makes all of
    // them read 0, so no branch, and no wait, surrounds them)
    const bool ring_early = a.hcap > 0 && a.hcap <= NT * HPT;
    int hraw[HPT];
    {
      const __amdgpu_buffer_rsrc_t hr = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<int32_t*>(a.hist + (ring_early ? (int64_t)row * a.hcap : 0)), (short)0,
          ring_early ? a.hcap * 4 : 0, 0x00020000);
  #pragma unroll
      for (int h = 0; h < HPT; ++h) {
        const int slot = h * NT + tid;
        hraw[h] = (int)__builtin_amdgcn_raw_buffer_load_b32(hr, slot < a.hcap ? slot * 4 : kOutOfRange, 0, 0);
      }
    }
    const bool bias_early = a.bstride > 0 && a.bstride <= NT;
    int braw;
    float bval;
    {
      const int off = tid < a.bstride ? tid * 4 : kOutOfRange;
      const int64_t base = bias_early ? (int64_t)row * a.bstride : 0;
      const int nrec = bias_early ? a.bstride * 4 : 0;
      const __amdgpu_buffer_rsrc_t bi = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<int32_t*>(a.bias_ids + base), (short)0, nrec, 0x00020000);
      const __amdgpu_buffer_rsrc_t bv = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<float*>(a.bias_vals + base), (short)0, nrec, 0x00020000);
      braw = (int)__builtin_amdgcn_raw_buffer_load_b32(bi, off, 0, 0);
      bval = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(bv, off, 0, 0));
    }
    // The first unit of the slice follows at once (it needs no row constant);
    // the reads above return before it.
    const int lo = sl * a.L;
    const int len = (int)min((int64_t)a.L, a.V - (int64_t)lo);
    const float* __restrict__ src = a.logits + (int64_t)row * a.V + lo;
    const __amdgpu_buffer_rsrc_t rs = slice_rsrc(src, len);
    f32x4 R0[NV4];  // the unit in flight
    const int uth = WAVE ? lane : tid;        // this thread's place in a unit
    const int u0 = WAVE ? wv : 0;             // its first unit
  #pragma unroll
    for (int j = 0; j < NV4; ++j) R0[j] = load_group<GS, VEC>(rs, u0 * UE, j, uth);
    __builtin_amdgcn_sched_barrier(0);  // keep the requests here, ahead of the row constants
    // Row constants through the scalar unit: the constant address space tells
    // the compiler that nothing in this kernel writes them.
    const RowParams P = load_const(a.rp + row);
    const int64_t hlen = load_const(a.hist_len + row);
    if (a.row_done && load_const(a.row_done + row) != 0) {  // a finished row of a batched loop
      if (sl == 0 && tid == 0) a.out[row] = -1;
      return;
    }
    if (P.mode == kModeFull || !P.fast) {
      if (sl == 0 && tid == 0) pushed = push_generic(a.generic_list, a.generic_count, row);
      return;
    }
    const bool greedy = P.mode == kModeGreedy;
    const bool topk = P.mode == kModeTopK;
    const int k = P.k;

    uint64_t* cand = reinterpret_cast<uint64_t*>(lds);
    unsigned char* regA = lds + a.offA;
    uint32_t* bitmap = reinterpret_cast<uint32_t*>(regA);
    uint16_t* wpre = reinterpret_cast<uint16_t*>(regA + (size_t)a.nwords * 4);
    float* pfin = reinterpret_cast<float*>(regA + (size_t)a.nwords * 4 + (((size_t)a.nwords * 2 + 3) & ~(size_t)3));
    float* pbias = pfin + a.pcap;
    uint32_t* pflag = reinterpret_cast<uint32_t*>(pbias + a.pcap);  // flags | count << 2
    int32_t* pid = reinterpret_cast<int32_t*>(pflag + a.pcap);
    // patch slot of a patched slice-local offset: patched offsets are numbered
    // in index order (wpre holds the count before each bitmap word)
    auto slot_of = [&](int loc) -> int {
      const int w = loc >> 5;
      return wpre[w] + __popc(bitmap[w] & ((1u << (loc & 31)) - 1u));
    };

    // the row's uniform or RNG state, read now (scalar loads) so the tail
    // does not wait
    double u_in = 0.0;
    uint64_t st0 = 0ull, st1 = 0ull;
    if (!greedy) {
      if (a.d_u) {
        u_in = load_const(a.d_u + row);
      } else {
        st0 = load_const(a.rng + 2 * row);
        st1 = load_const(a.rng + 2 * row + 1);
      }
    }
    for (int q = tid; q < kHistWords; q += NT) shist[q] = 0u;  // the selects need it zeroed
    if (tid < kWave) s_mid[tid] = 0u;
    if (tid == 0) {
      s_tile_cnt[0] = 0;
      s_tile_cnt[1] = 0;
      s_tile_cnt[2] = 0;
      s_cnt = 0;
      s_tau = 0u;
      s_midn = 0;
      s_next = 2 * NW;
    }

    // ---- patched ids (penalties :64-74, bias :75-76) ----
    bool ovf = false;
    int npatch = 0;
    int n_hist = 0;
    if (P.pen_active && hlen > 0)
      n_hist = (int)((P.repeat_last_n > 0 && P.repeat_last_n < hlen) ? P.repeat_last_n : hlen);
    const bool has_patch = n_hist > 0 || P.bias_cnt > 0;
    // the whole window from the ring slots read above (else in rounds below)
    const bool one_round = ring_early;
    const bool bias_one = P.bias_cnt <= NT;  // one bias entry per thread at most
    const int hbase = n_hist > 0 ? (int)((hlen - n_hist) % a.hcap) : 0;
    const int32_t* __restrict__ hrow = a.hist + (int64_t)row * a.hcap;
    // History slot of window entry i (the ring wraps at hcap).
    auto hist_slot = [&](int i) -> int {
      const int slot = hbase + i;
      return slot >= a.hcap ? slot - a.hcap : slot;
    };
    // Slice-local offset of a window id, or -1 when it is not in the slice (ids
    // outside [0, V) are stored as -1 by accept).
    auto id_loc = [&](int id) -> int {
      const int loc = id - lo;
      return (id >= 0 && loc >= 0 && loc < len) ? loc : -1;
    };
    // Without the fixed bias stride the entries are read now, after the row
    // constants (and behind the first unit's traffic).
    if (!bias_early && P.bias_cnt > 0 && bias_one) {
      const int off = tid < P.bias_cnt ? tid * 4 : kOutOfRange;
      const __amdgpu_buffer_rsrc_t bi = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<int32_t*>(a.bias_ids + P.bias_off), (short)0, P.bias_cnt * 4, 0x00020000);
      const __amdgpu_buffer_rsrc_t bv = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<float*>(a.bias_vals + P.bias_off), (short)0, P.bias_cnt * 4, 0x00020000);
      braw = (int)__builtin_amdgcn_raw_buffer_load_b32(bi, off, 0, 0);
      bval = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(bv, off, 0, 0));
    }
    // slice-local offsets of this thread's window entries (one round) and bias
    // entry (-1: none): ring slot s holds window entry (s - hbase) mod hcap
    int hl[HPT];
  #pragma unroll
    for (int h = 0; h < HPT; ++h) {
      const int slot = h * NT + tid;
      int i = slot - hbase;
      if (i < 0) i += a.hcap;
      hl[h] = (one_round && n_hist > 0 && slot < a.hcap && i < n_hist) ? id_loc(hraw[h]) : -1;
    }
    const int b_loc = (bias_one && tid < P.bias_cnt) ? id_loc(braw) : -1;
    const float b_val = bval;
    if (has_patch) {
      const int nw = (len + 31) >> 5;
      // fn(loc) for every window entry of the slice (loc < 0: not in it)
      auto for_window = [&](auto fn) __attribute__((always_inline)) {
        if (one_round) {
  #pragma unroll
          for (int h = 0; h < HPT; ++h) fn(hl[h]);
        } else {
          for (int b0 = 0; b0 < n_hist; b0 += NT * HPT) {
            int l[HPT];
  #pragma unroll
            for (int h = 0; h < HPT; ++h) {
              const int i = b0 + h * NT + tid;
              l[h] = (i < n_hist) ? id_loc(hrow[hist_slot(i)]) : -1;
            }
  #pragma unroll
            for (int h = 0; h < HPT; ++h) fn(l[h]);
          }
        }
      };
      for (int w = tid; w < nw; w += NT) bitmap[w] = 0u;
      __syncthreads();
      for_window([&](int loc) {
        if (loc >= 0) atomicOr(&bitmap[loc >> 5], 1u << (loc & 31));
      });
      if (bias_one) {
        if (b_loc >= 0) atomicOr(&bitmap[b_loc >> 5], 1u << (b_loc & 31));
      } else {
        for (int j = tid; j < P.bias_cnt; j += NT) {
          const int loc = a.bias_ids[P.bias_off + j] - lo;
          if (loc >= 0 && loc < len) atomicOr(&bitmap[loc >> 5], 1u << (loc & 31));
        }
      }
      __syncthreads();
      const int wpt = (nw + NT - 1) / NT;
      const int w0 = min(nw, tid * wpt), w1 = min(nw, w0 + wpt);
      int c = 0;
      for (int w = w0; w < w1; ++w) c += __popc(bitmap[w]);
      int pre = block_excl_scan<NT>(c, smem, npatch);
      if (npatch > a.pcap) {
        ovf = true;  // uniform
      } else {
        for (int w = w0; w < w1; ++w) {
          wpre[w] = (uint16_t)pre;
          pre += __popc(bitmap[w]);
        }
        for (int p = tid; p < npatch; p += NT) {
          pbias[p] = 0.0f;
          pflag[p] = 0u;
        }
        __syncthreads();
        // every writer of pid[p] stores the same value
        for_window([&](int loc) {
          if (loc >= 0) {
            const int p = slot_of(loc);
            atomicAdd(&pflag[p], 1u << kPatchCountShift);  // the window count
            pid[p] = lo + loc;
          }
        });
        auto put_bias = [&](int loc, float val) {
          const int p = slot_of(loc);
          pbias[p] = val;  // bias ids are unique per row
          atomicOr(&pflag[p], (uint32_t)kPatchBias | (!(val <= 0.0f) ? (uint32_t)kPatchRise : 0u));
          pid[p] = lo + loc;
        };
        if (bias_one) {
          if (b_loc >= 0) put_bias(b_loc, b_val);
        } else {
          for (int j = tid; j < P.bias_cnt; j += NT) {
            const int loc = a.bias_ids[P.bias_off + j] - lo;
            if (loc >= 0 && loc < len) put_bias(loc, a.bias_vals[P.bias_off + j]);
          }
        }
      }
    }
    __syncthreads();
    auto patched = [&](int loc) -> bool {  // loc: slice-local offset
      return has_patch && ((bitmap[loc >> 5] >> (loc & 31)) & 1u);
    };
    // A patched logit met at or above the threshold keeps its original value
    // for the final pass.  One that stays below it cannot be a member unless
    // its patch can raise it (a positive or NaN bias, or penalties of the
    // raising sign): every other patch only lowers a logit (division by
    // rp >= 1 of a positive value, multiplication of a non-positive one,
    // subtraction of count * frequency + presence >= 0, a bias <= 0), and so
    // does the temperature's positive factor, in float rounding too.
    auto capture = [&](int loc, float raw) {
      const int p = slot_of(loc);
      pfin[p] = raw;
      atomicOr(&pflag[p], (uint32_t)kPatchSeen);
    };
    const bool row_rise =
        (P.rp_active && !(P.rp32 >= 1.0f)) || !(P.freq >= 0.0) || !(P.pres >= 0.0);
    auto may_rise = [&](uint32_t fl) -> bool {
      return (fl & kPatchRise) || (row_rise && (fl >> kPatchCountShift) > 0);
    };
    // The original logits of the ids whose patch may raise them are requested
    // now (slots tid + r * NT; the rest, if any, are read after the stream):
    // requests past the slice return 0 without reading memory, so the slots
    // without such a patch need no branch around the load.
    constexpr int RPT = 2;
    float rraw[RPT];
  #pragma unroll
    for (int r = 0; r < RPT; ++r) {
      const int p = tid + r * NT;
      const bool want = !ovf && p < npatch && may_rise(pflag[p]);
      rraw[r] = __builtin_bit_cast(
          float, __builtin_amdgcn_raw_buffer_load_b32(rs, want ? (pid[p] - lo) * 4 : kOutOfRange, 0, 0));
    }
    // greedy rows: the original logit at index 0 (argmax stays at 0 when the
    // final value there is NaN), read from the first tile
    float x0raw = 0.0f;

    // ---- the stream ----
    if (wv == 0) NLS_STAMP(row, 1);
    float bv = -__builtin_inff();
    int bi = 0x7fffffff;
    int buf_n = 0, cur = 0;
    uint32_t tau = 0u;
    // Block path on a whole row: the first refresh (tile 0) sets a threshold
    // that lets about 2k elements of the row through when the tile is typical
    // of it, so that the buffer rarely fills again: the spec_rank-th largest of
    // the threads' maxima of the tile, where spec_rank is the number of the NT
    // maxima (each over NE values) expected at or above the value that a
    // fraction want / len of the row's values reach.  Such a threshold need
    // not bound the k-th largest from below: the candidates are then checked
    // to number at least k, and the row goes to the whole-row path otherwise.
    int spec_rank = 0;
    if (!WAVE && topk && a.S == 1 && len > UE) {
      const int64_t want = min(2LL * k, (int64_t)a.ccap * 7 / 8);  // passing elements aimed at
      const double miss = 1.0 - (double)want / (double)len;     // of one value
      double all = 1.0;                                          // of the NE values of a thread
  #pragma unroll
      for (int e = 0; e < NE; ++e) all *= miss;
      const int r = (int)((1.0 - all) * NT + 0.5);
      spec_rank = (want < k || r < 1) ? 0 : min(r, NT);
    }
    bool spec_used = false;
#ifdef NLS_PHASE_STAMPS
    uint64_t st_refresh_ticks = 0;  // time inside block-path refreshes
    int st_refreshes = 0;
    uint64_t st_tiles = 0;
    uint64_t st_data_ticks = 0;  // waiting for a unit's data (and issuing the next)
    uint64_t st_bar_ticks = 0;   // at the block path's tile barrier
#endif
    // wave path (k <= 64): this wave's buffer count, threshold and overflow
    int wn = 0;
    uint32_t wtau = 0u;
    bool wovf = false;
    int nu = 0;  // wave path: units this wave has processed after its first

    // t: the unit; first: the first unit of every thread (tile 0 of the row)
    auto process = [&](float (&v)[NE], int t, bool first) __attribute__((always_inline)) {
      const int toff = t * UE;
      const bool full = toff + UE <= len;  // no element of the unit lies past the slice
      // This thread's first element of the unit, made opaque so that the
      // per-element offsets below are formed here, not hoisted out of the
      // loop into one register each.
      int obase = toff + uth * 4;
      asm volatile("" : "+v"(obase));
      // With 16-byte loads len % 4 == 0, so a float4 group is wholly in or out.
      auto loc_of = [&](int q) -> int { return obase + (q >> 2) * GS + (q & 3); };
      auto valid = [&](int q) -> bool {
        const int o = obase + (q >> 2) * GS;
        return full || (VEC ? o < len : o + (q & 3) < len);
      };
      if (greedy) {
        // argmax (:45-49): only a lane whose tile maximum beats its running
        // best walks the tile in index order (strict >, so the first index wins)
        float tmx = -__builtin_inff();
  #pragma unroll
        for (int q = 0; q < NE; ++q)
          if (valid(q) && v[q] > tmx) tmx = v[q];
        // (nothing chosen yet: equal values still pick the first index, so a
        // row of -inf answers its first id)
        if (first && tid == 0) x0raw = v[0];
        if (tmx > bv || (tmx == bv && bi == 0x7fffffff)) {
  #pragma unroll
          for (int q = 0; q < NE; ++q)
            if (valid(q)) {
              if (patched(loc_of(q)))
                capture(loc_of(q), v[q]);
              else
                argmax_merge(bv, bi, v[q], lo + loc_of(q));
            }
        }
        return;
      }
      // temperature (:80-81); v keeps the original logits for the patched ids
      // met on the way
      float sv[NE];
      {
        const float invT = P.invT;
  #pragma unroll
        for (int q = 0; q < NE; ++q) sv[q] = v[q] * invT;
      }
      auto gid = [&](int q) -> uint32_t { return (uint32_t)(lo + loc_of(q)); };
      if constexpr (WAVE) {
        // ---- wave path: this wave's own buffer, no barrier ----
        // Prefilter in the float domain: key(v) >= t implies !(v < key2f(t))
        // (NaN passes too), so keys are formed only where some lane passes.
        uint64_t* wb = cand + (size_t)wv * kWaveCap;
        uint32_t* whist = shist + wv * kWaveBins;
        if (!first && nu++ == kMidUnits - 1) {
          // After its first kMidUnits units every wave offers the M largest
          // keys of its buffer (distinct elements at or above the threshold),
          // and the last to do so takes the k-th largest of all NW * M offers:
          // a bound from NW * kMidUnits units rather than the first tile,
          // published through s_tau.  (An offer not yet written reads 0, which
          // only lowers the bound.)
          uint32_t kr[PER];
  #pragma unroll
          for (int j = 0; j < PER; ++j) {
            const int i = lane + j * kWave;
            kr[j] = i < wn ? (uint32_t)(wb[i] >> 32) : 0u;
          }
  #pragma unroll
          for (int i = 0; i < M0; ++i) {
            uint32_t lm = 0u;
  #pragma unroll
            for (int j = 0; j < PER; ++j) lm = max(lm, kr[j]);
            const uint32_t m = wave_max_u32(lm);
            const uint64_t at = __ballot(lm == m);
            if (lane == __ffsll((unsigned long long)at) - 1) {
              bool done = false;
  #pragma unroll
              for (int j = 0; j < PER; ++j)
                if (!done && kr[j] == m) {
                  kr[j] = 0u;
                  done = true;
                }
            }
            if (lane == 0) s_mid[wv * M0 + i] = m;
          }
          int prev = 0;
          if (lane == 0) prev = atomicAdd(&s_midn, 1);
          if (__builtin_amdgcn_readfirstlane(prev) == NW - 1) {
            const uint32_t t = wave_kth_largest(lane < NW * M0 ? s_mid[lane] : 0u, k);
            wtau = max(wtau, t);
            if (lane == 0) atomicMax(&s_tau, t);
          }
        }
        if (first) {
          // Block-wide start: every wave puts the M largest of its lanes'
          // maxima (distinct elements) into LDS, and the k-th largest of those
          // NW * M >= k real elements bounds the row's k-th largest from below.
          constexpr int M = (kWave + NW - 1) / NW;
          uint32_t lmax = 0u;  // 0: no unpatched value in this lane
          // (every lane reads a bitmap word, clamped into the slice, so that no
          // branch surrounds the LDS reads; the patch bits of each float4 group
          // sit in one word)
          uint32_t pbits[NV4];
  #pragma unroll
          for (int j = 0; j < NV4; ++j) {
            const int o = obase + j * GS;
            pbits[j] = bitmap[min(o, len - 1) >> 5] >> (o & 31);
          }
          // (the maximum is taken on the floats and keyed once: v_max_f32
          // returns one of its operands, so the lane's maximum is one of its
          // own unpatched elements whatever NaNs or signed zeros it meets)
          float fmx = -__builtin_inff();
  #pragma unroll
          for (int j = 0; j < NV4; ++j) {
            const uint32_t pb = has_patch ? pbits[j] : 0u;
  #pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int q = 4 * j + e;
              const bool ok = valid(q) & !((pb >> e) & 1u);
              fmx = __builtin_fmaxf(fmx, ok ? sv[q] : -__builtin_inff());
            }
          }
          lmax = fmx == -__builtin_inff() ? 0u : f2key(fmx);
  #pragma unroll
          for (int i = 0; i < M; ++i) {
            const uint32_t m = wave_max_u32(lmax);
            const uint64_t at = __ballot(lmax == m);
            if (lane == __ffsll((unsigned long long)at) - 1) lmax = 0u;
            if (lane == 0) s_top[wv * M + i] = m;
          }
          __syncthreads();
          // every wave takes the k-th largest of the NW * M maxima itself (key 0,
          // fewer than k real values, leaves no bound)
          wtau = wave_kth_largest(lane < NW * M ? s_top[lane] : 0u, k);
        }
        // any wave's threshold is a lower bound of the k-th largest of the row
        wtau = max(wtau, __hip_atomic_load(&s_tau, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
        float thr_f = key2f(wtau);
        int npf = 0;  // prefilter passes of this tile, over the wave
  #pragma unroll
        for (int q = 0; q < NE; ++q) npf += __popcll(__ballot(valid(q) && !(sv[q] < thr_f)));
        if (npf == 0) return;
        if (wn + npf > kWaveCap) {
          // Raise the threshold to a lower bound of the k-th largest of all this
          // wave has seen (buffer + tile): the k-th largest of the per-lane top-2.
          uint32_t tops[2] = {0u, 0u};
          int nm = 0;
  #pragma unroll
          for (int j = 0; j < PER; ++j) {
            const int i = lane + j * kWave;
            if (i < wn) {
              topq_insert<2>(tops, (uint32_t)(wb[i] >> 32));
              ++nm;
            }
          }
  #pragma unroll
          for (int q = 0; q < NE; ++q) {
            if (valid(q) && !(sv[q] < thr_f) && !patched(loc_of(q))) {
              const uint32_t kq = f2key(sv[q]);
              if (kq >= wtau) {
                topq_insert<2>(tops, kq);
                ++nm;
              }
            }
          }
          const int nv = min(nm, 2);
          int tv;
          (void)wave_excl_sum_small<2>(nv, tv);
          if (tv >= k) {
            wtau = wave_select(
                       [&](auto fn) {
  #pragma unroll
                         for (int q = 0; q < 2; ++q) fn(tops[q], q < nv);
                       },
                       k, k + k / 2, whist)
                       .tau;
            thr_f = key2f(wtau);
          }
          // compact the buffer to the new threshold
          uint64_t xs[PER];
          int keep = 0;
  #pragma unroll
          for (int j = 0; j < PER; ++j) {
            const int i = lane + j * kWave;
            xs[j] = (i < wn) ? wb[i] : 0ull;
            keep += (i < wn && (uint32_t)(xs[j] >> 32) >= wtau);
          }
          int ktot;
          int pos = wave_excl_sum_small<3>(keep, ktot);  // keep <= PER = 4
  #pragma unroll
          for (int j = 0; j < PER; ++j) {
            const int i = lane + j * kWave;
            if (i < wn && (uint32_t)(xs[j] >> 32) >= wtau) wb[pos++] = xs[j];
          }
          wn = ktot;
          npf = 0;
  #pragma unroll
          for (int q = 0; q < NE; ++q) npf += __popcll(__ballot(valid(q) && !(sv[q] < thr_f)));
          if (wn + npf > kWaveCap) {
            wovf = true;  // ties or an adversarial order crowd the buffer
            return;
          }
        }
        // append every unpatched value >= the threshold (each passes the prefilter)
  #pragma unroll
        for (int q = 0; q < NE; ++q) {
          if (__ballot(valid(q) && !(sv[q] < thr_f)) == 0ull) continue;
          const uint32_t kq = f2key(sv[q]);
          const bool pass = valid(q) && kq >= wtau;
          const bool pat = pass && patched(loc_of(q));
          if (pat) capture(loc_of(q), v[q]);
          const bool keep = pass && !pat;
          const uint64_t m = __ballot(keep);
          if (keep) wb[wn + (int)__popcll(m & lanes_below())] = ((uint64_t)kq << 32) | gid(q);
          wn += (int)__popcll(m);
        }
        if (wn >= 2 * k + kWave) {
          // tighten: the k-th largest of the buffer (which holds every value >=
          // the old threshold) is a lower bound of the k-th largest of the row
          uint64_t xs[PER];
  #pragma unroll
          for (int j = 0; j < PER; ++j) {
            const int i = lane + j * kWave;
            xs[j] = (i < wn) ? wb[i] : 0ull;
          }
          const int n0 = wn;
          const SelectResult r = wave_select(
              [&](auto fn) {
  #pragma unroll
                for (int j = 0; j < PER; ++j) fn((uint32_t)(xs[j] >> 32), lane + j * kWave < n0);
              },
              k, k + k / 4, whist);
          int keep = 0;
  #pragma unroll
          for (int j = 0; j < PER; ++j) keep += (lane + j * kWave < n0 && (uint32_t)(xs[j] >> 32) >= r.tau);
          int ktot;
          int pos = wave_excl_sum_small<3>(keep, ktot);
  #pragma unroll
          for (int j = 0; j < PER; ++j)
            if (lane + j * kWave < n0 && (uint32_t)(xs[j] >> 32) >= r.tau) wb[pos++] = xs[j];
          wn = ktot;
          wtau = r.tau;
          if (lane == 0) atomicMax(&s_tau, wtau);
        }
        return;
      } else {
        // ---- block path (k > 64): one buffer, a barrier per tile ----
        auto use = [&](int q) -> bool { return valid(q) && !patched(loc_of(q)); };
        uint32_t key[NE];
  #pragma unroll
        for (int q = 0; q < NE; ++q) key[q] = f2key(sv[q]);
  #pragma unroll
        for (int q = 0; q < NE; ++q)
          if (valid(q) && key[q] >= tau && patched(loc_of(q))) capture(loc_of(q), v[q]);
        int mine = 0;
  #pragma unroll
        for (int q = 0; q < NE; ++q) mine += (use(q) && key[q] >= tau);
        int wtot;
        const int wex = wave_excl_sum_small<5>(mine, wtot);  // mine <= NE = 16
        const int slot = t % 3;
        int wbase = 0;
        if (lane == 0 && wtot) wbase = atomicAdd(&s_tile_cnt[slot], wtot);
        wbase = __shfl(wbase, 0, kWave);
#ifdef NLS_PHASE_STAMPS
        const uint64_t st_b0 = __builtin_amdgcn_s_memrealtime();
        __syncthreads();
        st_bar_ticks += __builtin_amdgcn_s_memrealtime() - st_b0;
#else
        __syncthreads();
#endif
        const int ttot = s_tile_cnt[slot];
        if (tid == 0) s_tile_cnt[(t + 2) % 3] = 0;
        uint64_t* cb = cand + (size_t)cur * a.ccap;
        if (buf_n + ttot <= a.ccap) {
          int pos = buf_n + wbase + wex;
  #pragma unroll
          for (int q = 0; q < NE; ++q)
            if (use(q) && key[q] >= tau) cb[pos++] = ((uint64_t)key[q] << 32) | gid(q);
          buf_n += ttot;
          return;
        }
        // threshold refresh (uniform): raise tau, compact into the other buffer
#ifdef NLS_PHASE_STAMPS
        const uint64_t st_r0 = __builtin_amdgcn_s_memrealtime();
        ++st_refreshes;
#endif
        uint64_t* nb = cand + (size_t)(cur ^ 1) * a.ccap;
        auto count_ge = [&](uint32_t th) -> int {
          int c = 0;
          for (int i = tid; i < buf_n; i += NT) c += ((uint32_t)(cb[i] >> 32) >= th);
  #pragma unroll
          for (int q = 0; q < NE; ++q) c += (use(q) && key[q] >= th);
          return block_sum<NT>(c, smem);
        };
        uint32_t t1 = tau;
        int cnt = buf_n + ttot;
        if (spec_rank > 0) {
          // the speculative threshold (above): one maximum per thread, a thread
          // with no usable value offering the lowest key
          uint32_t mx = 0u;
  #pragma unroll
          for (int q = 0; q < NE; ++q) mx = (use(q) && key[q] > mx) ? key[q] : mx;
          if (buf_n == 0 && a.ccap >= 2048) {
            // (both buffers are empty: they hold the two histograms)
            t1 = block_rank24<NT>(mx, spec_rank, reinterpret_cast<uint32_t*>(cand),
                                  reinterpret_cast<uint32_t*>(cand + a.ccap), smem);
            cnt = -1;  // counted by the compaction below
          } else {
            t1 = block_select<NT>([&](auto fn) { fn(mx, true); }, spec_rank, -1, shist, smem).tau;
            cnt = count_ge(t1);
          }
          spec_used = true;
        } else {
          uint32_t tops[Q];
  #pragma unroll
          for (int q = 0; q < Q; ++q) tops[q] = 0u;
          int nmine = 0;
          for (int i = tid; i < buf_n; i += NT) {
            topq_insert<Q>(tops, (uint32_t)(cb[i] >> 32));
            ++nmine;
          }
  #pragma unroll
          for (int q = 0; q < NE; ++q) {
            if (use(q) && key[q] >= tau) {
              topq_insert<Q>(tops, key[q]);
              ++nmine;
            }
          }
          const int nv = min(nmine, Q);
          const int tv = block_sum<NT>(nv, smem);
          // t1 <= the k-th largest of the per-thread tops (k real elements), so
          // t1 is a lower bound of the k-th largest of everything seen.  A
          // coarse digit prefix is enough while it admits few elements;
          // otherwise refine to the exact k-th largest of the tops.
          auto tops_select = [&](int rank, int fit) -> uint32_t {
            return block_select<NT>(
                       [&](auto fn) {
  #pragma unroll
                         for (int q = 0; q < Q; ++q) fn(tops[q], q < nv);
                       },
                       rank, fit, shist, smem)
                .tau;
          };
          if (tv >= k) {
            t1 = tops_select(k, 2 * k);
            cnt = count_ge(t1);
            if (cnt > a.ccap / 2) {
              t1 = tops_select(k, -1);
              cnt = count_ge(t1);
            }
          }
        }
        spec_rank = 0;
        if (cnt > a.ccap) {
          // only ties at t1, or values crowded into few threads, get here: the
          // whole-row kernel takes the row
          ovf = true;
          return;
        }
        int c1 = 0;
        for (int i = tid; i < buf_n; i += NT) c1 += ((uint32_t)(cb[i] >> 32) >= t1);
  #pragma unroll
        for (int q = 0; q < NE; ++q) c1 += (use(q) && key[q] >= t1);
        int tot;
        int pos = block_excl_scan<NT>(c1, smem, tot);
        if (tot > a.ccap) {  // (uniform; a count left to this scan)
          ovf = true;
          return;
        }
        for (int i = tid; i < buf_n; i += NT) {
          const uint64_t x = cb[i];
          if ((uint32_t)(x >> 32) >= t1) nb[pos++] = x;
        }
  #pragma unroll
        for (int q = 0; q < NE; ++q)
          if (use(q) && key[q] >= t1) nb[pos++] = ((uint64_t)key[q] << 32) | gid(q);
        __syncthreads();
#ifdef NLS_PHASE_STAMPS
        st_refresh_ticks += __builtin_amdgcn_s_memrealtime() - st_r0;
#endif
        cur ^= 1;
        buf_n = tot;
        tau = t1;
      }
    };

    if (!ovf) {
      // One unit is in flight while the previous one is processed: as each
      // float4 group of unit t lands it is copied out and the same group of the
      // next unit is requested into its registers, so the memory queue stays
      // full.  (A workgroup can keep about one tile of requests outstanding;
      // more only stalls the issuing wave.)  The requests are unconditional
      // (past the slice they return zeros without reading memory) and the loop
      // runs on wave-uniform conditions, so the compiler's waits follow the
      // request order exactly.  ovf and wovf agree over the wave; the scalar
      // read makes that visible.
      auto stop = [&]() -> bool { return __builtin_amdgcn_readfirstlane((int)(ovf || wovf)) != 0; };
      const int nunits = (len + UE - 1) / UE;
      int t = u0;
      for (bool first = true;; first = false) {
        int tn = t + 1;
        if constexpr (WAVE) {
          // the next chunk for this wave: the second is fixed (NW + wv), the
          // later ones are claimed
          if (first) {
            tn = NW + wv;
          } else {
            int c = 0;
            if (lane == 0) c = atomicAdd(&s_next, 1);
            tn = __builtin_amdgcn_readfirstlane(c);
          }
        }
        float v[NE];
#ifdef NLS_PHASE_STAMPS
        const uint64_t st_d0 = __builtin_amdgcn_s_memrealtime();
#endif
  #pragma unroll
        for (int j = 0; j < NV4; ++j) {
          v[4 * j + 0] = R0[j].x;
          v[4 * j + 1] = R0[j].y;
          v[4 * j + 2] = R0[j].z;
          v[4 * j + 3] = R0[j].w;
          R0[j] = load_group<GS, VEC>(rs, tn * UE, j, uth);
        }
#ifdef NLS_PHASE_STAMPS
        asm volatile("" ::"v"(v[NE - 1]));
        st_data_ticks += __builtin_amdgcn_s_memrealtime() - st_d0;
#endif
        process(v, t, first);
#ifdef NLS_PHASE_STAMPS
        ++st_tiles;
#endif
        if (stop() || tn >= nunits) break;
        t = tn;
      }
    }
    if (wv == 0) NLS_STAMP(row, 2);
#ifdef NLS_PHASE_STAMPS
    if (wv == 0) {
      NLS_STAMP_VALUE(row, 13, st_refreshes);
      NLS_STAMP_VALUE(row, 14, st_refresh_ticks);
      NLS_STAMP_VALUE(row, 15, st_tiles);
      NLS_STAMP_VALUE(row, 7, st_data_ticks);
      NLS_STAMP_VALUE(row, 11, st_bar_ticks);
    }
#endif
    // The final value of patched slot p from its original logit: penalties then
    // bias (:71-76), then temperature (:80-81) on the sampling rows.
    auto patched_final = [&](int p, float v, uint32_t fl) -> float {
      const uint32_t cnt = fl >> kPatchCountShift;
      if (cnt) {
        if (P.rp_active) v = (v > 0.0f) ? (v / P.rp32) : (v * P.rp32);
        v = v - (float)((double)cnt * P.freq + P.pres);  // float64, one rounding (:74)
      }
      if (fl & kPatchBias) v = v + pbias[p];
      if (!greedy) v = v * P.invT;
      return v;
    };
    // original logit of slot p for the final pass (met during the stream,
    // requested before it, or read now)
    // (the late read goes through the slice's buffer resource, so that the
    // compiler cannot merge it with the LDS read into one generic-address load)
    auto patched_raw = [&](int p, uint32_t fl) -> float {
      const int r = (p - tid) / NT;
      if (fl & kPatchSeen) return pfin[p];
      if (r < RPT) return r == 0 ? rraw[0] : rraw[1];
      return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, (pid[p] - lo) * 4, 0, 0));
    };

    uint64_t* ent;
    int N;
    // Top-k rows of the wave path on one slice: the candidates are narrowed
    // before any select.  Every wave offers its M largest buffer keys (64
    // distinct real elements in all); the k-th largest of those bounds the
    // row's k-th largest from below, and typically leaves few more than k
    // entries above it.  With at most 128 survivors and no excess ties at the
    // k-th value one wave finishes the row alone.
    const bool wave_flow = WAVE && topk && a.S == 1;
    if (wave_flow) {
      constexpr int M = (kWave + NW - 1) / NW;
      uint64_t* wb = cand + (size_t)wv * kWaveCap;
      uint64_t xs[PER];
      uint32_t ks[PER];
  #pragma unroll
      for (int j = 0; j < PER; ++j) {
        const int i = lane + j * kWave;
        xs[j] = (!wovf && i < wn) ? wb[i] : 0ull;
        ks[j] = (uint32_t)(xs[j] >> 32);
      }
      {
        uint32_t kr[PER];
  #pragma unroll
        for (int j = 0; j < PER; ++j) kr[j] = ks[j];
  #pragma unroll
        for (int i = 0; i < M; ++i) {
          uint32_t lm = 0u;
  #pragma unroll
          for (int j = 0; j < PER; ++j) lm = max(lm, kr[j]);
          const uint32_t m = wave_max_u32(lm);
          const uint64_t at = __ballot(lm == m);
          if (lane == __ffsll((unsigned long long)at) - 1) {
            bool done = false;
  #pragma unroll
            for (int j = 0; j < PER; ++j)
              if (!done && kr[j] == m) {
                kr[j] = 0u;
                done = true;
              }
          }
          if (lane == 0) s_top[wv * M + i] = m;
        }
      }
      if (lane == 0) {
        s_wn[wv] = wovf ? -1 : wn;
        s_wt[wv] = wtau;
      }
      __syncthreads();  // every wave's stream, captures and offers are in
      // lane w reads wave w's record
      ovf = ovf || __ballot(lane < NW && s_wn[min(lane, NW - 1)] < 0) != 0ull;
      ent = cand + a.ccap;  // free: holds NW * kWaveCap entries and more
      // One wave computes what every wave needs next (the scalar unit and the
      // SIMDs are shared: sixteen waves computing the same bound take longer
      // than one); the others wait at the barrier.
      const bool lead = __builtin_amdgcn_readfirstlane(wv) == 0;
      if (!ovf) {  // uniform
        if (lead) {
          const uint32_t tau_all = wave_max_u32(lane < NW ? s_wt[min(lane, NW - 1)] : 0u);
          const uint32_t t = max(tau_all, wave_kth_largest(lane < NW * M ? s_top[lane] : 0u, k));
          if (lane == 0) s_te = t;
        }
        __syncthreads();
        const uint32_t te = __builtin_amdgcn_readfirstlane(s_te);
        // this wave's entries >= te
        int c = 0;
  #pragma unroll
        for (int j = 0; j < PER; ++j) c += __popcll(__ballot(ks[j] >= te && ks[j] != 0u));
        int base = 0;
        if (lane == 0 && c) base = atomicAdd(&s_cnt, c);
        base = __builtin_amdgcn_readfirstlane(base);
  #pragma unroll
        for (int j = 0; j < PER; ++j) {
          const bool keep = ks[j] >= te && ks[j] != 0u;
          const uint64_t mk = __ballot(keep);
          if (keep) ent[base + (int)__popcll(mk & lanes_below())] = xs[j];
          base += (int)__popcll(mk);
        }
        // patched ids: final values, those >= te join
        for (int p = tid; p < npatch; p += NT) {
          const uint32_t fl = pflag[p];
          if (!(fl & kPatchSeen) && !may_rise(fl)) continue;
          const float v = patched_final(p, patched_raw(p, fl), fl);
          const uint32_t kp = f2key(v);
          if (kp >= te) {
            const int i = atomicAdd(&s_cnt, 1);
            if (i < a.ccap) ent[i] = ((uint64_t)kp << 32) | (uint32_t)pid[p];
          }
        }
      }
      __syncthreads();
      N = s_cnt;
      if (!ovf && N > a.ccap) ovf = true;  // uniform
      if (ovf) {
        if (tid == 0) pushed = push_generic(a.generic_list, a.generic_count, row);
        return;
      }
      if (N >= k && N <= 2 * kWave) {
        // the lead wave finds the k-th largest key T of the survivors
        uint64_t e0 = 0ull, e1 = 0ull;
        uint32_t k0 = 0u, k1 = 0u, T = 0u;
        if (lead) {
          e0 = lane < N ? ent[lane] : 0ull;
          e1 = lane + kWave < N ? ent[lane + kWave] : 0ull;
          k0 = (uint32_t)(e0 >> 32);
          k1 = (uint32_t)(e1 >> 32);
          if (N <= kWave) {
            T = wave_kth_largest(k0, k);
          } else {
  #pragma unroll
            for (int b = 31; b >= 0; --b) {
              const uint32_t c = T | (1u << b);
              if (__popcll(__ballot(k0 >= c)) + __popcll(__ballot(k1 >= c)) >= k) T = c;
            }
          }
          const int ge = __popcll(__ballot(lane < N && k0 >= T)) + __popcll(__ballot(lane + kWave < N && k1 >= T));
          if (lane == 0) s_te = (ge == k) ? 1u : 0u;
        }
        __syncthreads();
        if (__builtin_amdgcn_readfirstlane(s_te) != 0u) {
          // no excess ties at T: the members are exactly the survivors >= T
          if (!lead) return;
          uint64_t* mem = reinterpret_cast<uint64_t*>(regA);
          const bool in0 = lane < N && k0 >= T, in1 = lane + kWave < N && k1 >= T;
          const uint64_t m0 = __ballot(in0), m1 = __ballot(in1);
          if (in0) mem[__popcll(m0 & lanes_below())] = e0;
          if (in1) mem[__popcll(m0) + __popcll(m1 & lanes_below())] = e1;
          double u = 0.0;
          if (lane == 0) u = take_uniform(a.d_u, u_in, st0, st1, a.rng, row);
          wave_tail(mem, k, P, u, row, a.out, a.dbg);
          return;
        }
      }
      // many survivors or excess ties: the block-wide member selection
      __syncthreads();
      if (tid == 0) s_cnt = 0;
    } else {
      // Ids that can be members were met during the stream; only the ids whose
      // patch may raise them are read again here.  The others are left out
      // (flag kPatchSeen clear).
      if (!ovf && npatch > 0) {
        __syncthreads();  // every wave's captures are in
        for (int p = tid; p < npatch; p += NT) {
          uint32_t fl = pflag[p];
          const uint32_t cnt = fl >> kPatchCountShift;
          if (!(fl & kPatchSeen) && !may_rise(fl)) continue;
          float v = patched_raw(p, fl);
          if (cnt) {
            if (P.rp_active) v = (v > 0.0f) ? (v / P.rp32) : (v * P.rp32);
            v = v - (float)((double)cnt * P.freq + P.pres);  // float64, one rounding (:74)
          }
          if (fl & kPatchBias) v = v + pbias[p];
          if (!greedy) v = v * P.invT;
          pfin[p] = v;
          if (!(fl & kPatchSeen)) pflag[p] = fl | kPatchSeen;
        }
        __syncthreads();
      }

      // ---- the slice's candidates: stream buffer(s) + patched values ----
      ent = cand + (size_t)cur * a.ccap;
      N = buf_n;
      if (topk) {
        uint32_t tau_all = tau;  // a lower bound of the row's k-th largest, uniform
        if constexpr (WAVE) {
          // concatenate the wave buffers into the second buffer
          if (lane == 0) {
            s_wn[wv] = wovf ? -1 : wn;
            s_wt[wv] = wtau;
          }
          __syncthreads();
          int off = 0;
          N = 0;
          tau_all = 0u;
          for (int w = 0; w < NW; ++w) {
            const int nw_ = s_wn[w];
            tau_all = max(tau_all, s_wt[w]);
            if (nw_ < 0) {
              ovf = true;
            } else {
              if (w == wv) off = N;
              N += nw_;
            }
          }
          ent = cand + a.ccap;
          if (!ovf) {
            const uint64_t* wb = cand + (size_t)wv * kWaveCap;
            for (int i = lane; i < wn; i += kWave) ent[off + i] = wb[i];
          }
          __syncthreads();
        }
        if (!ovf && npatch > 0) {
          // patched values >= tau_all join the candidates
          if (tid == 0) s_cnt = N;
          __syncthreads();
          for (int p = tid; p < npatch; p += NT) {
            if (!(pflag[p] & kPatchSeen)) continue;
            const uint32_t kp = f2key(pfin[p]);
            if (kp >= tau_all) {
              const int i = atomicAdd(&s_cnt, 1);
              if (i < a.ccap) ent[i] = ((uint64_t)kp << 32) | (uint32_t)pid[p];
            }
          }
          __syncthreads();
          N = s_cnt;
          if (N > a.ccap) ovf = true;  // uniform
          __syncthreads();
          if (tid == 0) s_cnt = 0;
        }
      } else {
        // greedy: patched final values join the argmax
        for (int p = tid; p < npatch; p += NT)
          if (pflag[p] & kPatchSeen) argmax_merge(bv, bi, pfin[p], pid[p]);
      }
      // argmax (:45-49) starts from index 0: when its value is NaN nothing
      // compares greater and the answer stays 0
      bool nan0 = false;
      if (greedy && lo == 0 && len > 0 && tid == 0) {
        float x0 = x0raw;
        if (patched(0)) x0 = pfin[wpre[0] + 0];
        nan0 = x0 != x0;
      }

      // ---- slice argmax (first index on ties) ----
      wave_argmax(bv, bi);
      if (lane == 0) {
        s_rv[wv] = bv;
        s_ri[wv] = bi;
      }
      __syncthreads();
      float rv = s_rv[0];
      int ri = s_ri[0];
    #pragma unroll
      for (int w = 1; w < NW; ++w) argmax_merge(rv, ri, s_rv[w], s_ri[w]);

      if (a.S > 1) {
        // ---- publish this slice; the last one to arrive completes the row ----
        const int64_t part = (int64_t)row * a.S + sl;
        uint64_t* pdst = a.part_cand + part * a.pc;
        int nout = 0;
        int flags = (ovf ? kSliceOverflow : 0) | (nan0 ? kSliceNan0 : 0);
        if (topk && !ovf) {
          if (N > a.pc) {
            const SelectResult r = block_select<NT>(
                [&](auto fn) {
                  for (int i0 = 0; i0 < N; i0 += NT) {
                    const int i = i0 + tid;
                    const bool in = i < N;
                    fn(in ? (uint32_t)(ent[i] >> 32) : 0u, in);
                  }
                },
                k, a.pc, shist, smem);
            if (r.ge > a.pc) {
              flags = kSliceOverflow;
            } else {
              int mine = 0;
              for (int i = tid; i < N; i += NT) mine += ((uint32_t)(ent[i] >> 32) >= r.tau);
              int tot;
              int pos = block_excl_scan<NT>(mine, smem, tot);
              for (int i = tid; i < N; i += NT)
                if ((uint32_t)(ent[i] >> 32) >= r.tau) store_agent(&pdst[pos++], ent[i]);
              nout = tot;
            }
          } else {
            for (int i = tid; i < N; i += NT) store_agent(&pdst[i], ent[i]);
            nout = N;
          }
        }
        if (tid == 0) {
          store_agent(&a.part_info[part].n, nout);
          store_agent(&a.part_info[part].flags, flags);
          store_agent(&a.part_info[part].amax, ri);
          store_agent(&a.part_info[part].vmax, __float_as_int(rv));
        }
        // Release/acquire at agent scope: every thread's slice stores happen
        // before the barrier, and so before thread 0's acquire-release increment
        // of the arrival count.  The slice that completes the count has
        // acquired every other slice's release, and its other threads follow
        // thread 0 through the barrier.
        __syncthreads();
        if (tid == 0)
          s_last = (__hip_atomic_fetch_add(&a.arrive[row], 1u, __ATOMIC_ACQ_REL,
                                           __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)(a.S - 1));
        __syncthreads();
        if (!s_last) return;
        if (tid == 0) __hip_atomic_store(&a.arrive[row], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // slice records: one per thread, then every thread reads them from LDS.
        // s_off borrows the select histogram (free here; 5 * kMaxSlices words < kSelWords).
        int* s_off = reinterpret_cast<int*>(shist);
        static_assert(5 * kMaxSlices <= kSelWords, "slice records must fit the histogram");
        if (tid < a.S) {
          const SliceInfo* in = a.part_info + (int64_t)row * a.S + tid;
          const int nj = load_agent(&in->n);
          const int fl = load_agent(&in->flags);
          s_off[kMaxSlices + tid] = (nj < 0 || nj > a.pc) ? -1 : nj;  // never trust a count past the buffer
          s_off[2 * kMaxSlices + tid] = fl;
          s_off[3 * kMaxSlices + tid] = load_agent(&in->amax);
          s_off[4 * kMaxSlices + tid] = load_agent(&in->vmax);
        }
        __syncthreads();
        int any = 0;
        N = 0;
        rv = -__builtin_inff();
        ri = 0x7fffffff;
        for (int j = 0; j < a.S; ++j) {
          const int nj = s_off[kMaxSlices + j];
          any |= s_off[2 * kMaxSlices + j] | (nj < 0 ? kSliceOverflow : 0);
          nan0 = nan0 || (s_off[2 * kMaxSlices + j] & kSliceNan0);
          argmax_merge(rv, ri, __int_as_float(s_off[4 * kMaxSlices + j]), s_off[3 * kMaxSlices + j]);
          s_off[j] = N;  // start of slice j in the merged buffer
          if (nj > 0) N += nj;
        }
        ovf = (any & kSliceOverflow) != 0;
        if (topk && !ovf) {
          ent = cand;  // both ping-pong buffers: 2 * ccap >= S * pc entries
          constexpr int MR = 8;  // loads in flight per thread
          for (int b0 = 0; b0 < N; b0 += NT * MR) {
            uint64_t xv[MR];
    #pragma unroll
            for (int r = 0; r < MR; ++r) {
              const int i = b0 + r * NT + tid;
              xv[r] = 0ull;
              if (i < N) {
                int j = 0;
                while (j + 1 < a.S && s_off[j + 1] <= i) ++j;
                xv[r] = load_agent(a.part_cand + ((int64_t)row * a.S + j) * a.pc + (i - s_off[j]));
              }
            }
    #pragma unroll
            for (int r = 0; r < MR; ++r) {
              const int i = b0 + r * NT + tid;
              if (i < N) ent[i] = xv[r];
            }
          }
        }
        __syncthreads();
        for (int q = tid; q < 5 * kMaxSlices; q += NT) s_off[q] = 0;  // restore the zeroed histogram
        __syncthreads();
      }
      if (ovf) {
        if (tid == 0) pushed = push_generic(a.generic_list, a.generic_count, row);
        return;
      }
      if (!topk) {
        if (tid == 0) {
          a.out[row] = nan0 ? 0 : ri;
          if (a.dbg.n) a.dbg.n[row] = 0;
          if (a.dbg.ncand) a.dbg.ncand[row] = 0;
          if (a.dbg.total) a.dbg.total[row] = 0.0f;
          if (a.dbg.path) a.dbg.path[row] = 1;
        }
        return;
      }
    }
    // ---- the row's heap-path members, then the reference's tail ----
    uint64_t* mem = reinterpret_cast<uint64_t*>(regA);
    if (wv == 0) NLS_STAMP(row, 3);
    NLS_STAMP_VALUE(row, 12, N);
    // (after a speculative threshold fewer than k elements may reach it)
    if ((spec_used && N < k) || !topk_members<NT>(ent, N, k, mem, a.mcap, shist, smem, &s_cnt)) {
      if (tid == 0) pushed = push_generic(a.generic_list, a.generic_count, row);
      return;
    }
    if (wv == 0) NLS_STAMP(row, 4);
    if (k <= kWave) {
      if (wv != 0) return;
      double u = 0.0;
      if (lane == 0) u = take_uniform(a.d_u, u_in, st0, st1, a.rng, row);
      wave_tail(mem, k, P, u, row, a.out, a.dbg);
      return;
    }
    // k > 64: block-wide sort of the members, then the block tail
    float* vals = reinterpret_cast<float*>(mem + a.mcap);
    int32_t* ids = reinterpret_cast<int32_t*>(vals + a.kcap);
    float* ebuf = reinterpret_cast<float*>(ids + a.kcap);
    const int kpow = next_pow2(k);
    for (int i = k + tid; i < kpow; i += NT) mem[i] = 0ull;
    __syncthreads();
    bitonic_sort_u64<NT>(mem, kpow, true);
    for (int i = tid; i < k; i += NT) {
      vals[i] = key2f((uint32_t)(mem[i] >> 32));
      ids[i] = (int32_t)(uint32_t)mem[i];
    }
    if (tid == 0) s_u = take_uniform(a.d_u, u_in, st0, st1, a.rng, row);
    __syncthreads();
    if (wv == 0) NLS_STAMP(row, 5);
    const TailOut to = softmax_cutoff_draw<NT, true>(vals, ids, ebuf, k, P, s_u, smem);
    if (wv == 0) NLS_STAMP(row, 6);
    if (tid == 0) a.out[row] = to.id;
    write_debug<NT>(a.dbg, row, 2 | to.nan_cand, to.n, k, to.total, ids, ebuf);
  };
  run();
  if (a.gen_inline) {
    // The last workgroup to finish serves the rows handed on to the
    // whole-row path (their pushes precede every count below).
    // Thread 0 listed this workgroup's rows (if any) itself, so a release
    // increment of `done` by it publishes them; workgroups that listed none
    // have nothing to publish and count relaxed (the release sequence of every
    // release increment runs on through the later ones).  Thread 0 of the last
    // workgroup acquires with a fence after its increment; the workgroup's
    // other threads follow it through the barrier.
    __syncthreads();
    if (threadIdx.x == 0) {
      const uint32_t prev =
          pushed ? __hip_atomic_fetch_add(a.done, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT)
                 : __hip_atomic_fetch_add(a.done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = prev == gridDim.x - 1;
      if (s_last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    }
    __syncthreads();
    if (s_last) {
      const int count = load_agent(a.ga.generic_count);
      __syncthreads();
      if (threadIdx.x == 0) {
        store_agent(a.done, 0u);
        store_agent(a.ga.next_count, 0);
      }
      uint32_t* dl = reinterpret_cast<uint32_t*>(lds);
      generic_rows<NT>(a.ga, 0, 1, count, shist, dl, dl + 256, smem, &s_u, reinterpret_cast<int*>(dl + 512),
                       s_rv, s_ri);
    }
  }
}

// ---------------------------------------------------------------------------
// 2. generic_kernel: whole-row stable radix sort, then the reference's tail
// ---------------------------------------------------------------------------
// Scratch per workgroup: keysA, idxA, keysB, idxB (uint32 each, vpad) and
// f32 work (vpad).  Keys are ~f2key(value): an ascending stable sort gives
// descending value with ascending index on ties (sampler.nim:97).
constexpr int kGenIPT = 8;

template <int NT>
__device__ __forceinline__ void radix_sort_pass(const uint32_t* __restrict__ kin, const uint32_t* __restrict__ iin,
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


// ---------------------------------------------------------------------------
// Grouped sort path: a full-sort row (sampler.nim:96-121) without the sort.
// The row's final values (penalties, bias and temperature applied, :64-81)
// are counted per distinct value in an LDS hash table, for every value whose
// exp(v - mx) can still move the softmax sum (fl(v - mx) >= kGroupFloor).
// The distinct values are sorted, and the reference's sequential fp32 chains
// -- softmax sum, top-p, total, draw -- run over them with each value's
// multiplicity (nls_grouped.h).  The drawn candidate is the t-th lowest index
// among the members of its value, as the stable sort orders equal values.
// Rows that need more (patched ids, distinct values or candidates past the
// table) report failure and take the whole-row sort.
// ---------------------------------------------------------------------------
struct GroupLds {
  uint32_t* bitmap;  // [nw] patched ids of the row
  uint32_t* wpre;    // [nw] patched ids before each bitmap word
  int32_t* pid;      // [kGrpPatchCap] patched ids, in index order
  uint32_t* pcnt;    //   their window counts
  int32_t* pbias;    //   their bias entries (-1: none)
  float* pfin;       //   their final values
  uint32_t* hkey;    // [kGrpHashCap] f2key of a distinct value (kGrpEmpty: free)
  uint32_t* hcnt;    //   its multiplicity
  uint64_t* gsort;   // [kGrpHashCap] (~f2key(value) << 32) | multiplicity (or kGrpOne | index), ascending
};
constexpr uint32_t kGrpEmpty = 0xffffffffu;  // f2key of a NaN, which never enters
// A group's multiplicity in the low word of its sort record; a value that
// occurs once carries its element's index instead (V < 2^31), flagged.
constexpr uint32_t kGrpOne = 0x80000000u;
__device__ __forceinline__ uint32_t group_count(uint64_t rec) {
  const uint32_t lo = (uint32_t)rec;
  return (lo & kGrpOne) ? 1u : lo;
}

__device__ __forceinline__ GroupLds group_lds(unsigned char* base, int nw) {
  GroupLds L;
  L.bitmap = reinterpret_cast<uint32_t*>(base);
  L.wpre = L.bitmap + nw;
  L.pid = reinterpret_cast<int32_t*>(L.wpre + nw);
  L.pcnt = reinterpret_cast<uint32_t*>(L.pid + kGrpPatchCap);
  L.pbias = reinterpret_cast<int32_t*>(L.pcnt + kGrpPatchCap);
  L.pfin = reinterpret_cast<float*>(L.pbias + kGrpPatchCap);
  L.hkey = reinterpret_cast<uint32_t*>(L.pfin + kGrpPatchCap);
  L.hcnt = L.hkey + kGrpHashCap;
  L.gsort = reinterpret_cast<uint64_t*>(L.hcnt + kGrpHashCap);  // byte offset 8*nw + 16*caps
  return L;
}
// Per hash slot: the index of the occurrence that inserted it (the sort
// array's first half, until the groups are collected; addressed from the
// count array, which it follows, so no other base stays live).
__device__ __forceinline__ int32_t* group_first(const GroupLds& L) {
  return reinterpret_cast<int32_t*>(L.hcnt + kGrpHashCap);
}

// Count one more occurrence of key, the element at index `idx`; false when
// the table is full.  The inserting occurrence's index is kept per slot (in
// the sort array, unused until the groups are collected): for a value that
// occurs once it is the value's only member.
__device__ __forceinline__ bool group_insert(const GroupLds& L, uint32_t key, int* distinct, int idx) {
  uint32_t h = (key * 0x9E3779B1u) >> (32 - kGrpHashBits);
  for (int probe = 0; probe < kGrpHashCap; ++probe) {
    uint32_t cur = L.hkey[h];
    if (cur == kGrpEmpty) {
      cur = atomicCAS(&L.hkey[h], kGrpEmpty, key);
      if (cur == kGrpEmpty) {
        cur = key;
        group_first(L)[h] = idx;
        if (atomicAdd(distinct, 1) >= kGrpHashLimit) return false;
      }
    }
    if (cur == key) {
      atomicAdd(&L.hcnt[h], 1u);
      return true;
    }
    h = (h + 1) & (kGrpHashCap - 1);
  }
  return false;
}

struct GroupOut {
  int ok;
  int id;
  int n;
  float total;
};

// STAGE 0: the whole grouped path.  STAGE 1 (the grouped launch): the same,
// except that with a.walk_split the row's groups are stored once sorted and
// the row is left for the walk launch (ok = 2).  STAGE 3 (the search launch):
// the patch table, then the search for the member a.p3_* names.
template <int NT, int STAGE = 0>
__device__ __forceinline__ GroupOut grouped_row(const GenericArgs& a, int row, const RowParams& P, double u,
                                const GroupLds& L, int* smem) {
  constexpr int NW = NT / kWave;
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int V = (int)a.V;
  const int nw = (V + 31) >> 5;
  const float* __restrict__ src = a.logits + (int64_t)row * a.V;
  __shared__ int s_fail, s_distinct, s_G, s_id, s_found;
  __shared__ int64_t s_left;
  __shared__ unsigned long long s_held;
  __shared__ uint32_t s_wmax[NW];
  __shared__ int s_wnan[NW];
  __shared__ float s_sum;
  __shared__ GroupDraw s_draw;
  __shared__ int s_g;
  __shared__ int64_t s_t;
  GroupOut res;
  res.ok = 0;
  res.id = 0;
  res.n = 0;
  res.total = 0.0f;

  if constexpr (STAGE != 3) NLS_GSTAMP(row, 0);
  if constexpr (STAGE == 3) NLS_GSTAMP(row, 9);
  for (int i = tid; i < nw; i += NT) L.bitmap[i] = 0u;
  if constexpr (STAGE != 3) {
    for (int i = tid; i < kGrpHashCap; i += NT) {
      L.hkey[i] = kGrpEmpty;
      L.hcnt[i] = 0u;
    }
  }
  for (int i = tid; i < kGrpPatchCap; i += NT) {
    L.pcnt[i] = 0u;
    L.pbias[i] = -1;
  }
  if (tid == 0) {
    s_fail = 0;
    s_distinct = 0;
    s_G = 0;
    s_id = -1;
    s_held = 0ull;
  }
  __syncthreads();
  // ---- patch table: the window's ids (:64-70) and the bias ids (:75-76) ----
  const int64_t hlen = a.hist_len[row];
  int n_hist = 0;
  if (P.pen_active && hlen > 0)
    n_hist = (int)((P.repeat_last_n > 0 && P.repeat_last_n < hlen) ? P.repeat_last_n : hlen);
  const int32_t* __restrict__ hrow = a.hist + (int64_t)row * a.hcap;
  const int hbase = n_hist > 0 ? (int)((hlen - n_hist) % a.hcap) : 0;
  auto hist_id = [&](int i) {
    int slot = hbase + i;
    if (slot >= a.hcap) slot -= a.hcap;
    return hrow[slot];
  };
  for (int i = tid; i < n_hist; i += NT) {
    const int id = hist_id(i);
    if (id >= 0 && id < V) atomicOr(&L.bitmap[id >> 5], 1u << (id & 31));
  }
  for (int j = tid; j < P.bias_cnt; j += NT) {
    const int id = a.bias_ids[P.bias_off + j];
    if (id >= 0 && id < V) atomicOr(&L.bitmap[id >> 5], 1u << (id & 31));
  }
  __syncthreads();
  const int per = (nw + NT - 1) / NT;
  const int wlo = tid * per;
  int pc = 0;
  for (int q = 0; q < per; ++q)
    if (wlo + q < nw) pc += __popc(L.bitmap[wlo + q]);
  int np;
  int run = block_excl_scan<NT>(pc, smem, np);
  if (np > kGrpPatchCap) return res;  // np is the same in every thread
  for (int q = 0; q < per; ++q)
    if (wlo + q < nw) {
      L.wpre[wlo + q] = (uint32_t)run;
      run += __popc(L.bitmap[wlo + q]);
    }
  __syncthreads();
  auto slot_of = [&](int id) {
    const int ww = id >> 5;
    return (int)L.wpre[ww] + __popc(L.bitmap[ww] & ((1u << (id & 31)) - 1u));
  };
  for (int i = tid; i < n_hist; i += NT) {
    const int id = hist_id(i);
    if (id >= 0 && id < V) {
      const int sl = slot_of(id);
      atomicAdd(&L.pcnt[sl], 1u);
      L.pid[sl] = id;
    }
  }
  for (int j = tid; j < P.bias_cnt; j += NT) {
    const int id = a.bias_ids[P.bias_off + j];
    if (id >= 0 && id < V) {
      const int sl = slot_of(id);
      L.pbias[sl] = j;
      L.pid[sl] = id;
    }
  }
  __syncthreads();
  for (int sl = tid; sl < np; sl += NT) {
    const int id = L.pid[sl];
    float v = src[id];
    const uint32_t c = L.pcnt[sl];
    if (c) {
      if (P.rp_active) v = (v > 0.0f) ? (v / P.rp32) : (v * P.rp32);
      v = v - (float)((double)c * P.freq + P.pres);
    }
    if (L.pbias[sl] >= 0) v = v + a.bias_vals[P.bias_off + L.pbias[sl]];
    L.pfin[sl] = v * P.invT;  // (:80-81)
  }
  __syncthreads();
  if constexpr (STAGE != 3) NLS_GSTAMP(row, 1);
  const bool vec = (V % 4 == 0) && ((reinterpret_cast<uintptr_t>(src) & 15) == 0);
  const float4* __restrict__ src4 = reinterpret_cast<const float4*>(src);
  const float invT = P.invT;
  const int V4 = V >> 2;
  // the drawn member: its group's value and count record, its rank among them
  float vg = 0.0f;
  int64_t t = 0;
  uint64_t grec = 0;
  if constexpr (STAGE == 3) {
    vg = key2f(a.p3_key[row]);
    grec = a.p3_rec[row];
    t = a.p3_t[row];
  } else {
  // ---- the row maximum (:53) and the values that can move the sum ----
  // Counting needs the maximum: a value counts when fl(v - mx) >= kGroupFloor.
  // One fused pass counts every value within kGroupFloor of a running
  // maximum instead (the workgroup's, shared through LDS after each step):
  // the running maximum never exceeds mx, so every occurrence of a needed
  // value is counted, and the values that fall below the final floor are
  // dropped afterwards.  A table that fills (a row whose running maximum
  // rose late over many distinct values) is counted again in two passes.
  // Eight values at a time (the kernel runs at its register limit): their
  // table slots are read together, a value already in the table at its first
  // slot is counted with one atomic add, and only the others (first
  // occurrences, collisions) probe.
  bool bad = false;
  auto count8 = [&](const float* vv, uint32_t want, auto&& ix) __attribute__((always_inline)) {
    if (__ballot(want != 0u) == 0ull) return;  // (uniform) nothing of the wave's within the floor
    uint32_t hs[8], cur[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) hs[q] = (f2key(vv[q]) * 0x9E3779B1u) >> (32 - kGrpHashBits);
#pragma unroll
    for (int q = 0; q < 8; ++q) cur[q] = L.hkey[hs[q]];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      if (!((want >> q) & 1u)) continue;
      const uint32_t key = f2key(vv[q]);
      if (cur[q] == key)
        atomicAdd(&L.hcnt[hs[q]], 1u);
      else
        bad |= !group_insert(L, key, &s_distinct, ix(q));
    }
  };
  // the row's final values 8 per thread at a time: fn(vv, in, ix) with in's
  // bit q set where vv[q] is an unpatched value of the row, whose index is
  // ix(q).  With 16-byte loads the next 8 are requested before these are
  // counted, so the counting runs while they are in flight (16 values in
  // registers, as many as a CU's request queue keeps in flight for the
  // workgroup).  The loops run the same number of times on every lane of a
  // wave (fn reduces over the wave) and stop when a lane has filled the
  // table.
  const int wbase = __builtin_amdgcn_readfirstlane(tid - lane);  // (uniform over the wave)
  // the lane's index, computed where it is used (the compiler cannot move it
  // earlier and keep it in a register)
  auto lane_here = []() __attribute__((always_inline)) {
    int l;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
    return l;
  };
  auto for_each8 = [&](auto&& fn) __attribute__((always_inline)) {
    if (vec) {
      float4 nx[2];
      auto request = [&](int w4) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < 2; ++u) nx[u] = src4[min(w4 + lane + u * NT, V4 - 1)];
      };
      if (wbase < V4) request(wbase);
      for (int w4 = wbase; w4 < V4; w4 += 2 * NT) {
        const float4 x[2] = {nx[0], nx[1]};
        if (w4 + 2 * NT < V4) request(w4 + 2 * NT);  // (uniform)
        float vv[8];
        uint32_t in = 0u;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int i4 = w4 + lane + u * NT;
          const uint32_t pb = i4 < V4 ? (L.bitmap[i4 >> 3] >> ((i4 & 7) * 4)) & 15u : 15u;
          vv[4 * u + 0] = x[u].x * invT;
          vv[4 * u + 1] = x[u].y * invT;
          vv[4 * u + 2] = x[u].z * invT;
          vv[4 * u + 3] = x[u].w * invT;
          in |= ((~pb) & 15u) << (4 * u);
        }
        // (the index is formed where a value is inserted, from the wave's
        // scalar base and the lane read there: nothing is held for it)
        fn(vv, in, [&](int q) { return 4 * (w4 + lane_here() + (q >> 2) * NT) + (q & 3); });
        if (__ballot(bad)) break;
      }
    } else {
      for (int w0 = wbase; w0 < V; w0 += 8 * NT) {
        const int b = w0 + lane;
        float vv[8];
        uint32_t in = 0u;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const int i = b + q * NT;
          vv[q] = i < V ? src[i] * invT : 0.0f;
          if (i < V && !((L.bitmap[i >> 5] >> (i & 31)) & 1u)) in |= 1u << q;
        }
        fn(vv, in, [&](int q) { return w0 + lane_here() + q * NT; });
        if (__ballot(bad)) break;
      }
    }
  };
  __shared__ uint32_t s_rkey;  // the workgroup's running maximum (key)
  if (tid == 0) s_rkey = f2key(-__builtin_inff());
  __syncthreads();
  bool nan = false;
  float rmx = -__builtin_inff();
  for (int sl = tid; sl < np; sl += NT) {
    const float v = L.pfin[sl];
    nan |= (v != v);
    rmx = __builtin_fmaxf(rmx, v);
  }
  if (rmx > -__builtin_inff()) atomicMax(&s_rkey, f2key(rmx));
  __syncthreads();
  rmx = key2f(s_rkey);
  for_each8([&](const float (&vv)[8], uint32_t in, auto&& ix) {
#pragma unroll
    for (int q = 0; q < 8; ++q)
      if ((in >> q) & 1u) {
        nan |= (vv[q] != vv[q]);
        rmx = __builtin_fmaxf(rmx, vv[q]);
      }
    // share the running maximum (the read may lag: any value up to mx is sound)
    const uint32_t wk = wave_max_u32(f2key(rmx));
    if (lane == 0) atomicMax(&s_rkey, wk);
    rmx = __builtin_fmaxf(rmx, key2f(s_rkey));
    uint32_t want = 0u;
#pragma unroll
    for (int q = 0; q < 8; ++q)
      if (((in >> q) & 1u) && vv[q] - rmx >= kGroupFloor) want |= 1u << q;
    count8(vv, want, ix);
  });
  for (int sl = tid; sl < np && !bad; sl += NT) {
    const float v = L.pfin[sl];
    if (v - rmx >= kGroupFloor) bad |= !group_insert(L, f2key(v), &s_distinct, L.pid[sl]);
  }
  // the row maximum: every thread's running maximum (NaN never taken)
  const uint64_t nb = __ballot(nan);
  const uint64_t bb = __ballot(bad);
  const uint32_t wk = wave_max_u32(f2key(rmx));
  if (lane == 0) {
    s_wmax[tid >> 6] = wk;
    s_wnan[tid >> 6] = (nb != 0ull ? 1 : 0) | (bb != 0ull ? 2 : 0);
  }
  __syncthreads();
  uint32_t mk = 0u;
  int flags = 0;
  for (int q = 0; q < NW; ++q) {
    mk = max(mk, s_wmax[q]);
    flags |= s_wnan[q];
  }
  const float mx = key2f(mk);
  NLS_GSTAMP(row, 2);
  if ((flags & 1) || !(mx > -__builtin_inff() && mx < __builtin_inff())) return res;
  if (flags & 2) {
    // the table filled: count again against the final maximum
    __syncthreads();
    for (int i = tid; i < kGrpHashCap; i += NT) {
      L.hkey[i] = kGrpEmpty;
      L.hcnt[i] = 0u;
    }
    if (tid == 0) s_distinct = 0;
    bad = false;
    __syncthreads();
    for_each8([&](const float (&vv)[8], uint32_t in, auto&& ix) {
      uint32_t want = 0u;
#pragma unroll
      for (int q = 0; q < 8; ++q)
        if (((in >> q) & 1u) && vv[q] - mx >= kGroupFloor) want |= 1u << q;
      count8(vv, want, ix);
    });
    for (int sl = tid; sl < np && !bad; sl += NT) {
      const float v = L.pfin[sl];
      if (v - mx >= kGroupFloor) bad |= !group_insert(L, f2key(v), &s_distinct, L.pid[sl]);
    }
    if (bad) s_fail = 1;
  }
  __syncthreads();
  NLS_GSTAMP(row, 3);
  if (s_fail) return res;
  // a value that occurs once: its index replaces the count (read before any
  // record is written over the inserting indices)
  for (int h = tid; h < kGrpHashCap; h += NT)
    if (L.hcnt[h] == 1u) L.hcnt[h] = kGrpOne | (uint32_t)group_first(L)[h];
  __syncthreads();
  for (int h = tid; h < kGrpHashCap; h += NT) {
    const uint32_t k = L.hkey[h];
    // (values counted against a running maximum that fall below the floor of
    // the final one are dropped)
    if (k != kGrpEmpty && key2f(k) - mx >= kGroupFloor) {
      const int at = atomicAdd(&s_G, 1);
      L.gsort[at] = ((uint64_t)(~k) << 32) | (uint64_t)L.hcnt[h];
    }
  }
  __syncthreads();
  const int G = s_G;
  const int Gp = next_pow2(G > 0 ? G : 1);
  for (int i = G + tid; i < Gp; i += NT) L.gsort[i] = ~0ull;
  __syncthreads();
  bitonic_sort_u64<NT>(L.gsort, Gp, false);  // descending value
  NLS_GSTAMP(row, 4);
  // per group: its exponential (:56) and multiplicity (hash arrays reused)
  float* ge = reinterpret_cast<float*>(L.hkey);
  uint32_t* gc = L.hcnt;
  for (int g = tid; g < G; g += NT) {
    const uint64_t e = L.gsort[g];
    const float v = key2f(~(uint32_t)(e >> 32));
    gc[g] = group_count(e);
    ge[g] = expf_cr(v - mx);
    atomicAdd(&s_held, (unsigned long long)group_count(e));
  }
  __syncthreads();
  if constexpr (STAGE == 1) {
    if (a.walk_split) {
      // the groups for the walk launch
      const size_t o = (size_t)row * kGrpHashCap;
      for (int g = tid; g < G; g += NT) {
        const uint64_t e = L.gsort[g];
        a.gt_e[o + g] = ge[g];
        a.gt_c[o + g] = (uint32_t)e;
        a.gt_k[o + g] = ~(uint32_t)(e >> 32);
      }
      if (tid == 0) a.gt_n[row] = G | (s_held == (unsigned long long)V ? kGtComplete : 0);
      res.ok = 2;
      __syncthreads();
      return res;
    }
  }
  // wave 0 walks the groups (its lanes look ahead 64 groups at a time)
  if (tid < kWave) {
    float s = 0.0f;
    const bool ok = group_sum(ge, gc, G, s);
    if (tid == 0) {
      if (!ok) s_fail = 1;
      s_sum = s;
    }
  }
  __syncthreads();
  NLS_GSTAMP(row, 5);
  if (s_fail) return res;
  const float s = s_sum;
  for (int g = tid; g < G; g += NT) ge[g] = ge[g] / s;  // (:57)
  __syncthreads();
  if (tid < kWave) {
    const GroupDraw dr = group_cut_draw(ge, gc, G, s_held == (unsigned long long)V, a.V,
                                        P.topp_active != 0, P.topP, P.minp_active != 0, P.minP32, u);
    // the drawn group: the first g with gc[0] + ... + gc[g] > pos, 64 groups
    // per step
    int g = 0;
    int64_t pos = dr.pos;
    if (dr.status == kGroupOk) {
      for (int base = 0; base < G; base += kWave) {
        const int c = base + lane < G ? (int)gc[base + lane] : 0;
        const int incl = wave_incl_scan(c);
        const int tot = __shfl(incl, kWave - 1, kWave);
        if (pos < (int64_t)tot || base + kWave >= G) {
          const uint64_t past = __ballot((int64_t)incl > pos);
          const int hl = past ? __ffsll((unsigned long long)past) - 1 : min(G - base, kWave) - 1;
          g = base + hl;
          pos -= (int64_t)(__shfl(incl, hl, kWave) - __shfl(c, hl, kWave));
          break;
        }
        pos -= tot;
      }
    }
    if (tid == 0) {
      s_draw = dr;
      s_g = g;
      s_t = pos;
    }
  }
  __syncthreads();
  NLS_GSTAMP(row, 6);
  if (s_draw.status != kGroupOk) return res;
  vg = key2f(~(uint32_t)(L.gsort[s_g] >> 32));
  t = s_t;
  grec = L.gsort[s_g];
  }
  // ---- the drawn candidate: the t-th lowest index holding value vg ----
  // Blocks of 64 lanes x W values (W = 4 with 16-byte loads): each wave
  // counts the members of its blocks (counts kept in the patch table's
  // count/bias arrays, free by now), then wave 0 finds the block holding the
  // t-th member and the lane and element inside it.
  const int wv = tid >> 6;
  uint32_t* bcnt = L.pcnt;  // pcnt and pbias are adjacent: 2 * kGrpPatchCap entries
  auto final_at = [&](int i, float x) -> float {
    const uint32_t wb = L.bitmap[i >> 5];
    if ((wb >> (i & 31)) & 1u) return L.pfin[slot_of(i)];
    return x * invT;
  };
  // members among this lane's W values of block bk (bit j: value j)
  auto lane_members = [&](int bk) -> uint32_t {
    uint32_t m = 0u;
    if (vec) {
      const int i4 = bk * kWave + lane;
      if (i4 < V4) {
        const float4 x = src4[i4];
        const int i = i4 * 4;
        m |= (final_at(i, x.x) == vg) ? 1u : 0u;
        m |= (final_at(i + 1, x.y) == vg) ? 2u : 0u;
        m |= (final_at(i + 2, x.z) == vg) ? 4u : 0u;
        m |= (final_at(i + 3, x.w) == vg) ? 8u : 0u;
      }
    } else {
      const int i = bk * kWave + lane;
      if (i < V) m = (final_at(i, src[i]) == vg) ? 1u : 0u;
    }
    return m;
  };
  const int W = vec ? 4 : 1;
  const int nblk = (V + kWave * W - 1) / (kWave * W);  // <= 2 * kGrpPatchCap for V <= kGrpMaxV
  // Counting pass: the unpatched members by value alone (the bitmap is read
  // only where a value matches), then the patched members from the patch
  // table; the exact search below walks one block with final_at.
  auto unpatched_at = [&](int i) -> bool { return !((L.bitmap[i >> 5] >> (i & 31)) & 1u); };
  auto lane_count = [&](int bk) -> int {
    int m = 0;
    if (vec) {
      const int i4 = bk * kWave + lane;
      if (i4 < V4) {
        const float4 x = src4[i4];
        const int i = i4 * 4;
        if (x.x * invT == vg && unpatched_at(i)) ++m;
        if (x.y * invT == vg && unpatched_at(i + 1)) ++m;
        if (x.z * invT == vg && unpatched_at(i + 2)) ++m;
        if (x.w * invT == vg && unpatched_at(i + 3)) ++m;
      }
    } else {
      const int i = bk * kWave + lane;
      if (i < V && src[i] * invT == vg && unpatched_at(i)) m = 1;
    }
    return m;
  };
  // A value that occurs once needs no search.  Otherwise the row is counted
  // in rounds of 4 * NW blocks and the walk stops at the round holding the
  // t-th member: in index order when t lies in the lower half of the group's
  // c members, else from the row's end for the (c - 1 - t)-th member from the
  // top (on average a quarter of the row is read).  The patched members go
  // in first.
  if ((uint32_t)grec & kGrpOne) {
    // a value that occurs once: its member was kept when it was counted
    if (tid == 0) s_id = (int)((uint32_t)grec & ~kGrpOne);
    __syncthreads();
  } else {
    const int64_t cg = (int64_t)group_count(grec);
    const bool rev = 2 * t >= cg;  // uniform
    for (int i = tid; i < nblk; i += NT) bcnt[i] = 0u;
    __syncthreads();
    for (int sl = tid; sl < np; sl += NT)
      if (L.pfin[sl] == vg) atomicAdd(&bcnt[L.pid[sl] / (kWave * W)], 1u);
    if (tid == 0) {
      s_left = rev ? cg - 1 - t : t;
      s_found = 0;
    }
    __syncthreads();
    // (one instance per direction: the index order's loop stays as plain as
    // when it was the only one)
    auto search = [&](auto rev_c) __attribute__((always_inline)) {
      constexpr bool REV = decltype(rev_c)::value;
      auto phys = [&](int lb) { return REV ? nblk - 1 - lb : lb; };  // logical block -> block
      constexpr int RB = 4 * NW;
      for (int r0 = 0; r0 < nblk; r0 += RB) {
        int m[4];
  #pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int lb = r0 + wv + u * NW;
          m[u] = lb < nblk ? lane_count(phys(lb)) : 0;
        }
  #pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int lb = r0 + wv + u * NW;
          const int c = wave_sum_i(m[u]);
          if (lane == 0 && lb < nblk) bcnt[phys(lb)] += (uint32_t)c;
        }
        __syncthreads();
        if (wv == 0) {
          int64_t left = s_left;
          const int rend = min(r0 + RB, nblk);
          for (int base = r0; base < rend; base += kWave) {
            const int c = (base + lane < rend) ? (int)bcnt[phys(base + lane)] : 0;
            const int incl = wave_incl_scan(c);
            const int sum = __shfl(incl, kWave - 1, kWave);
            if (left < sum) {
              // the block: the first lane whose inclusive count passes `left`
              const uint64_t past = __ballot((int64_t)incl > left);
              const int bl = __ffsll((unsigned long long)past) - 1;
              const int bk = phys(base + bl);
              const int64_t within = left - (__shfl(incl, bl, kWave) - __shfl(c, bl, kWave));
              const uint32_t mb = lane_members(bk);
              const int mc = __popc(mb);
              const int mi = wave_incl_scan(mc);
              // members before this lane's, in the walk's order
              const int64_t before = REV ? (int64_t)(__shfl(mi, kWave - 1, kWave) - mi) : (int64_t)(mi - mc);
              if (before <= within && within < before + mc) {
                uint32_t mm = mb;
                int e;
                if (REV) {
                  for (int r = (int)(within - before); r > 0; --r) mm &= ~(1u << (31 - __clz(mm)));
                  e = 31 - __clz(mm);
                } else {
                  for (int r = (int)(within - before); r > 0; --r) mm &= mm - 1u;
                  e = __ffs(mm) - 1;
                }
                s_id = (bk * kWave + lane) * W + e;
              }
              if (lane == 0) s_found = 1;
              break;
            }
            left -= sum;
          }
          if (lane == 0) s_left = left;
        }
        __syncthreads();
        if (s_found) break;
      }
    };
    if (rev)
      search(std::true_type{});
    else
      search(std::false_type{});
  }
  NLS_GSTAMP(row, 7);
  if (s_id < 0) return res;
  res.ok = 1;
  res.id = s_id;
  if constexpr (STAGE != 3) {
    res.n = (int)s_draw.n;
    res.total = s_draw.total;
  }
  __syncthreads();
  return res;
}

// Top-k rows (k <= NT) of the whole-row path without the sort: kA holds the
// row's ~keys (final values, patches and temperature applied), and each
// thread's largest key (tmax) is a distinct element, so the k-th largest of
// the NT thread maxima bounds the row's k-th largest key from below.  The
// elements at or above it go to an LDS list, the heap rule picks the k
// members (sampler.nim:85-95) and the tail runs (:98-121).  False, before
// the row's uniform is taken, when the list or the tie set does not fit:
// the caller sorts the row instead.
constexpr int kWinEnt = 8192;  // listed elements
constexpr int kWinMem = 2048;  // members / tie set
constexpr size_t kWinLdsBytes = (size_t)kWinEnt * 8 + (size_t)kWinMem * 8 + 3 * 1024 * 4;
static_assert(kWinLdsBytes <= (size_t)kGrpPatchCap * 16 + (size_t)kGrpHashCap * 16,
              "the list fits the whole-row kernel's dynamic LDS (group_lds_bytes)");
template <int NT>
__device__ __forceinline__ bool window_topk(const GenericArgs& a, int row, const RowParams& P,
                                            const uint32_t* kA, uint32_t tmax, uint32_t* hist,
                                            int* smem, double* s_u_p, int* s_i, unsigned char* glds) {
  static_assert(NT <= 1024, "vals/ids/e hold k <= 1024 members");
  const int n = (int)a.V;
  const int k = P.k;
  const int tid = threadIdx.x;
  uint64_t* ent = reinterpret_cast<uint64_t*>(glds);
  uint64_t* mem = ent + kWinEnt;
  float* vals = reinterpret_cast<float*>(mem + kWinMem);
  int32_t* ids = reinterpret_cast<int32_t*>(vals + 1024);
  float* ebuf = reinterpret_cast<float*>(ids + 1024);
  for (int q = tid; q < kSelWords; q += NT) hist[q] = 0u;
  if (tid == 0) {
    s_i[2] = 0;
    s_i[3] = 0;
  }
  __syncthreads();
  const SelectResult b0 = block_select<NT>([&](auto fn) { fn(tmax, tid < n); }, k, -1, hist, smem);
  const uint32_t t0 = b0.tau;
  for (int i = tid; i < n; i += NT) {
    const uint32_t key = ~kA[i];
    if (key >= t0) {
      const int p = atomicAdd(&s_i[2], 1);
      if (p < kWinEnt) ent[p] = ((uint64_t)key << 32) | (uint32_t)i;
    }
  }
  __syncthreads();
  const int N = s_i[2];
  if (N > kWinEnt || !topk_members<NT>(ent, N, k, mem, kWinMem, hist, smem, &s_i[3])) {
    __syncthreads();
    return false;
  }
  if (tid == 0) *s_u_p = row_uniform(a.d_u, a.rng, row);
  __syncthreads();
  if (k <= kWave) {
    if ((tid >> 6) == 0) wave_tail(mem, k, P, *s_u_p, row, a.out, a.dbg, 5);
    __syncthreads();
    return true;
  }
  const int kpow = next_pow2(k);
  for (int i = k + tid; i < kpow; i += NT) mem[i] = 0ull;
  __syncthreads();
  bitonic_sort_u64<NT>(mem, kpow, true);
  for (int i = tid; i < k; i += NT) {
    vals[i] = key2f((uint32_t)(mem[i] >> 32));
    ids[i] = (int32_t)(uint32_t)mem[i];
  }
  __syncthreads();
  const TailOut to = softmax_cutoff_draw<NT>(vals, ids, ebuf, k, P, *s_u_p, smem);
  if (tid == 0) a.out[row] = to.id;
  write_debug<NT>(a.dbg, row, 5 | to.nan_cand, to.n, k, to.total, ids, ebuf);
  __syncthreads();
  return true;
}

// Rows of the list from index w0 on, every nw-th: the whole-row path.  LDS
// scratch is passed in (wcnt: NW * 256 words, dbase and drun: 256 each), so
// that the streaming kernel's last workgroup can run it too.
template <int NT, bool GROUPED, bool CLAIM, bool ONLY>
__device__ __forceinline__ void generic_rows(const GenericArgs& a, int w0, int nw, int count, uint32_t* wcnt,
                                             uint32_t* dbase, uint32_t* drun, int* smem, double* s_u_p,
                                             int* s_i, float* s_rv, int* s_ri, unsigned char* glds) {
  constexpr int NW = NT / kWave;
  const int n = (int)a.V;
  const int tid = threadIdx.x;
  uint32_t* kA = a.scratch + (int64_t)w0 * a.vpad * 5;
  uint32_t* iA = kA + a.vpad;
  uint32_t* kB = iA + a.vpad;
  uint32_t* iB = kB + a.vpad;
  float* work = reinterpret_cast<float*>(iB + a.vpad);
  const int nfx = a.fixed_list ? a.n_fixed : 0;
  // With a claim counter every workgroup takes the next unclaimed row when it
  // is done with one, so rows of uneven cost spread evenly; the barriers keep
  // the broadcast slot from being overwritten before every thread has read it.
  // (only the whole-row kernel's claiming instance: the others keep their
  // code, and the streaming kernels' last workgroup serves its rows alone)
  __shared__ int s_claim;
  auto next_row = [&](int li_static) -> int {
    if constexpr (!CLAIM) return li_static;
    if (!a.claim) return li_static;
    __syncthreads();
    if (tid == 0) s_claim = atomicAdd(a.claim, 1);
    __syncthreads();
    return s_claim;
  };
  for (int li = next_row(w0); li < nfx + count; li = next_row(li + nw)) {
    int row = li < nfx ? a.fixed_list[li] : load_agent(&a.generic_list[li - nfx]);
    // (a fallback list's row may carry the uniform the grouped launch drew)
    const bool u_saved = a.fb_in && (row & kFbUSaved) != 0;
    row &= ~kFbUSaved;
    if (a.row_done && a.row_done[row] != 0) {  // a finished row of a batched loop
      if (tid == 0) a.out[row] = -1;
      continue;
    }
    const RowParams P = a.rp[row];
    const float* __restrict__ src = a.logits + (int64_t)row * a.V;
    bool u_taken = false;
    GroupOut gout;
    gout.ok = 0;
    if constexpr (GROUPED) {
      if (P.mode == kModeFull && a.grouped && !a.fb_in) {
        if (tid == 0) *s_u_p = row_uniform(a.d_u, a.rng, row);
        __syncthreads();
        u_taken = true;
        gout = grouped_row<NT, ONLY ? 1 : 0>(a, row, P, *s_u_p, group_lds(glds, (int)((a.V + 31) >> 5)), smem);
        if constexpr (ONLY) {
          if (gout.ok == 2) {
            // groups stored: the walk launch takes the row, with its uniform
            if (tid == 0) {
              a.fb_u[row] = *s_u_p;
              const int i = atomicAdd(a.w_count, 1);
              if (i < a.list_cap) a.w_list[i] = row;  // (a list never holds more than the batch)
            }
            __syncthreads();
            continue;
          }
        }
        if (gout.ok) {
          if (tid == 0) {
            a.out[row] = gout.id;
            if (a.dbg.n) a.dbg.n[row] = gout.n;
            if (a.dbg.ncand) a.dbg.ncand[row] = n;
            if (a.dbg.total) a.dbg.total[row] = gout.total;
            if (a.dbg.path) a.dbg.path[row] = 3;
          }
          // candidate lists are asked for: the whole-row sort below writes
          // them (its id, n and total are replaced by these afterwards)
          if (!a.dbg.cand_ids && !a.dbg.cand_probs) {
            __syncthreads();
            continue;
          }
        }
        __syncthreads();
      }
    }
    if constexpr (ONLY) {
      // the grouped launch: every other row (or a grouped one that failed)
      // goes to the fallback list for the next launch
      if (tid == 0) {
        const int i = atomicAdd(a.fb_count, 1);
        if (i < a.list_cap) a.fb_list[i] = row | (u_taken ? kFbUSaved : 0);
        if (u_taken) a.fb_u[row] = *s_u_p;
      }
      __syncthreads();
      continue;
    }
    // window counts (kB) and bias slots + 1 (iB) per id (:64-76)
    for (int i = tid; i < n; i += NT) {
      kB[i] = 0u;
      iB[i] = 0u;
    }
    __syncthreads();
    const int64_t hlen = a.hist_len[row];
    int n_hist = 0;
    if (P.pen_active && hlen > 0)
      n_hist = (int)((P.repeat_last_n > 0 && P.repeat_last_n < hlen) ? P.repeat_last_n : hlen);
    if (n_hist > 0) {
      const int hbase = (int)((hlen - n_hist) % a.hcap);
      const int32_t* __restrict__ hrow = a.hist + (int64_t)row * a.hcap;
      for (int i = tid; i < n_hist; i += NT) {
        int slot = hbase + i;
        if (slot >= a.hcap) slot -= a.hcap;
        const int id = hrow[slot];
        if (id >= 0 && id < n) atomicAdd(&kB[id], 1u);
      }
    }
    for (int j = tid; j < P.bias_cnt; j += NT) iB[a.bias_ids[P.bias_off + j]] = (uint32_t)j + 1u;
    __syncthreads();
    const bool greedy = P.mode == kModeGreedy;
    float bv = -__builtin_inff();
    int bi = 0x7fffffff;
    uint32_t tmax = 0u;  // the thread's largest key (a distinct element per thread)
    for (int i = tid; i < n; i += NT) {
      float v = src[i];
      const uint32_t c = kB[i];
      if (c) {
        if (P.rp_active) v = (v > 0.0f) ? (v / P.rp32) : (v * P.rp32);
        v = v - (float)((double)c * P.freq + P.pres);
      }
      const uint32_t bj = iB[i];
      if (bj) v = v + a.bias_vals[P.bias_off + (int)bj - 1];
      if (greedy) {
        argmax_merge(bv, bi, v, i);
      } else {
        const uint32_t key = f2key(v * P.invT);
        tmax = max(tmax, key);
        kA[i] = ~key;
        iA[i] = (uint32_t)i;
      }
    }
    if (greedy) {
      wave_argmax(bv, bi);
      if (lane_id() == 0) {
        s_rv[tid >> 6] = bv;
        s_ri[tid >> 6] = bi;
      }
      __syncthreads();
      if (tid == 0) {
        float rv = s_rv[0];
        int ri = s_ri[0];
        for (int w = 1; w < NW; ++w) argmax_merge(rv, ri, s_rv[w], s_ri[w]);
        // argmax (:45-49) starts at index 0 and NaN compares greater than nothing
        float x0 = src[0];
        if (kB[0]) {
          if (P.rp_active) x0 = (x0 > 0.0f) ? (x0 / P.rp32) : (x0 * P.rp32);
          x0 = x0 - (float)((double)kB[0] * P.freq + P.pres);
        }
        if (iB[0]) x0 = x0 + a.bias_vals[P.bias_off + (int)iB[0] - 1];
        a.out[row] = (x0 != x0) ? 0 : ri;
        if (a.dbg.n) a.dbg.n[row] = 0;
        if (a.dbg.ncand) a.dbg.ncand[row] = 0;
        if (a.dbg.total) a.dbg.total[row] = 0.0f;
        if (a.dbg.path) a.dbg.path[row] = 1;
      }
      __syncthreads();
      continue;
    }
    __syncthreads();
    if constexpr (GROUPED) {
      if (P.mode == kModeTopK && P.k <= NT && glds && a.grouped &&
          window_topk<NT>(a, row, P, kA, tmax, wcnt, smem, s_u_p, s_i, glds))
        continue;
    }
    radix_sort_pass<NT>(kA, iA, kB, iB, n, 0, wcnt, dbase, drun);
    radix_sort_pass<NT>(kB, iB, kA, iA, n, 8, wcnt, dbase, drun);
    radix_sort_pass<NT>(kA, iA, kB, iB, n, 16, wcnt, dbase, drun);
    radix_sort_pass<NT>(kB, iB, kA, iA, n, 24, wcnt, dbase, drun);
    // kA: ~key ascending (value descending, index ascending on ties)
    if (tid == 0 && !u_taken) *s_u_p = u_saved ? a.fb_u[row] : row_uniform(a.d_u, a.rng, row);
    __syncthreads();
    if (P.mode == kModeFull) {
      // candidates = the whole sorted row (:96-97); values into work, ids stay in iA
      for (int i = tid; i < n; i += NT) work[i] = key2f(~kA[i]);
      __syncthreads();
      const TailOut t = softmax_cutoff_draw<NT>(work, iA, reinterpret_cast<float*>(kB), n, P, *s_u_p,
                                                smem);
      if (tid == 0) a.out[row] = t.id;
      write_debug<NT>(a.dbg, row, 4 | t.nan_cand, t.n, n, t.total, iA, reinterpret_cast<float*>(kB));
      if (gout.ok && tid == 0) {
        a.out[row] = gout.id;
        if (a.dbg.n) a.dbg.n[row] = gout.n;
        if (a.dbg.total) a.dbg.total[row] = gout.total;
        if (a.dbg.path) a.dbg.path[row] = 3;
      }
      __syncthreads();
      continue;
    }
    // ---- top-k row (k < V) by the heap rule (:85-95) ----
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
      for (int i = tid; i < gp; i += NT) gs[i] = (i < g) ? (uint64_t)iA[i] : ~0ull;
      __syncthreads();
      bitonic_sort_u64<NT>(gs, gp, false);
      if (tid == 0) {
        int x = 0, y = 0;  // x over G, y over ties
        int taken = 0;
        while (taken < k) {
          const uint64_t gi = (x < g) ? gs[x] : ~0ull;
          const uint64_t ti = (g + y < tend) ? (uint64_t)iA[g + y] : ~0ull;
          if (gi < ti)
            ++x;
          else
            ++y;
          ++taken;
        }
        s_i[0] = g + y - m;  // the last m ties taken
        s_i[1] = g + y;
      }
      __syncthreads();
      take_lo = s_i[0];
      take_hi = s_i[1];
      __syncthreads();
    }
    // reference order: value descending, index descending on ties.  Reverse
    // every run of equal values among G; the selected ties come last, reversed.
    for (int i = tid; i < g; i += NT) {
      const uint32_t key = kA[i];
      const int x = lower_bound_u32(kA, g, key);
      const int y = upper_bound_u32(kA, g, key);
      const int o = x + (y - 1 - i);
      work[o] = key2f(~key);
      reinterpret_cast<int32_t*>(kB)[o] = (int32_t)iA[i];
    }
    for (int i = take_lo + tid; i < take_hi; i += NT) {
      const int o = g + (take_hi - 1 - i);
      work[o] = key2f(~kA[i]);
      reinterpret_cast<int32_t*>(kB)[o] = (int32_t)iA[i];
    }
    __syncthreads();
    const TailOut t = softmax_cutoff_draw<NT>(work, reinterpret_cast<int32_t*>(kB),
                                              reinterpret_cast<float*>(iB), k, P, *s_u_p, smem);
    if (tid == 0) a.out[row] = t.id;
    write_debug<NT>(a.dbg, row, 4 | t.nan_cand, t.n, k, t.total, reinterpret_cast<int32_t*>(kB),
                    reinterpret_cast<float*>(iB));
    __syncthreads();
  }
}

// CLAIM: workgroups claim rows one at a time (a.claim); otherwise workgroup w
// takes list positions w, w + gridDim.x, ...
template <int NT, bool CLAIM>
__global__ __launch_bounds__(NT) void generic_kernel(const GenericArgs a) {
  constexpr int NW = NT / kWave;
  __shared__ uint32_t wcnt[NW * 256];
  __shared__ uint32_t dbase[256];
  __shared__ uint32_t drun[256];
  __shared__ int smem[NW + 4];
  __shared__ double s_u;
  __shared__ int s_i[4];
  __shared__ float s_rv[NW];
  __shared__ int s_ri[NW];
  extern __shared__ __align__(16) unsigned char glds[];  // group_lds_bytes(V) when a.grouped
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    *a.next_count = 0;
    if (a.next_claim) *a.next_claim = 0;
    zero_next_counters(a);
  }
  const int count = min(*a.generic_count, a.list_cap);  // (a list never holds more than the batch)
  generic_rows<NT, true, CLAIM>(a, blockIdx.x, gridDim.x, count, wcnt, dbase, drun, smem, &s_u, s_i, s_rv, s_ri,
                         glds);
}

// The grouped rows alone (a launch without the whole-row sort's code, whose
// registers it does not share): the rows it does not finish are listed for a
// generic_kernel launch after it.
template <int NT, bool CLAIM>
__global__ __launch_bounds__(NT) void generic_grouped_kernel(const GenericArgs a) {
  constexpr int NW = NT / kWave;
  __shared__ uint32_t wcnt[NW * 256];
  __shared__ uint32_t dbase[256];
  __shared__ uint32_t drun[256];
  __shared__ int smem[NW + 4];
  __shared__ double s_u;
  __shared__ int s_i[4];
  __shared__ float s_rv[NW];
  __shared__ int s_ri[NW];
  extern __shared__ __align__(16) unsigned char glds[];  // group_lds_bytes(V) when a.grouped
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    *a.next_count = 0;
    if (a.next_claim) *a.next_claim = 0;
    zero_next_counters(a);
  }
  const int count = min(*a.generic_count, a.list_cap);  // (a list never holds more than the batch)
  generic_rows<NT, true, CLAIM, true>(a, blockIdx.x, gridDim.x, count, wcnt, dbase, drun, smem, &s_u, s_i, s_rv, s_ri,
                         glds);
}


// A row that leaves the grouped path for the whole-row launch, its uniform
// kept (fb_u holds it).
__device__ __forceinline__ void push_fallback(const GenericArgs& a, int row) {
  const int i = atomicAdd(a.fb_count, 1);
  if (i < a.list_cap) a.fb_list[i] = row | kFbUSaved;
}

// The walk over the groups the grouped launch stored for `row`, by one wave:
// the softmax sum, top-p, min-p, total and the draw over the groups
// (nls_grouped.h), then the drawn group.  A group of one candidate names the
// id; a row that cannot be finished goes to the fallback list.  Returns true
// when the drawn member must be searched for: the group's count record,
// value key and the member's rank are then in a.p3_*[row].  ge/gc: this
// wave's LDS for kGrpHashCap exponentials and counts.
__device__ __forceinline__ bool walk_row(const GenericArgs& a, int row, float* ge, uint32_t* gc) {
  const int lane = lane_id();
  // (LDS writes of the wave before its lanes read them: a workgroup-scope
  // fence waits for them; no barrier, since the other waves do not take part)
  auto lds_sync = []() { __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup"); };
  NLS_GSTAMP(row, 8);
  const RowParams P = a.rp[row];
  const double u = a.fb_u[row];
  const int gn = a.gt_n[row];
  const int G = gn & ~kGtComplete;
  const bool complete = (gn & kGtComplete) != 0;
  const size_t o = (size_t)row * kGrpHashCap;
  for (int g = lane; g < G; g += kWave) {
    ge[g] = a.gt_e[o + g];
    gc[g] = group_count((uint64_t)a.gt_c[o + g]);
  }
  lds_sync();
  float s = 0.0f;
  if (!group_sum(ge, gc, G, s)) {
    if (lane == 0) push_fallback(a, row);
    return false;
  }
  NLS_GSTAMP(row, 5);
  for (int g = lane; g < G; g += kWave) ge[g] = ge[g] / s;  // (:57)
  lds_sync();
  const GroupDraw dr = group_cut_draw(ge, gc, G, complete, a.V, P.topp_active != 0, P.topP,
                                      P.minp_active != 0, P.minP32, u);
  if (dr.status != kGroupOk) {
    if (lane == 0) push_fallback(a, row);
    return false;
  }
  // the drawn group: the first g with gc[0] + ... + gc[g] > pos, 64 groups
  // per step
  int g = 0;
  int64_t pos = dr.pos;
  for (int base = 0; base < G; base += kWave) {
    const int c = base + lane < G ? (int)gc[base + lane] : 0;
    const int incl = wave_incl_scan(c);
    const int tot = __shfl(incl, kWave - 1, kWave);
    if (pos < (int64_t)tot || base + kWave >= G) {
      const uint64_t past = __ballot((int64_t)incl > pos);
      const int hl = past ? __ffsll((unsigned long long)past) - 1 : min(G - base, kWave) - 1;
      g = base + hl;
      pos -= (int64_t)(__shfl(incl, hl, kWave) - __shfl(c, hl, kWave));
      break;
    }
    pos -= tot;
  }
  NLS_GSTAMP(row, 6);
  const uint32_t rec = a.gt_c[o + g];
  if (lane == 0) {
    if (a.dbg.n) a.dbg.n[row] = (int)dr.n;
    if (a.dbg.ncand) a.dbg.ncand[row] = (int)a.V;
    if (a.dbg.total) a.dbg.total[row] = dr.total;
    if (a.dbg.path) a.dbg.path[row] = 3;
    if (rec & kGrpOne) {
      // a value that occurs once: its member was kept when it was counted
      a.out[row] = (int32_t)(rec & ~kGrpOne);
      NLS_GSTAMP(row, 9);
      NLS_GSTAMP(row, 7);
    } else {
      a.p3_rec[row] = rec;
      a.p3_key[row] = a.gt_k[o + g];
      a.p3_t[row] = pos;
    }
  }
  return (rec & kGrpOne) == 0u;
}

// The walks and member searches of the rows the grouped launch stored
// (a.w_list), kWalkRows rows at a time per workgroup: waves 0 .. kWalkRows-1
// walk one row each (walk_row), then the whole workgroup runs the member
// search of each row whose drawn value occurs more than once (the row's patch
// table again, then grouped_row's last step).  Dynamic LDS: the waves' walk
// tables, later the search's patch table (walk_member_lds_bytes).
template <int NT>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(2 * NT / kWave / 4))) void walk_member_kernel(
    const GenericArgs a) {
  static_assert(NT / kWave >= kWalkRows, "one wave per row");
  __shared__ int smem[NT / kWave + 4];
  __shared__ int s_row[kWalkRows];
  extern __shared__ __align__(16) unsigned char glds[];
  const int wv = threadIdx.x >> 6;
  if (blockIdx.x == 0 && threadIdx.x == 0) *a.w_next = 0;
  const int count = min(*a.w_count, a.list_cap);
  const int nw = (int)((a.V + 31) >> 5);
  for (int l0 = blockIdx.x * kWalkRows; l0 < count; l0 += gridDim.x * kWalkRows) {
    if (wv < kWalkRows) {
      int need = -1;
      if (l0 + wv < count) {
        const int row = a.w_list[l0 + wv];
        float* ge = reinterpret_cast<float*>(glds) + (size_t)wv * 2 * kGrpHashCap;
        if (walk_row(a, row, ge, reinterpret_cast<uint32_t*>(ge + kGrpHashCap))) need = row;
      }
      if (lane_id() == 0) s_row[wv] = need;
    }
    __syncthreads();  // the walks (and their p3_* records) are done
    for (int j = 0; j < kWalkRows; ++j) {
      const int row = s_row[j];
      if (row < 0) continue;  // (uniform)
      const RowParams P = a.rp[row];
      const GroupOut r = grouped_row<NT, 3>(a, row, P, 0.0, group_lds(glds, nw), smem);
      if (threadIdx.x == 0) {
        if (r.ok)
          a.out[row] = r.id;
        else
          push_fallback(a, row);
      }
      __syncthreads();
    }
    __syncthreads();  // s_row and the LDS are free for the next rows
  }
}

}  // namespace nls
