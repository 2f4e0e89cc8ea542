// floor_kernel: the full-sort rows (src/nimllm/sampler.nim:96-121) of a batch
// made only of such rows, each row split over workgroups of one slice each.
//
// On the sort path every step after the sort is an fp32 chain in descending
// order whose first term is the maximum's: the softmax sum starts at
// exp(0) = 1, the top-p running sum and the total at 1/s, the draw at
// u * total.  A value with fl(v - mx) < kGroupFloor has exp(v - mx) < 2^-25, a
// term below half a spacing of any of these sums, so it changes none of them
// (nls_grouped.h).  The row's values at or above the floor are therefore all
// the sort path needs -- unless a chain runs past them (top-p not reached,
// min-p keeping all of them, the draw not ended), which only happens when the
// row's mass is spread thin, and then the row goes to the whole-row launch.
//
// A row's slices are read by one workgroup each, straight into registers,
// while the slice's patch table (window ids and bias ids in the slice) is
// built in LDS.  The slice keeps its values within the floor of its own
// maximum (a superset of those within the floor of the row's, which is no
// smaller), publishes them with its maximum, and the last slice of the row to
// arrive merges: it filters them against the row maximum, sorts them by value
// (descending) then index, and runs softmax, top-p, min-p and the draw over
// them.  Rows with a NaN, an infinite maximum, more kept values than the
// buffers hold, or a chain past the kept values are listed for the whole-row
// launch (the row's RNG state untouched, so that launch draws its uniform).
#include "nls_device.h"
#include "nls_launch.h"

namespace nls {

namespace {

// Phase 1 (one slice): bitmap [kFloorSlice / 32] | wpre [kFloorSlice / 32] |
// pid | pcnt | pbias | pfin [kFloorPatchCap] | keep [kFloorKeep].
// Phase 2 (the merge, after the slice is published): sorted (value, index)
// records [kFloorMerge] | vals | ids | e [kFloorMerge].
struct FloorLds {
  uint32_t* bitmap;
  uint32_t* wpre;
  int32_t* pid;
  uint32_t* pcnt;
  int32_t* pbias;
  float* pfin;
  uint64_t* keep;
};

__device__ __forceinline__ FloorLds floor_lds(unsigned char* base) {
  FloorLds L;
  L.bitmap = reinterpret_cast<uint32_t*>(base);
  L.wpre = L.bitmap + kFloorSlice / 32;
  L.pid = reinterpret_cast<int32_t*>(L.wpre + kFloorSlice / 32);
  L.pcnt = reinterpret_cast<uint32_t*>(L.pid + kFloorPatchCap);
  L.pbias = reinterpret_cast<int32_t*>(L.pcnt + kFloorPatchCap);
  L.pfin = reinterpret_cast<float*>(L.pbias + kFloorPatchCap);
  L.keep = reinterpret_cast<uint64_t*>(L.pfin + kFloorPatchCap);
  return L;
}

__device__ __forceinline__ float f4_at(const f32x4& x, int e) { return x[e]; }

// A kept value's record: the key in the high word, the index's complement in
// the low word, so that a descending sort orders by value, then by index.
__device__ __forceinline__ uint64_t floor_rec(float v, int idx) {
  return ((uint64_t)f2key(v) << 32) | (uint32_t)~(uint32_t)idx;
}

// softmax_cutoff_draw (nls_device.h) for at most 64 candidates: one wave
// holds them, one per lane, and runs each fp32 chain in order with the
// terms read across lanes -- the same operations in the same sequence (the
// softmax sum :51-57, top-p :103-108, min-p :110-114, the total :115-116 and
// the draw :117-120).  Every thread of the workgroup calls it.
template <int NT>
__device__ __forceinline__ TailOut small_tail(const float* vals, const int32_t* ids, float* probs, int ncand,
                                              const RowParams& P, double u, int* beyond) {
  __shared__ float s_total;
  __shared__ int s_n, s_pos;
  if (threadIdx.x < kWave) {
    const int lane = (int)threadIdx.x;
    auto at = [](float x, int i) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), i)); };
    const float mx = vals[0];  // candidates are in non-increasing order
    float e = lane < ncand ? expf_cr(vals[lane] - mx) : 0.0f;
    float s = 0.0f;
    for (int i = 0; i < ncand; ++i) s = s + at(e, i);
    e = e / s;
    if (lane < ncand) probs[lane] = e;
    int n = ncand;
    float cum_n = 0.0f;
    bool past = false;
    if (P.topp_active) {
      float cum = 0.0f;
      int stop = ncand;
      for (int i = 0; i < ncand; ++i) {
        cum = cum + at(e, i);
        if ((double)cum >= P.topP) {
          stop = i;
          break;
        }
      }
      if (stop < ncand) n = stop + 1;
      cum_n = cum;
      past = stop >= ncand;
    }
    const int n_topp = n;
    if (P.minp_active) {
      const float thr = at(e, 0) * P.minP32;
      int m = n;
      const uint64_t fail = __ballot(lane >= 1 && lane < n && !(e >= thr));
      if (fail) m = __ffsll((unsigned long long)fail) - 1;
      past |= m == ncand;
      n = m;
    }
    float total = 0.0f;
    if (P.topp_active && n == n_topp) {
      total = cum_n;
    } else {
      for (int i = 0; i < n; ++i) total = total + at(e, i);
    }
    float r = (float)u * total;
    int hit = n;
    for (int i = 0; i < n; ++i) {
      r = r - at(e, i);
      if (r <= 0.0f) {
        hit = i;
        break;
      }
    }
    past |= hit >= n && n == ncand;
    if (lane == 0) {
      s_n = n;
      s_total = total;
      s_pos = hit < n ? hit : n - 1;
      *beyond = past ? 1 : 0;
    }
  }
  __syncthreads();
  TailOut t;
  t.n = s_n;
  t.total = s_total;
  t.id = ids[s_pos];
  t.nan_cand = 0;  // (rows with a NaN never reach the merge)
  return t;
}

}  // namespace

// Two 512-thread workgroups per CU: registers held to 128 (the slice takes 64
// of them), kFloorLds bytes of dynamic LDS each.
template <int NT, bool VEC>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(2 * NT / kWave / 4))) void floor_kernel(
    const FloorArgs a) {
  static_assert(NT == kFloorThreads, "a slice is kFloorVec4 float4 per thread of kFloorThreads");
  constexpr int NW = NT / kWave;
  constexpr int NV = kFloorVec4;
  constexpr int NWD = kFloorSlice / 32;
  constexpr int PER = NWD / NT;  // bitmap words per thread in the prefix scan
  static_assert(NWD % NT == 0, "bitmap words split evenly over the threads");
  extern __shared__ __align__(16) unsigned char lds[];
  __shared__ int smem[NW + 4];
  __shared__ int s_n, s_bad, s_last, s_beyond;
  __shared__ uint32_t s_max;
  __shared__ int s_off[kFloorMaxSlices + 1];
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int row = blockIdx.x / a.S;
  const int sl = blockIdx.x - row * a.S;
  const int V = (int)a.V;
  const int lo = sl * kFloorSlice;
  const int len = min(kFloorSlice, V - lo);
  const float* __restrict__ src = a.logits + (int64_t)row * a.V;
  // phase stamps (the `phases` build): per workgroup 0 start, 1 row constants
  // in, 2 patch table, 3 slice maximum (the slice is in), 4 kept values, 5
  // published; the merging workgroup 6 records read, 7 merged, 8 sorted, 9 tail
  auto stamp = [&](int i) {
    if (threadIdx.x == 0) NLS_STAMP((int)blockIdx.x, i);
  };
  stamp(0);
  // ---- requests, before anything is waited for: the history ring and the
  // bias list when each fits one entry per thread, then the slice (loads past
  // a range read 0 without touching memory); the row constants follow as
  // scalar loads.  Load counters complete in issue order, so the patch table
  // is built while the slice is in flight. ----
  constexpr int kOutOfRange = 0x7ffffff0;
  const bool ring_early = a.hcap > 0 && a.hcap <= NT;
  const bool bias_early = a.bstride > 0 && a.bstride <= NT;
  int ring_id, bias_id;
  {
    const __amdgpu_buffer_rsrc_t hr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int32_t*>(a.hist + (ring_early ? (int64_t)row * a.hcap : 0)), (short)0,
        ring_early ? a.hcap * 4 : 0, 0x00020000);
    ring_id = (int)__builtin_amdgcn_raw_buffer_load_b32(hr, tid < a.hcap ? tid * 4 : kOutOfRange, 0, 0);
    const __amdgpu_buffer_rsrc_t br = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int32_t*>(a.bias_ids + (bias_early ? (int64_t)row * a.bstride : 0)), (short)0,
        bias_early ? a.bstride * 4 : 0, 0x00020000);
    bias_id = (int)__builtin_amdgcn_raw_buffer_load_b32(br, tid < a.bstride ? tid * 4 : kOutOfRange, 0, 0);
  }
  f32x4 x[NV];
  {
    const __amdgpu_buffer_rsrc_t rs = slice_rsrc(src + lo, len);
#pragma unroll
    for (int j = 0; j < NV; ++j) x[j] = load_group<4 * NT, VEC>(rs, 0, j, tid);
  }
  __builtin_amdgcn_sched_barrier(0);  // keep the requests here
  const RowParams P = load_const(a.rp + row);
  const int64_t hlen = load_const(a.hist_len + row);
  if (a.row_done && load_const(a.row_done + row) != 0) {  // a finished row of a batched loop
    if (sl == 0 && tid == 0) a.out[row] = -1;
    return;
  }
  const FloorLds L = floor_lds(lds);
  // ---- patch table: the window's ids (:64-70) and the bias ids (:75-76) in the slice ----
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
  // Each thread's first window id and bias id, read once for both passes:
  // from the early requests (ring slot tid holds window position
  // (tid - hbase) mod hcap), else by loads that need no branch.
  int hid0, bid0;
  if (ring_early) {
    int wpos = tid - hbase;
    if (wpos < 0) wpos += a.hcap;
    hid0 = (tid < a.hcap && wpos < n_hist) ? ring_id : -1;
  } else {
    int slot = hbase + tid;
    if (slot >= a.hcap) slot -= a.hcap;
    const __amdgpu_buffer_rsrc_t hr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int32_t*>(hrow), (short)0, n_hist > 0 ? a.hcap * 4 : 0, 0x00020000);
    const int h = (int)__builtin_amdgcn_raw_buffer_load_b32(hr, tid < n_hist ? slot * 4 : kOutOfRange, 0, 0);
    hid0 = tid < n_hist ? h : -1;
  }
  if (bias_early) {
    bid0 = tid < P.bias_cnt ? bias_id : -1;
  } else {
    const __amdgpu_buffer_rsrc_t br = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int32_t*>(a.bias_ids + P.bias_off), (short)0, P.bias_cnt * 4, 0x00020000);
    const int bb = (int)__builtin_amdgcn_raw_buffer_load_b32(br, tid < P.bias_cnt ? tid * 4 : kOutOfRange, 0, 0);
    bid0 = tid < P.bias_cnt ? bb : -1;
  }
  // (a ring that fits one slot per thread holds the whole window: n_hist <= hcap <= NT)
  const int n_hist_rest = ring_early ? 0 : n_hist;
  stamp(1);
  for (int i = tid; i < NWD; i += NT) L.bitmap[i] = 0u;
  for (int i = tid; i < kFloorPatchCap; i += NT) {
    L.pcnt[i] = 0u;
    L.pbias[i] = -1;
  }
  if (tid == 0) {
    s_n = 0;
    s_bad = 0;
    s_max = 0u;
  }
  __syncthreads();
  auto in_slice = [&](int id) { return id >= lo && id < lo + len; };
  auto mark = [&](int id) {
    if (in_slice(id)) atomicOr(&L.bitmap[(id - lo) >> 5], 1u << ((id - lo) & 31));
  };
  mark(hid0);
  for (int i = tid + NT; i < n_hist_rest; i += NT) mark(hist_id(i));
  mark(bid0);
  for (int j = tid + NT; j < P.bias_cnt; j += NT) mark(a.bias_ids[P.bias_off + j]);
  __syncthreads();
  int pc = 0;
#pragma unroll
  for (int q = 0; q < PER; ++q) pc += __popc(L.bitmap[tid * PER + q]);
  int np;
  int run = block_excl_scan<NT>(pc, smem, np);
  const bool ptab = np <= kFloorPatchCap;  // uniform
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    L.wpre[tid * PER + q] = (uint32_t)run;
    run += __popc(L.bitmap[tid * PER + q]);
  }
  __syncthreads();
  auto slot_of = [&](int r) {  // r: index in the slice of a patched id
    const int w = r >> 5;
    return (int)L.wpre[w] + __popc(L.bitmap[w] & ((1u << (r & 31)) - 1u));
  };
  if (ptab) {
    auto count = [&](int id) {
      if (in_slice(id)) {
        const int p = slot_of(id - lo);
        atomicAdd(&L.pcnt[p], 1u);
        L.pid[p] = id;
      }
    };
    auto biased = [&](int id, int j) {
      if (in_slice(id)) {
        const int p = slot_of(id - lo);
        L.pbias[p] = j;
        L.pid[p] = id;
      }
    };
    count(hid0);
    for (int i = tid + NT; i < n_hist_rest; i += NT) count(hist_id(i));
    biased(bid0, tid);
    for (int j = tid + NT; j < P.bias_cnt; j += NT) biased(a.bias_ids[P.bias_off + j], j);
  }
  const int npt = ptab ? np : 0;
  stamp(2);
  // ---- the slice maximum over the final values (:53) ----
  // Each thread's patched values: one bit per value, from one bitmap word per
  // float4 (4 ids that share a word); their original logits go to pfin.
  const float invT = P.invT;
  uint32_t pmask = 0u;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int b = 4 * (j * NT + tid);
    const uint32_t bits = (L.bitmap[b >> 5] >> (b & 31)) & 0xfu;
    pmask |= bits << (4 * j);
  }
  auto patched = [&](int j, int e) -> bool { return (pmask >> (4 * j + e)) & 1u; };
  if (pmask && ptab) {
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (patched(j, e)) L.pfin[slot_of(4 * (j * NT + tid) + e)] = f4_at(x[j], e);
  }
  // The slice's final values in place: unpatched values scaled (:80-81);
  // patched ones (they rejoin from pfin) and those past the slice at -inf.
  const bool part_slice = len < kFloorSlice;  // uniform
  float tmax = -__builtin_inff();
  bool nan = !ptab;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      bool out = patched(j, e);
      if (part_slice) out |= 4 * (j * NT + tid) + e >= len;
      const float v = out ? -__builtin_inff() : x[j][e] * invT;
      nan |= v != v;
      tmax = __builtin_fmaxf(tmax, v);  // (a NaN is flagged, never taken)
      x[j][e] = v;
    }
  }
  __syncthreads();  // pcnt, pbias and the original logits are in
  for (int p = tid; p < npt; p += NT) {
    float v = L.pfin[p];
    const uint32_t c = L.pcnt[p];
    if (c) {
      if (P.rp_active) v = (v > 0.0f) ? (v / P.rp32) : (v * P.rp32);  // (:71-73)
      v = v - (float)((double)c * P.freq + P.pres);                    // (:74)
    }
    if (L.pbias[p] >= 0) v = v + a.bias_vals[P.bias_off + L.pbias[p]];  // (:76)
    v = v * P.invT;                                                     // (:80-81)
    L.pfin[p] = v;
    nan |= v != v;
    tmax = __builtin_fmaxf(tmax, v);
  }
  const uint32_t wmax = wave_max_u32(f2key(tmax));
  if (lane == 0) atomicMax(&s_max, wmax);
  if (__ballot(nan) && lane == 0) s_bad = 1;
  __syncthreads();
  const float ms = key2f(s_max);
  stamp(3);
  // ---- the slice's values within the floor of its maximum ----
  auto kept = [&](float v) { return v - ms >= kGroupFloor; };
  if (!s_bad) {
    int c = 0;
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) c += kept(x[j][e]) ? 1 : 0;
    int tot;
    int pos = wave_excl_sum_small<7>(c, tot);  // c <= 64
    int base = 0;
    if (lane == 0 && tot) base = atomicAdd(&s_n, tot);
    base = __shfl(base, 0, kWave);
    if (base + tot > kFloorKeep) {
      if (lane == 0) s_bad = 1;
    } else if (c) {
      pos += base;
#pragma unroll
      for (int j = 0; j < NV; ++j) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (kept(x[j][e])) L.keep[pos++] = floor_rec(x[j][e], lo + 4 * (j * NT + tid) + e);
      }
    }
    for (int p = tid; p < npt; p += NT) {
      const float v = L.pfin[p];
      if (kept(v)) {
        const int at = atomicAdd(&s_n, 1);
        if (at < kFloorKeep)
          L.keep[at] = floor_rec(v, L.pid[p]);
        else
          s_bad = 1;
      }
    }
  }
  __syncthreads();
  stamp(4);
  // ---- publish the slice; the last of the row's slices merges ----
  const int64_t part = (int64_t)row * a.S + sl;
  const int nk = s_bad ? -1 : s_n;
  uint64_t* dst = a.part + part * kFloorKeep;
  for (int i = tid; i < nk; i += NT) store_agent(&dst[i], L.keep[i]);
  if (tid == 0) {
    store_agent(&a.part_n[part], nk);
    store_agent(&a.part_max[part], s_max);
  }
  // Release/acquire at agent scope: every thread's stores precede the
  // barrier, and so thread 0's acquire-release increment; the slice that
  // completes the count has acquired every other slice's release, and its
  // other threads follow thread 0 through the barrier.
  __syncthreads();
  if (tid == 0)
    s_last = __hip_atomic_fetch_add(&a.arrive[row], 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) ==
             (uint32_t)(a.S - 1);
  __syncthreads();
  stamp(5);
  if (!s_last) return;
  if (tid == 0) __hip_atomic_store(&a.arrive[row], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // slice records (counts and maxima) and each slice's first SP kept values,
  // read in one round; values past SP (rare) in a second
  const int SP = NT / a.S;  // >= NT / kFloorMaxSlices
  if (tid == 0) {
    s_bad = 0;
    s_max = 0u;
    s_n = 0;
  }
  __syncthreads();
  const int sj = tid / SP, si = tid - sj * SP;  // this thread's slice and value
  uint64_t spec = 0ull;
  if (sj < a.S) spec = load_agent(&a.part[((int64_t)row * a.S + sj) * kFloorKeep + si]);
  if (tid < a.S) {
    const int nj = load_agent(&a.part_n[(int64_t)row * a.S + tid]);
    s_off[tid] = nj;
    if (nj < 0 || nj > kFloorKeep) s_bad = 1;  // never trust a count past the buffer
    atomicMax(&s_max, load_agent(&a.part_max[(int64_t)row * a.S + tid]));
  }
  __syncthreads();
  stamp(6);
  const float mx = key2f(s_max);
  auto hand_on = [&]() {
    if (tid == 0) push_generic(a.generic_list, a.generic_count, row);
  };
  if (s_bad || !(mx > -__builtin_inff() && mx < __builtin_inff())) {
    hand_on();
    return;
  }
  // the row's values within the floor of its maximum: a prefix of the sort order
  uint64_t* rec = reinterpret_cast<uint64_t*>(lds);
  float* vals = reinterpret_cast<float*>(rec + kFloorMerge);
  int32_t* ids = reinterpret_cast<int32_t*>(vals + kFloorMerge);
  float* ebuf = reinterpret_cast<float*>(ids + kFloorMerge);
  auto merge = [&](uint64_t r) {
    if (key2f((uint32_t)(r >> 32)) - mx >= kGroupFloor) {
      const int at = atomicAdd(&s_n, 1);
      if (at < kFloorMerge) rec[at] = r;
    }
  };
  if (sj < a.S && si < s_off[sj]) merge(spec);
  for (int j = 0; j < a.S; ++j)
    for (int i = SP + tid; i < s_off[j]; i += NT)
      merge(load_agent(&a.part[((int64_t)row * a.S + j) * kFloorKeep + i]));
  __syncthreads();
  stamp(7);
  const int n = s_n;
  if (n > kFloorMerge) {
    hand_on();
    return;
  }
  if (n <= NT) {
    // a record's place is the number of records above it (they are distinct:
    // their indices differ); every thread reads the same record at once
    if (tid < n) {
      const uint64_t r = rec[tid];
      int rank = 0;
      for (int j = 0; j < n; ++j) rank += rec[j] > r ? 1 : 0;
      vals[rank] = key2f((uint32_t)(r >> 32));
      ids[rank] = (int32_t)~(uint32_t)r;
    }
  } else {
    int npow = 1;
    while (npow < n) npow <<= 1;
    for (int i = n + tid; i < npow; i += NT) rec[i] = 0ull;  // below every record
    __syncthreads();
    bitonic_sort_u64<NT>(rec, npow, true);
    for (int i = tid; i < n; i += NT) {
      const uint64_t r = rec[i];
      vals[i] = key2f((uint32_t)(r >> 32));
      ids[i] = (int32_t)~(uint32_t)r;
    }
  }
  __syncthreads();
  stamp(8);
  // the uniform (:117) -- the RNG state is written back only when the row is
  // finished here
  double u;
  uint64_t st[2] = {0ull, 0ull};
  if (a.d_u) {
    u = a.d_u[row];
  } else {
    st[0] = a.rng[2 * row];
    st[1] = a.rng[2 * row + 1];
    u = nim_rand_unit(st);
  }
  const TailOut to = n <= kWave ? small_tail<NT>(vals, ids, ebuf, n, P, u, &s_beyond)
                                : softmax_cutoff_draw<NT, true>(vals, ids, ebuf, n, P, u, smem, &s_beyond);
  const bool complete = n == V;
  // with neither top-p nor min-p the sort path keeps every candidate (n = V)
  const bool no_cut = !P.topp_active && !P.minp_active;
  const int n_rep = (no_cut && !complete) ? V : to.n;
  // (candidate lists asked for past the values held: the whole-row launch writes them)
  const bool lists_short = (a.dbg.cand_ids || a.dbg.cand_probs) && n_rep > n && n < a.dbg.cap;
  if (!complete && (s_beyond || lists_short)) {
    hand_on();
    return;
  }
  if (tid == 0) {
    a.out[row] = to.id;
    if (!a.d_u) {
      a.rng[2 * row] = st[0];
      a.rng[2 * row + 1] = st[1];
    }
  }
  write_debug<NT>(a.dbg, row, 3, n_rep, V, to.total, ids, ebuf);
  stamp(9);
  if (threadIdx.x == 0) NLS_STAMP_VALUE((int)blockIdx.x, 10, n);
}

hipError_t launch_floor(const FloorArgs& fa, const LaunchPlan& lp, bool vec4, hipStream_t s) {
  (void)lp;
  const dim3 grid((unsigned)(fa.B * fa.S));
  if (vec4)
    hipLaunchKernelGGL((floor_kernel<kFloorThreads, true>), grid, dim3(kFloorThreads), kFloorLds, s, fa);
  else
    hipLaunchKernelGGL((floor_kernel<kFloorThreads, false>), grid, dim3(kFloorThreads), kFloorLds, s, fa);
  return hipGetLastError();
}

hipError_t set_floor_attributes() {
  const void* fns[2] = {reinterpret_cast<const void*>(&floor_kernel<kFloorThreads, true>),
                        reinterpret_cast<const void*>(&floor_kernel<kFloorThreads, false>)};
  for (const void* f : fns) {
    const hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kFloorLds);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace nls

#ifdef NLS_PHASE_STAMPS
// floor_kernel's phase stamps, by workgroup: [4096 x 16] uint64 (host).
extern "C" int nls_floor_stamps(uint64_t* out) {
  const size_t bytes = sizeof(uint64_t) * nls::kStampRows * 16;
  return hipMemcpyFromSymbol(out, HIP_SYMBOL(nls::nls_phase_stamp), bytes) == hipSuccess ? 0 : 3;
}
#endif
