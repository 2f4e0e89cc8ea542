// nls_k64.hip -- k64_kernel: the single HBM pass for rows of greedy decoding
// (sampler.nim:77-78) or top-k with k <= 64 (:85-95), one 1024-thread
// workgroup per row, then the reference's tail (:98-121) on one wave.
//
// Phases of a workgroup:
//   1. Requests: the history ring slots, the bias entries and every wave's
//      first chunk of logits go out before the row constants are read.
//   2. Patched ids: the window's ids and the bias ids go into an LDS bitmap
//      (is an id patched?) and an LDS hash table (id -> window count, bias,
//      flags and, later, its original logit).  One pair of barriers.
//   3. First bound (top-k rows): every lane's largest unpatched value of its
//      first chunk enters a 4096-bin histogram of the keys' top 12 bits; one
//      wave finds the bin where the count from the top reaches k.  Its lowest
//      key bounds the row's k-th largest final value from below, since the k
//      values counted are final values of distinct unpatched ids.
//   4. Stream: chunks of 1024 floats, one wave each, claimed in index order
//      from an LDS counter; each wave keeps the unpatched values at or above
//      its threshold in its own LDS buffer, tightens the threshold when the
//      buffer fills, and shares bounds through an LDS atomicMax.  A patched id
//      met at or above the threshold has its original logit stored in its
//      hash slot (and its slot listed); one whose patch may raise it was
//      requested in phase 2.
//   5. End, without a barrier: each wave appends its entries at or above the
//      shared bound to one candidate list and counts itself out; the last wave
//      adds the listed patched ids' final values, selects the k members by the
//      heap rule and runs the tail.  Rows that overflow a table go to the
//      whole-row path, served by the grid's last workgroup.
#include "nls_device.h"
#include "nls_launch.h"

namespace nls {

namespace {
constexpr int kNT = kK64Threads;
constexpr int kNW = kNT / kWave;        // waves per workgroup
constexpr int kNV4 = kStreamVec4;       // float4 groups per lane and chunk
constexpr int kNE = kNV4 * 4;           // floats per lane and chunk
constexpr int kUE = kWave * kNE;        // floats per chunk
constexpr int kGS = kWave * 4;          // floats between a lane's groups
constexpr int kPER = kWaveCap / kWave;  // wave-buffer entries per lane
constexpr int kMidUnits = 3;            // chunks before every wave offers its buffer maxima
constexpr int kM0 = (kWave + kNW - 1) / kNW;  // offers per wave (kNW * kM0 >= 64 >= k)
constexpr int kHashEmpty = -1;
constexpr int kOutOfRange = 0x7ffffff0;  // buffer-load offset that reads 0 without touching memory
constexpr int kHPT = 8;                  // ring slots per thread read up front

__device__ __forceinline__ uint32_t hash_home(int id, int hbits) {
  return ((uint32_t)id * 0x9E3779B1u) >> (32 - hbits);
}
constexpr int kBootBits = 12;
constexpr int kBootBins = kK64BootBins;
static_assert(kBootBins == 1 << kBootBits && kBootBins == kWave * kWave, "64 ranges of 64 bins");
static_assert((size_t)kBootBins * 4 == kK64BootBytes && (size_t)kK64CandCap * 8 == kK64BootBytes,
              "the candidate list reuses the bootstrap histogram's bytes");
// LDS word of bootstrap bin b: bins form 64 ranges r of 64 consecutive bins
// j; the 4 bins 4q..4q+3 of range r sit at words (q * 64 + r) * 4 .. +3, so
// that the 64 lanes reading their ranges' bins 4q..4q+3 with one 16-byte
// load each cover 1 KB without bank conflicts
__device__ __forceinline__ uint32_t boot_addr(uint32_t b) {
  const uint32_t r = b >> 6, j = b & 63u;
  return ((j >> 2) * 64u + r) * 4u + (j & 3u);
}
}  // namespace

// Lanes of one wave handing values to each other through LDS: the hardware
// runs a wave's LDS instructions in order, and this fence keeps the compiler
// from moving or forwarding an LDS access across the handoff (per thread it
// would otherwise see no writer of another lane's slot).
__device__ __forceinline__ void wave_lds_sync() { __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront"); }

// Heap-rule members (sampler.nim:88-95) when ties at the k-th largest key T
// exceed k: mem[0..ge) holds every candidate >= T (ge <= 64, one per lane; gt
// of them > T).  Members = {> T} plus the m = k - gt largest indices among the
// ties whose index is at most p*, the index at which the running count of
// {>= T} in index order reaches k.  Indices are below 2^ibits.  Writes the k
// members to mem[0..k) (any order).
__device__ __forceinline__ bool tie_members(uint64_t* mem, int ge, int gt, int k, uint32_t T, int ibits) {
  const int lane = lane_id();
  const bool have = lane < ge;
  const uint64_t x = have ? mem[lane] : 0ull;
  const uint32_t idx = have ? (uint32_t)x : 0xffffffffu;
  // p*: the smallest r with at least k indices <= r
  uint32_t r = 0u;
  for (int b = ibits - 1; b >= 0; --b) {
    const uint32_t c = r | ((1u << b) - 1u);
    if ((int)__popcll(__ballot(idx <= c)) < k) r |= 1u << b;
  }
  const uint32_t pstar = r;
  const int m = k - gt;
  const bool tie = have && (uint32_t)(x >> 32) == T && idx <= pstar;
  // the m-th largest tie index: the largest q with at least m tie indices >= q
  uint32_t q = 0u;
  for (int b = ibits - 1; b >= 0; --b) {
    const uint32_t c = q | (1u << b);
    if ((int)__popcll(__ballot(tie && idx >= c)) >= m) q = c;
  }
  wave_lds_sync();
  const bool in = have && ((uint32_t)(x >> 32) > T || (tie && idx >= q));
  const uint64_t mk = __ballot(in);
  if (in) mem[(int)__popcll(mk & lanes_below())] = x;
  wave_lds_sync();
  return (int)__popcll(mk) == k;
}

// Descending rank sort of n <= 64 distinct 64-bit entries mem[0..n) (LDS,
// 16-byte aligned; what lies past n is ignored): every lane counts the entries
// above its own, reading them two at a time, then the entries move to their
// ranks in place.  Returns the entry of rank `lane` (0 past n).
__device__ __forceinline__ uint64_t rank_sort64(uint64_t* mem, int n) {
  const int lane = lane_id();
  wave_lds_sync();
  const uint64_t x = lane < n ? mem[lane] : 0ull;
  const ulonglong2* m2 = reinterpret_cast<const ulonglong2*>(mem);
  int rank = 0;
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    ulonglong2 y[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) y[j] = m2[h * 8 + j];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int i = (h * 8 + j) * 2;
      rank += (i < n && y[j].x > x) ? 1 : 0;
      rank += (i + 1 < n && y[j].y > x) ? 1 : 0;
    }
    wave_lds_sync();  // (keeps the next quarter's reads from being hoisted: 8 in flight)
  }
  wave_lds_sync();  // every lane's reads above precede these writes
  if (lane < n) mem[rank] = x;
  wave_lds_sync();
  return lane < n ? mem[lane] : 0ull;
}

// A sequential fp32 chain over buf[0..64) (LDS, 16-byte aligned) in one lane:
// buf[i] becomes init OP buf[0] OP ... OP buf[i], each step one add or
// subtraction in index order (the reference's sequential accumulation).  One
// dependent operation per step: lane 0 holds all 64 values in registers.
template <bool SUB>
__device__ __forceinline__ void chain64(float* buf, float init) {
  wave_lds_sync();  // every lane's value is in buf
  if (lane_id() == 0) {
    float4* b4 = reinterpret_cast<float4*>(buf);
    float acc = init;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float4 c[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) c[j] = b4[h * 8 + j];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        acc = SUB ? acc - c[j].x : acc + c[j].x;
        c[j].x = acc;
        acc = SUB ? acc - c[j].y : acc + c[j].y;
        c[j].y = acc;
        acc = SUB ? acc - c[j].z : acc + c[j].z;
        c[j].z = acc;
        acc = SUB ? acc - c[j].w : acc + c[j].w;
        c[j].w = acc;
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) b4[h * 8 + j] = c[j];
    }
  }
  wave_lds_sync();  // the chain's values are in buf for every lane
}

// The reference's tail on one wave: lane i holds candidate i of the k <= 64
// members in descending (value, index) order (x: key << 32 | id; 0 past k).
// Softmax (sampler.nim:98-100, :51-57), top-p (:103-108), min-p (:110-114)
// and the draw (:115-121); the three sequential fp32 sums (the softmax sum,
// the top-p running sum, the draw's subtractions) run as single-lane chains
// over `buf` (64 floats).  Past k the terms are +0, which leave a sum
// unchanged; the top-p running sum at n - 1 is also the reference's total.
__device__ __forceinline__ void k64_tail(uint64_t x, int k, const RowParams& P, double u_lane0, int row,
                                         int32_t* out, const DebugPtrs& dbg, float* buf) {
  const int lane = lane_id();
  const bool valid = lane < k;
  const int id = (int)(uint32_t)x;
  const float v = key2f((uint32_t)(x >> 32));
  const float mx = lane_f(v, 0);
  const float e = valid ? expf_cr(v - mx) : 0.0f;
  buf[lane] = e;
  chain64<false>(buf, 0.0f);
  const float ssum = buf[kWave - 1];
  wave_lds_sync();
  const float p = valid ? e / ssum : 0.0f;
  NLS_STAMP(row, 9);
  buf[lane] = p;
  chain64<false>(buf, 0.0f);
  const float cum = buf[lane];
  wave_lds_sync();
  int n = k;
  if (P.topp_active) {
    const uint64_t m = __ballot(valid && (double)cum >= P.topP);
    if (m) n = __ffsll((unsigned long long)m);
  }
  if (P.minp_active) {
    const float thr = lane_f(p, 0) * P.minP32;
    const uint64_t m = __ballot(lane >= 1 && lane < n && !(p >= thr));
    if (m) n = __ffsll((unsigned long long)m) - 1;
  }
  const float total = lane_f(cum, n - 1);
  NLS_STAMP(row, 10);
  const double u = __hiloint2double(__builtin_amdgcn_readlane(__double2hiint(u_lane0), 0),
                                    __builtin_amdgcn_readlane(__double2loint(u_lane0), 0));
  buf[lane] = p;
  chain64<true>(buf, (float)u * total);
  const float rl = buf[lane];
  wave_lds_sync();
  const uint64_t hit = __ballot(lane < n && rl <= 0.0f);
  const int pos = hit ? __ffsll((unsigned long long)hit) - 1 : n - 1;
  const int tok = __builtin_amdgcn_readlane(id, pos);
  const bool nan_c = dbg.path && __ballot(valid && v != v) != 0ull;  // a NaN candidate
  if (lane == 0) {
    out[row] = tok;
    if (dbg.n) dbg.n[row] = n;
    if (dbg.ncand) dbg.ncand[row] = k;
    if (dbg.total) dbg.total[row] = total;
    if (dbg.path) dbg.path[row] = 2 | (nan_c ? kPathNaN : 0);
  }
  if (lane < min(n, dbg.cap)) {
    if (dbg.cand_ids) dbg.cand_ids[(int64_t)row * dbg.cap + lane] = id;
    if (dbg.cand_probs) dbg.cand_probs[(int64_t)row * dbg.cap + lane] = p;
  }
}

// RK: the kinds of streamed rows the instance serves (kK64RowsAny: greedy and
// top-k, kK64RowsTopK, kK64RowsGreedy).  An instance for one kind compiles
// only that kind's code, so neither kind's registers and branches weigh on
// the other's.
template <bool VEC, int RK>
__global__ __launch_bounds__(kNT) __attribute__((amdgpu_waves_per_eu(2))) void k64_kernel(const StreamArgs a) {
  extern __shared__ __align__(16) unsigned char lds[];
  __shared__ int smem[kNW + 4];
  __shared__ uint32_t whist[kNW * kWaveBins];  // per-wave select histograms (zero between uses)
  __shared__ uint32_t s_tau;                   // the highest published bound (key)
  __shared__ uint32_t s_mid[kWave];            // buffer maxima offered after kMidUnits chunks
  __shared__ int s_midn;
  __shared__ int s_next;                       // next unclaimed chunk
  __shared__ int s_nf;                         // entries in the candidate list
  __shared__ int s_rank[kK64RankCap];          // each candidate's rank, summed over four threads
  __shared__ int s_mcnt;                       // members placed by the workgroup select
  __shared__ uint32_t s_key_k;                 // the key of rank k (the entry just past the k-th)
  __shared__ __align__(16) uint64_t s_flist[kWave];  // the last wave's candidates above its bound
  __shared__ __align__(16) float s_chain[kWave];     // the tail's chains
  __shared__ int s_npl;                        // listed patched slots
  __shared__ int s_hdist;                      // distinct ids in the hash table
  __shared__ int s_ovf;                        // the row goes to the whole-row path
  __shared__ uint32_t s_t0;
  __shared__ float s_rv[kNW];
  __shared__ int s_ri[kNW];
  __shared__ float s_x0;                       // the original logit at index 0 (greedy rows)
  __shared__ int s_last;
  __shared__ int s_pushed;
  __shared__ double s_u;

  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wv = tid >> 6;
  const int row = a.row_list ? a.row_list[blockIdx.x] : (int)blockIdx.x;
  const int len = (int)a.V;
  const int hcap = 1 << a.hbits;

  // dynamic LDS
  uint32_t* bitmap = reinterpret_cast<uint32_t*>(lds);
  size_t off = ((size_t)a.nwords * 4 + 15) & ~(size_t)15;
  int32_t* hkey = reinterpret_cast<int32_t*>(lds + off);
  uint32_t* hflag = reinterpret_cast<uint32_t*>(hkey + hcap);  // count << kPatchCountShift | flags
  float* hbias = reinterpret_cast<float*>(hflag + hcap);
  float* hraw = hbias + hcap;
  uint64_t* wbuf = reinterpret_cast<uint64_t*>(hraw + hcap);
  uint32_t* boot = reinterpret_cast<uint32_t*>(wbuf + (size_t)kNW * kWaveCap);  // bootstrap histogram
  uint64_t* cand = reinterpret_cast<uint64_t*>(boot);  // later: the candidate list (same bytes)
  int32_t* plist = reinterpret_cast<int32_t*>(boot + kK64BootBytes / 4);

  bool pushed = false;  // thread 0: this workgroup listed a row for the whole-row path
  auto run = [&]() __attribute__((always_inline)) {
    if (wv == 0) NLS_STAMP(row, 0);
    // ---- 1. requests ----
    // The history ring slots and bias entries go out first, then this wave's
    // first chunk: the patch table is built while the chunk is in flight
    // (load counters complete in issue order).  The row constants follow as
    // scalar loads (waiting for a kernel argument waits for every scalar load
    // issued before it, so they come after the requests that need only
    // arguments).  The second chunk (kNW + wv) follows the first bound: a CU
    // keeps only about 48 KB of requests in flight, and a wave asking for more
    // waits at the request, which would hold every barrier of the prologue.
    const bool ring_early = a.hcap > 0 && a.hcap <= kNT * kHPT;
    int hraw_ids[kHPT];
    {
      const __amdgpu_buffer_rsrc_t hr = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<int32_t*>(a.hist + (ring_early ? (int64_t)row * a.hcap : 0)), (short)0,
          ring_early ? a.hcap * 4 : 0, 0x00020000);
#pragma unroll
      for (int h = 0; h < kHPT; ++h) {
        const int slot = h * kNT + tid;
        hraw_ids[h] = (int)__builtin_amdgcn_raw_buffer_load_b32(hr, slot < a.hcap ? slot * 4 : kOutOfRange, 0, 0);
      }
    }
    const bool bias_early = a.bstride > 0 && a.bstride <= kNT;
    int braw;
    float bval;
    {
      const int o = tid < a.bstride ? tid * 4 : kOutOfRange;
      const int64_t base = bias_early ? (int64_t)row * a.bstride : 0;
      const int nrec = bias_early ? a.bstride * 4 : 0;
      const __amdgpu_buffer_rsrc_t bi = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<int32_t*>(a.bias_ids + base), (short)0, nrec, 0x00020000);
      const __amdgpu_buffer_rsrc_t bv = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<float*>(a.bias_vals + base), (short)0, nrec, 0x00020000);
      braw = (int)__builtin_amdgcn_raw_buffer_load_b32(bi, o, 0, 0);
      bval = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(bv, o, 0, 0));
    }
    const float* __restrict__ src = a.logits + (int64_t)row * a.V;
    const __amdgpu_buffer_rsrc_t rs = slice_rsrc(src, len);
    f32x4 R0[kNV4], R1[kNV4];
#pragma unroll
    for (int j = 0; j < kNV4; ++j) R0[j] = load_group<kGS, VEC>(rs, wv * kUE, j, lane);
    __builtin_amdgcn_sched_barrier(0);  // keep the requests here
    const RowParams P = load_const(a.rp + row);
    const int64_t hlen = load_const(a.hist_len + row);
    if (a.row_done && load_const(a.row_done + row) != 0) {  // a finished row of a batched loop
      if (tid == 0) a.out[row] = -1;
      return;
    }
    double u_in = 0.0;
    uint64_t st0 = 0ull, st1 = 0ull;
    if (a.d_u) {
      u_in = load_const(a.d_u + row);
    } else {
      st0 = load_const(a.rng + 2 * row);
      st1 = load_const(a.rng + 2 * row + 1);
    }
    // (a streamed row of a kind the instance does not serve cannot occur: the
    // host picks the instance from the rows' modes; the whole-row path would
    // take it)
    const bool served = RK == kK64RowsAny || (RK == kK64RowsGreedy) == (P.mode == kModeGreedy);
    if (P.mode == kModeFull || !P.fast || !served) {
      if (tid == 0) pushed = push_generic(a.generic_list, a.generic_count, row);
      return;
    }
    if (wv == 0) NLS_STAMP(row, 1);
    const bool greedy = RK == kK64RowsAny ? P.mode == kModeGreedy : RK == kK64RowsGreedy;
    const int k = P.k;

    // ---- 2. patched ids: bitmap and hash table ----
    int n_hist = 0;
    if (P.pen_active && hlen > 0)
      n_hist = (int)((P.repeat_last_n > 0 && P.repeat_last_n < hlen) ? P.repeat_last_n : hlen);
    const bool has_patch = n_hist > 0 || P.bias_cnt > 0;
    const int hbase = n_hist > 0 ? (int)((hlen - n_hist) % a.hcap) : 0;
    const int nw = (len + 31) >> 5;
    {
      // 16-byte stores (the bitmap's words are padded to a multiple of 4)
      const uint4 z = make_uint4(0u, 0u, 0u, 0u);
      uint4* bm4 = reinterpret_cast<uint4*>(bitmap);
      for (int w = tid; w < (nw + 3) / 4; w += kNT) bm4[w] = z;
      if (has_patch) {
        const uint4 e = make_uint4((uint32_t)kHashEmpty, (uint32_t)kHashEmpty, (uint32_t)kHashEmpty,
                                   (uint32_t)kHashEmpty);
        uint4* k4 = reinterpret_cast<uint4*>(hkey);
        uint4* f4 = reinterpret_cast<uint4*>(hflag);
        for (int h = tid; h < hcap / 4; h += kNT) {
          k4[h] = e;
          f4[h] = z;
        }
      }
      if (!greedy) {
        uint4* b4 = reinterpret_cast<uint4*>(boot);
        for (int q = tid; q < kBootBins / 4; q += kNT) b4[q] = z;
      }
      uint4* w4 = reinterpret_cast<uint4*>(whist);
      for (int q = tid; q < kNW * kWaveBins / 4; q += kNT) w4[q] = z;
    }
    if (tid < kWave) s_mid[tid] = 0u;
    if (tid < kK64RankCap) s_rank[tid] = 0;
    if (tid == 0) {
      s_tau = 0u;
      s_midn = 0;
      s_next = 2 * kNW;
      s_nf = 0;
      s_npl = 0;
      s_hdist = 0;
      s_ovf = 0;
      s_x0 = 0.0f;
      s_t0 = 0u;
      s_pushed = 0;
    }
    if (!bias_early && P.bias_cnt > 0 && P.bias_cnt <= kNT) {
      const int o = tid < P.bias_cnt ? tid * 4 : kOutOfRange;
      const __amdgpu_buffer_rsrc_t bi = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<int32_t*>(a.bias_ids + P.bias_off), (short)0, P.bias_cnt * 4, 0x00020000);
      const __amdgpu_buffer_rsrc_t bv = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<float*>(a.bias_vals + P.bias_off), (short)0, P.bias_cnt * 4, 0x00020000);
      braw = (int)__builtin_amdgcn_raw_buffer_load_b32(bi, o, 0, 0);
      bval = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(bv, o, 0, 0));
    }
    __syncthreads();
    if (wv == 0) NLS_STAMP(row, 2);
    // hash slot of a patched id (inserting it when `insert`); -1 when the
    // table is full, or for an insert that has probed 8 slots of a table past
    // its load limit (the row is handed on then, so a long window stops early
    // instead of probing a full table)
    auto hash_slot = [&](int id, bool insert) -> int {
      uint32_t h = hash_home(id, a.hbits);
      for (int probe = 0; probe < hcap; ++probe) {
        if (insert && probe == 8 && s_hdist > hcap - hcap / 4) return -1;
        int cur;
        if (insert) {
          cur = atomicCAS(&hkey[h], kHashEmpty, id);
          if (cur == kHashEmpty) {
            atomicAdd(&s_hdist, 1);
            return (int)h;
          }
        } else {
          cur = hkey[h];
          if (cur == kHashEmpty) return -1;
        }
        if (cur == id) return (int)h;
        h = (h + 1) & (uint32_t)(hcap - 1);
      }
      return -1;
    };
    if (has_patch) {
      // Window entries (ring slot s holds entry (s - hbase) mod hcap).  A
      // history repeats ids, so the wave's lanes holding one id are grouped
      // first (one ballot per bit of the id) and only the group's first lane
      // touches the tables, adding the group's size: same-address LDS atomics
      // would serialise.
      const int id_bits = 32 - __clz(len > 1 ? len - 1 : 1);
      auto add_window = [&](int id, bool in) {  // every lane of the wave calls it
        in = in && id >= 0 && id < len;  // out-of-range ids are stored as -1 (sampler.nim:70)
        uint64_t m = __ballot(in);
        if (m == 0ull) return;  // wave-uniform
        for (int b = 0; b < id_bits; ++b) {
          const bool bit = (id >> b) & 1;
          const uint64_t bal = __ballot(bit);
          m &= bit ? bal : ~bal;
        }
        if (in && (m & lanes_below()) == 0ull) {
          atomicOr(&bitmap[id >> 5], 1u << (id & 31));
          const int h = hash_slot(id, true);
          if (h < 0)
            s_ovf = 1;
          else
            atomicAdd(&hflag[h], (uint32_t)__popcll(m) << kPatchCountShift);
        }
      };
      if (ring_early) {
#pragma unroll
        for (int h = 0; h < kHPT; ++h) {
          const int slot = h * kNT + tid;
          int i = slot - hbase;
          if (i < 0) i += a.hcap;
          if (h * kNT < a.hcap) add_window(hraw_ids[h], n_hist > 0 && slot < a.hcap && i < n_hist);
        }
      } else {
        const int32_t* __restrict__ hrow = a.hist + (int64_t)row * a.hcap;
        for (int i0 = 0; i0 < n_hist; i0 += kNT) {
          const int i = i0 + tid;
          int slot = hbase + i;
          if (slot >= a.hcap) slot -= a.hcap;
          add_window(i < n_hist ? hrow[slot] : -1, i < n_hist);
        }
      }
      auto add_bias = [&](int id, float val) {
        if (id < 0 || id >= len) return;
        atomicOr(&bitmap[id >> 5], 1u << (id & 31));
        const int h = hash_slot(id, true);
        if (h < 0) {
          s_ovf = 1;
          return;
        }
        hbias[h] = val;  // bias ids are unique per row
        atomicOr(&hflag[h], (uint32_t)kPatchBias | (!(val <= 0.0f) ? (uint32_t)kPatchRise : 0u));
      };
      if (P.bias_cnt <= kNT) {
        if (tid < P.bias_cnt) add_bias(braw, bval);
      } else {
        for (int j = tid; j < P.bias_cnt; j += kNT) add_bias(a.bias_ids[P.bias_off + j], a.bias_vals[P.bias_off + j]);
      }
    }
    __syncthreads();
    if (wv == 0) NLS_STAMP(row, 3);
    if (wv == 0) NLS_DETAIL_STAMP(row, 0);
    const bool ovf = s_ovf != 0 || s_hdist > hcap - hcap / 4;  // uniform
    auto patched = [&](int loc) -> bool { return has_patch && ((bitmap[loc >> 5] >> (loc & 31)) & 1u); };
    // Penalties of the raising sign make every windowed id a possible riser;
    // otherwise only a positive (or NaN) bias raises a logit.  Every other
    // patch lowers it, in float rounding too (division of a positive value
    // by rp >= 1, multiplication of a non-positive one, subtraction of
    // cnt * freq + pres >= 0, a bias <= 0), and so does the temperature.
    const bool row_rise = (P.rp_active && !(P.rp32 >= 1.0f)) || !(P.freq >= 0.0) || !(P.pres >= 0.0);
    auto may_rise = [&](uint32_t fl) -> bool {
      return (fl & kPatchRise) || (row_rise && (fl >> kPatchCountShift) > 0);
    };
    // List a slot for the final evaluation (once per slot).
    auto list_slot = [&](int h) {
      const int i = atomicAdd(&s_npl, 1);
      if (i < kK64PListCap)
        plist[i] = h;
      else
        s_ovf = 1;
    };
    // Risers: their original logits are requested now, the slots listed.
    constexpr int kRPT = kK64MaxHash / kNT;
    float rr[kRPT];
#pragma unroll
    for (int r = 0; r < kRPT; ++r) {
      const int h = tid + r * kNT;
      bool want = false;
      int id = 0;
      if (has_patch && !ovf && h < hcap) {
        id = hkey[h];
        want = id != kHashEmpty && may_rise(hflag[h]);
      }
      rr[r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, want ? id * 4 : kOutOfRange, 0, 0));
      if (want) list_slot(h);
    }
    // Patched id met at or above the threshold (top-k) or above the lane's
    // best (greedy): its original logit goes to its slot, listed once.
    auto capture = [&](int loc, float raw) {
      const int h = hash_slot(loc, false);
      if (h < 0) {
        s_ovf = 1;
        return;
      }
      hraw[h] = raw;  // every writer stores the same value
      const uint32_t old = atomicOr(&hflag[h], (uint32_t)kPatchSeen);
      if (!(old & kPatchSeen) && !may_rise(old)) list_slot(h);
    };

    // ---- 3./4. the stream ----
    float bv = -__builtin_inff();  // greedy: the lane's running argmax
    int bi = 0x7fffffff;
    int wn = 0;                     // entries in this wave's buffer
    uint32_t wtau = 0u;             // this wave's threshold (key)
    bool wovf = false;
    int nu = 0;
    uint64_t* wb = wbuf + (size_t)wv * kWaveCap;
    uint32_t* wh = whist + wv * kWaveBins;
    const int nunits = (len + kUE - 1) / kUE;

    auto process = [&](float (&v)[kNE], int t, bool first) __attribute__((always_inline)) {
      const int toff = t * kUE;
      const bool full = toff + kUE <= len;
      int obase = toff + lane * 4;
      asm volatile("" : "+v"(obase));
      auto loc_of = [&](int q) -> int { return obase + (q >> 2) * kGS + (q & 3); };
      auto valid = [&](int q) -> bool {
        const int o = obase + (q >> 2) * kGS;
        return full || (VEC ? o < len : o + (q & 3) < len);
      };
      if (greedy) {
        // argmax (:45-49): one pass over the lane's values in index order
        // keeps the first of the largest unpatched ones (strict >), which is
        // then merged into the lane's running best.  Every lane of a wave
        // runs it on every chunk: with 64 lanes some lane nearly always
        // improves, so a per-lane gate would save nothing.  (A NaN is never
        // taken; -inf only when nothing larger is met, as index 0's rule
        // below and argmax_merge arrange.)
        if (first && tid == 0) s_x0 = v[0];
        uint32_t pm = 0u;  // bit q: value q is patched (one bitmap word per float4 group)
        if (has_patch) {
#pragma unroll
          for (int j = 0; j < kNV4; ++j) {
            const int o = obase + j * kGS;
            pm |= ((bitmap[min(o, len - 1) >> 5] >> (o & 31)) & 15u) << (4 * j);
          }
        }
        const float b0 = bv;  // the lane's best before this chunk
        const bool none = bi == 0x7fffffff;  // (no best yet: b0 is -inf and stands for no element)
        float cv = -__builtin_inff();
        int cq = -1;
#pragma unroll
        for (int q = 0; q < kNE; ++q) {
          const bool ok = valid(q) && !((pm >> q) & 1u);
          if (ok && v[q] > cv) {
            cv = v[q];
            cq = q;
          }
        }
        if (cq < 0) {
          // nothing above -inf: the first unpatched -inf, if any
#pragma unroll
          for (int q = kNE - 1; q >= 0; --q)
            if (valid(q) && !((pm >> q) & 1u) && v[q] == cv) cq = q;
        }
        if (cq >= 0) argmax_merge(bv, bi, cv, obase + (cq >> 2) * kGS + (cq & 3));
        // A patched id's original logit is captured when it beats the
        // earlier best (or equals -inf with none yet).  The others cannot
        // win: a non-riser's final value is at most its original logit
        // (risers are listed already), and that best's index is smaller,
        // since a lane meets its elements in index order.  (A NaN cannot
        // win either.)
        if (pm) {
          auto want = [&](int q) -> bool {
            return ((pm >> q) & 1u) && valid(q) && (v[q] > b0 || (none && v[q] == b0));
          };
          bool cap = false;
#pragma unroll
          for (int q = 0; q < kNE; ++q) cap |= want(q);
          if (cap) {
#pragma unroll
            for (int q = 0; q < kNE; ++q)
              if (want(q)) capture(loc_of(q), v[q]);
          }
        }
        return;
      }
      float sv[kNE];
#pragma unroll
      for (int q = 0; q < kNE; ++q) sv[q] = v[q] * P.invT;  // (:80-81)
      if (!first && nu++ == kMidUnits - 1) {
        // After its first kMidUnits chunks every wave offers the kM0 largest
        // keys of its buffer; the wave completing the set publishes the k-th
        // largest of all offers (an offer not yet written reads 0, which only
        // lowers the bound).
        uint32_t kr[kPER];
#pragma unroll
        for (int j = 0; j < kPER; ++j) {
          const int i = lane + j * kWave;
          kr[j] = i < wn ? (uint32_t)(wb[i] >> 32) : 0u;
        }
#pragma unroll
        for (int i = 0; i < kM0; ++i) {
          uint32_t lm = 0u;
#pragma unroll
          for (int j = 0; j < kPER; ++j) lm = max(lm, kr[j]);
          const uint32_t m = wave_max_u32(lm);
          const uint64_t at = __ballot(lm == m);
          if (lane == __ffsll((unsigned long long)at) - 1) {
            bool done = false;
#pragma unroll
            for (int j = 0; j < kPER; ++j)
              if (!done && kr[j] == m) {
                kr[j] = 0u;
                done = true;
              }
          }
          if (lane == 0) s_mid[wv * kM0 + i] = m;
        }
        int prev = 0;
        if (lane == 0) prev = atomicAdd(&s_midn, 1);
        if (__builtin_amdgcn_readfirstlane(prev) == kNW - 1) {
          const uint32_t t2 = wave_kth_largest(lane < kNW * kM0 ? s_mid[lane] : 0u, k);
          wtau = max(wtau, t2);
          if (lane == 0) atomicMax(&s_tau, t2);
        }
      }
      wtau = max(wtau, __hip_atomic_load(&s_tau, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
      float thr_f = key2f(wtau);
      int npf = 0;  // values passing the float prefilter, over the wave
#pragma unroll
      for (int q = 0; q < kNE; ++q) npf += __popcll(__ballot(valid(q) && !(sv[q] < thr_f)));
      if (npf == 0) return;
      if (wn + npf > kWaveCap) {
        // raise the threshold to the k-th largest of the per-lane top-2 of
        // everything this wave has seen (buffer + chunk), then compact
        uint32_t tops[2] = {0u, 0u};
        int nm = 0;
#pragma unroll
        for (int j = 0; j < kPER; ++j) {
          const int i = lane + j * kWave;
          if (i < wn) {
            topq_insert<2>(tops, (uint32_t)(wb[i] >> 32));
            ++nm;
          }
        }
#pragma unroll
        for (int q = 0; q < kNE; ++q) {
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
                     k, k + k / 2, wh)
                     .tau;
          thr_f = key2f(wtau);
        }
        uint64_t xs[kPER];
        int keep = 0;
#pragma unroll
        for (int j = 0; j < kPER; ++j) {
          const int i = lane + j * kWave;
          xs[j] = (i < wn) ? wb[i] : 0ull;
          keep += (i < wn && (uint32_t)(xs[j] >> 32) >= wtau);
        }
        int ktot;
        int pos = wave_excl_sum_small<3>(keep, ktot);
#pragma unroll
        for (int j = 0; j < kPER; ++j) {
          const int i = lane + j * kWave;
          if (i < wn && (uint32_t)(xs[j] >> 32) >= wtau) wb[pos++] = xs[j];
        }
        wn = ktot;
        npf = 0;
#pragma unroll
        for (int q = 0; q < kNE; ++q) npf += __popcll(__ballot(valid(q) && !(sv[q] < thr_f)));
        if (wn + npf > kWaveCap) {
          wovf = true;  // ties or an adversarial order crowd the buffer
          return;
        }
      }
      // append every unpatched value >= the threshold
#pragma unroll
      for (int q = 0; q < kNE; ++q) {
        if (__ballot(valid(q) && !(sv[q] < thr_f)) == 0ull) continue;
        const uint32_t kq = f2key(sv[q]);
        const bool pass = valid(q) && kq >= wtau;
        const bool pat = pass && patched(loc_of(q));
        if (pat) capture(loc_of(q), v[q]);
        const bool keep = pass && !pat;
        const uint64_t m = __ballot(keep);
        if (keep) wb[wn + (int)__popcll(m & lanes_below())] = ((uint64_t)kq << 32) | (uint32_t)loc_of(q);
        wn += (int)__popcll(m);
      }
      if (wn >= 2 * k + kWave) {
        // tighten to the k-th largest of the buffer
        uint64_t xs[kPER];
#pragma unroll
        for (int j = 0; j < kPER; ++j) {
          const int i = lane + j * kWave;
          xs[j] = (i < wn) ? wb[i] : 0ull;
        }
        const int n0 = wn;
        const SelectResult r = wave_select(
            [&](auto fn) {
#pragma unroll
              for (int j = 0; j < kPER; ++j) fn((uint32_t)(xs[j] >> 32), lane + j * kWave < n0);
            },
            k, k + k / 4, wh);
        int keep = 0;
#pragma unroll
        for (int j = 0; j < kPER; ++j) keep += (lane + j * kWave < n0 && (uint32_t)(xs[j] >> 32) >= r.tau);
        int ktot;
        int pos = wave_excl_sum_small<3>(keep, ktot);
#pragma unroll
        for (int j = 0; j < kPER; ++j)
          if (lane + j * kWave < n0 && (uint32_t)(xs[j] >> 32) >= r.tau) wb[pos++] = xs[j];
        wn = ktot;
        wtau = r.tau;
        if (lane == 0) atomicMax(&s_tau, wtau);
      }
    };

    // first chunk: the bootstrap bound of top-k rows
    float v0[kNE];
#pragma unroll
    for (int j = 0; j < kNV4; ++j) {
      v0[4 * j + 0] = R0[j].x;
      v0[4 * j + 1] = R0[j].y;
      v0[4 * j + 2] = R0[j].z;
      v0[4 * j + 3] = R0[j].w;
    }
    if (wv == 0) {
      __builtin_amdgcn_s_waitcnt(0);  // (the phases build: the first chunk is in)
      NLS_DETAIL_STAMP(row, 1);
    }
    if (!greedy && !ovf) {
      // this lane's largest unpatched value (float domain: v_max_f32 returns
      // one of its operands, so the maximum is one of the lane's own values)
      const int obase = wv * kUE + lane * 4;
      float fmx = -__builtin_inff();
      bool any = false;
#pragma unroll
      for (int j = 0; j < kNV4; ++j) {
        const int o = obase + j * kGS;
        const uint32_t pb = has_patch ? bitmap[min(o, len - 1) >> 5] >> (o & 31) : 0u;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bool ok = (VEC ? o < len : o + e < len) && !((pb >> e) & 1u);
          const float x = v0[4 * j + e] * P.invT;
          any |= ok;
          fmx = ok ? __builtin_fmaxf(fmx, x) : fmx;
        }
      }
      // (a lane whose values are all NaN offers nothing: fmax skips NaN)
      if (any && fmx == fmx) atomicAdd(&boot[boot_addr(f2key(fmx) >> (32 - kBootBits))], 1u);
    }
    if (wv == 0) NLS_DETAIL_STAMP(row, 2);
    __syncthreads();
    if (wv == 0) NLS_DETAIL_STAMP(row, 3);
    if (!greedy && !ovf && wv == 0) {
      // The highest bin at which the count from the top reaches k.  Bins
      // form 64 ranges of 64; lane l sums range 63 - l (largest first), the
      // lanes' scan finds the range, and its 64 bins, one per lane from the
      // top, are scanned again for the bin.
      const int range = kWave - 1 - lane;
      int c = 0;
      const uint4* b4 = reinterpret_cast<const uint4*>(boot);
#pragma unroll
      for (int q = 0; q < kWave / 4; ++q) {
        const uint4 v = b4[q * kWave + range];
        c += (int)(v.x + v.y + v.z + v.w);
      }
      const int incl = wave_incl_scan(c);
      const uint64_t mk = __ballot(incl - c < k && incl >= k);
      if (mk) {
        const int sl = __ffsll((unsigned long long)mk) - 1;
        const int above = __builtin_amdgcn_readlane(incl - c, sl);
        const int r = kWave - 1 - sl;
        const int off = kWave - 1 - lane;  // this lane's bin of range r, from the top
        const int cb = (int)boot[boot_addr((uint32_t)(r * kWave + off))];
        const int inc2 = wave_incl_scan(cb) + above;
        const uint64_t m2 = __ballot(inc2 - cb < k && inc2 >= k);
        const int l2 = __ffsll((unsigned long long)m2) - 1;
        if (lane == 0) s_t0 = (uint32_t)(r * kWave + (kWave - 1 - l2)) << (32 - kBootBits);
      }
    }
    __syncthreads();
    if (wv == 0) NLS_STAMP(row, 4);
    // the second chunk (requested now: see above)
#pragma unroll
    for (int j = 0; j < kNV4; ++j) R1[j] = load_group<kGS, VEC>(rs, (kNW + wv) * kUE, j, lane);
    if (!greedy) {
      wtau = s_t0;
      if (tid == 0) s_tau = s_t0;
    }
    // the riser logits requested above are in by now
#pragma unroll
    for (int r = 0; r < kRPT; ++r) {
      const int h = tid + r * kNT;
      if (has_patch && !ovf && h < hcap && hkey[h] != kHashEmpty && may_rise(hflag[h])) hraw[h] = rr[r];
    }
    if (!ovf) {
      int t = wv;
      auto stop = [&]() -> bool { return __builtin_amdgcn_readfirstlane((int)wovf) != 0; };
      process(v0, t, true);
      t = kNW + wv;
      if (!stop() && t < nunits) {
        for (;;) {
          int c = 0;
          if (lane == 0) c = atomicAdd(&s_next, 1);
          const int tn = __builtin_amdgcn_readfirstlane(c);
          float v[kNE];
#pragma unroll
          for (int j = 0; j < kNV4; ++j) {
            v[4 * j + 0] = R1[j].x;
            v[4 * j + 1] = R1[j].y;
            v[4 * j + 2] = R1[j].z;
            v[4 * j + 3] = R1[j].w;
            R1[j] = load_group<kGS, VEC>(rs, tn * kUE, j, lane);
          }
          process(v, t, false);
          if (stop() || tn >= nunits) break;
          t = tn;
        }
      }
    }

    // ---- 5. end: every wave hands in its part, then the workgroup finishes the row ----
    NLS_WAVE_STAMP(row, wv);
    if (greedy) {
      wave_argmax(bv, bi);
      if (lane == 0) {
        s_rv[wv] = bv;
        s_ri[wv] = bi;
      }
    } else if (!ovf && !wovf) {
      // this wave's entries at or above the shared bound join the candidate list
      const uint32_t g = max(wtau, __hip_atomic_load(&s_tau, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
      uint64_t xs[kPER];
      int c = 0;
#pragma unroll
      for (int j = 0; j < kPER; ++j) {
        const int i = lane + j * kWave;
        xs[j] = i < wn ? wb[i] : 0ull;
        c += (i < wn && (uint32_t)(xs[j] >> 32) >= g);
      }
      int tot;
      int pos = wave_excl_sum_small<3>(c, tot);
      int base = 0;
      if (lane == 0 && tot) base = atomicAdd(&s_nf, tot);
      base = __builtin_amdgcn_readfirstlane(base);
      if (base + tot > kK64CandCap) {
        if (lane == 0) s_ovf = 1;
      } else {
        pos += base;
#pragma unroll
        for (int j = 0; j < kPER; ++j) {
          const int i = lane + j * kWave;
          if (i < wn && (uint32_t)(xs[j] >> 32) >= g) cand[pos++] = xs[j];
        }
      }
    }
    if (wovf && lane == 0) s_ovf = 1;
    __syncthreads();  // every wave's stream, captures and candidates are in
    NLS_STAMP(row, 5);

    auto patched_final = [&](int h, float v) -> float {  // (:71-76, then :80-81)
      const uint32_t fl = hflag[h];
      const uint32_t cnt = fl >> kPatchCountShift;
      if (cnt) {
        if (P.rp_active) v = (v > 0.0f) ? (v / P.rp32) : (v * P.rp32);
        v = v - (float)((double)cnt * P.freq + P.pres);  // float64, one rounding (:74)
      }
      if (fl & kPatchBias) v = v + hbias[h];
      if (!greedy) v = v * P.invT;
      return v;
    };
    const int npl = min(s_npl, kK64PListCap);
    if (greedy) {
      if (wv != 0) return;
      float rv = s_rv[0];
      int ri = s_ri[0];
#pragma unroll
      for (int w = 1; w < kNW; ++w) argmax_merge(rv, ri, s_rv[w], s_ri[w]);
      // listed patched ids (met above a lane's best, or risers)
      float pv = -__builtin_inff();
      int pi = 0x7fffffff;
      for (int i = lane; i < npl; i += kWave) {
        const int h = plist[i];
        argmax_merge(pv, pi, patched_final(h, hraw[h]), hkey[h]);
      }
      wave_argmax(pv, pi);
      argmax_merge(rv, ri, pv, pi);
      if (ovf || s_ovf != 0) {
        if (lane == 0) {
          s_pushed = 1;
          push_generic(a.generic_list, a.generic_count, row);
        }
        return;
      }
      // argmax (:45-49) starts from index 0: a NaN there keeps the answer 0
      float x0 = s_x0;
      if (patched(0)) {
        const int h0 = hash_slot(0, false);
        if (h0 >= 0) x0 = patched_final(h0, x0);
      }
      if (lane == 0) {
        a.out[row] = (x0 != x0) ? 0 : ri;
        if (a.dbg.n) a.dbg.n[row] = 0;
        if (a.dbg.ncand) a.dbg.ncand[row] = 0;
        if (a.dbg.total) a.dbg.total[row] = 0.0f;
        if (a.dbg.path) a.dbg.path[row] = 1;
      }
      return;
    }
    // Top-k rows.  The listed patched ids whose final value reaches the
    // shared bound join the list (split over the workgroup).
    const uint32_t g = __hip_atomic_load(&s_tau, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (!ovf && s_ovf == 0) {
      for (int i = tid; i < npl; i += kNT) {
        const int h = plist[i];
        const uint32_t kp = f2key(patched_final(h, hraw[h]));
        if (kp >= g) {
          const int j = atomicAdd(&s_nf, 1);
          if (j < kK64CandCap)
            cand[j] = ((uint64_t)kp << 32) | (uint32_t)hkey[h];
          else
            s_ovf = 1;
        }
      }
    }
    __syncthreads();
    const int N = s_nf;
    const int kk = k;
    const bool rank_ok = !ovf && s_ovf == 0 && N >= kk && N <= kK64RankCap;  // uniform
    if (rank_ok) {
      // Ranks in descending (value, index) order: candidate c's count of
      // larger entries, summed over four threads each scanning a quarter of
      // the list.  (The list entries are distinct: no id enters it twice.)
      const int c = tid & (kK64RankCap - 1);
      const int seg = tid / kK64RankCap;  // uniform over a wave
      const int lo = seg * N / 4, hi = (seg + 1) * N / 4;
      if (c < N) {
        const uint64_t x = cand[c];
        int r = 0;
#pragma unroll 8
        for (int i = lo; i < hi; ++i) r += cand[i] > x ? 1 : 0;  // one LDS broadcast per entry
        atomicAdd(&s_rank[c], r);
      }
    }
    __syncthreads();
    if (rank_ok && tid < N) {
      const int r = s_rank[tid];
      if (r < kWave) s_flist[r] = cand[tid];
      if (r == k) s_key_k = (uint32_t)(cand[tid] >> 32);  // (ranks run over 0..N-1)
    }
    // A list longer than the rank table (a flat top of the row: many values
    // near the k-th): the heap rule's k members by a workgroup radix select
    // over the list, into the wave buffers (free now).
    bool sel_done = false;
    if (!ovf && s_ovf == 0 && N > kK64RankCap && N >= kk) {  // uniform
      if (tid == 0) s_mcnt = 0;
      __syncthreads();
      sel_done = topk_members<kNT>(cand, N, kk, wbuf, kNW * kWaveCap, whist, smem, &s_mcnt);  // uniform
      if (sel_done && tid < kk) s_flist[tid] = wbuf[tid];
    }
    __syncthreads();
    NLS_STAMP(row, 6);
    if (wv != 0) return;
    // wave 0: the members in order; ties at the k-th value beyond k take the
    // heap rule's closed form
    bool rovf = !rank_ok && !sel_done;
    uint64_t x = 0ull;
    if (sel_done) {
      x = rank_sort64(s_flist, kk);
    } else if (!rovf) {
      const int nl = min(N, kWave);  // s_flist[0..nl) holds ranks 0..nl-1
      x = lane < nl ? s_flist[lane] : 0ull;
      const uint32_t T = (uint32_t)__builtin_amdgcn_readlane((int)(x >> 32), kk - 1);
      // ties at the k-th key beyond k: the key of rank k (held in the wave
      // for k < 64, else read from LDS) equals it
      const uint32_t key_k = kk < kWave ? (uint32_t)__builtin_amdgcn_readlane((int)(x >> 32), kk) : s_key_k;
      const bool excess = N > kk && key_k == T;
      if (excess) {
        const uint32_t kx = (uint32_t)(x >> 32);
        const int ge = (int)__popcll(__ballot(lane < nl && kx >= T));
        const int gt = (int)__popcll(__ballot(lane < nl && kx > T));
        // all entries >= T must lie within the 64 ranks held
        if (ge == nl && N > nl) {
          rovf = true;
        } else if (tie_members(s_flist, ge, gt, kk, T, 32 - __clz(len > 1 ? len - 1 : 1))) {
          x = rank_sort64(s_flist, kk);
        } else {
          rovf = true;
        }
      } else if (lane >= kk) {
        x = 0ull;
      }
    }
    NLS_STAMP(row, 7);
    if (!rovf) {
      NLS_STAMP_VALUE(row, 12, N);
      NLS_STAMP_VALUE(row, 13, npl);
      NLS_STAMP_VALUE(row, 14, s_t0);
      NLS_STAMP_VALUE(row, 15, g);
      NLS_STAMP(row, 8);
      double u = 0.0;
      if (lane == 0) u = take_uniform(a.d_u, u_in, st0, st1, a.rng, row);
      k64_tail(x, kk, P, u, row, a.out, a.dbg, s_chain);
      NLS_STAMP(row, 11);
      return;
    }
    // Many candidates (an adversarial order) or a table overflow: the
    // whole-row path takes the row.
    if (lane == 0) {
      s_pushed = 1;
      push_generic(a.generic_list, a.generic_count, row);
    }
  };
  run();
  if (a.gen_inline) {
    // The last workgroup to finish serves the rows handed on to the
    // whole-row path.  A workgroup that listed a row publishes it with a
    // release increment of `done` (its lister's store happens before the
    // barrier below); thread 0 of the last workgroup acquires.
    __syncthreads();
    if (threadIdx.x == 0) {
      const bool pub = pushed || s_pushed;
      const uint32_t prev =
          pub ? __hip_atomic_fetch_add(a.done, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT)
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
      generic_rows<kNT>(a.ga, 0, 1, count, whist, dl, dl + 256, smem, &s_u, reinterpret_cast<int*>(dl + 512),
                        s_rv, s_ri);
    }
  }
}

template <bool VEC>
static void launch_k64_rows(const StreamArgs& a, const LaunchPlan& p, hipStream_t s) {
  const dim3 grid(a.row_list ? a.n_list : a.B);
  switch (p.k64_rows) {
    case kK64RowsTopK:
      hipLaunchKernelGGL((k64_kernel<VEC, kK64RowsTopK>), grid, dim3(kNT), p.lds, s, a);
      break;
    case kK64RowsGreedy:
      hipLaunchKernelGGL((k64_kernel<VEC, kK64RowsGreedy>), grid, dim3(kNT), p.lds, s, a);
      break;
    default:
      hipLaunchKernelGGL((k64_kernel<VEC, kK64RowsAny>), grid, dim3(kNT), p.lds, s, a);
  }
}

hipError_t launch_k64(const StreamArgs& a, const LaunchPlan& p, hipStream_t s) {
  if (p.vec4)
    launch_k64_rows<true>(a, p, s);
  else
    launch_k64_rows<false>(a, p, s);
  return hipGetLastError();
}

template <bool VEC, int RK>
static hipError_t set_k64_attr() {
  return hipFuncSetAttribute(reinterpret_cast<const void*>(&k64_kernel<VEC, RK>),
                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)kK64MaxDynLds);
}

hipError_t set_k64_attributes() {
  hipError_t e;
  if ((e = set_k64_attr<true, kK64RowsAny>()) != hipSuccess) return e;
  if ((e = set_k64_attr<true, kK64RowsTopK>()) != hipSuccess) return e;
  if ((e = set_k64_attr<true, kK64RowsGreedy>()) != hipSuccess) return e;
  if ((e = set_k64_attr<false, kK64RowsAny>()) != hipSuccess) return e;
  if ((e = set_k64_attr<false, kK64RowsTopK>()) != hipSuccess) return e;
  return set_k64_attr<false, kK64RowsGreedy>();
}

}  // namespace nls

#ifdef NLS_PHASE_STAMPS
// which = 0: phase stamps, 1: wave stamps; out: [4096 x 16] uint64 (host).
extern "C" int nls_phase_stamps(int which, uint64_t* out) {
  const size_t bytes = sizeof(uint64_t) * nls::kStampRows * 16;
  const hipError_t e = which == 2 ? hipMemcpyFromSymbol(out, HIP_SYMBOL(nls::nls_detail_stamp), bytes)
                      : which ? hipMemcpyFromSymbol(out, HIP_SYMBOL(nls::nls_wave_stamp), bytes)
                              : hipMemcpyFromSymbol(out, HIP_SYMBOL(nls::nls_phase_stamp), bytes);
  return e == hipSuccess ? 0 : 3;
}
#endif
