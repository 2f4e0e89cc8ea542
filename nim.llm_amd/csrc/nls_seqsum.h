// nls_seqsum.h -- the reference's sequential fp32 sum, s = ((0 + e0) + e1) +
// ... + e_{n-1} with round-to-nearest-even at every step, evaluated by a whole
// workgroup, bit for bit.
//
// softmaxInPlace (sampler.nim:54-56) adds the row's exponentials one at a time
// in index order; on a GPU a chain of V dependent adds on one lane costs ~4
// cycles each.  The terms here are >= 0, so the running sum only grows, and it
// stays in one binade [2^E, 2^(E+1)) for long stretches.  There every float is
// S * u with u = 2^(E-23) and S an integer in [2^23, 2^24) (the subnormal
// range and zero count as E = -126, u = 2^-149, S < 2^24), and while
// s + e < 2^(E+1)
//     fl(s + e) = u * RNE(S + e/u).
// With e/u = I + f (I an integer, 0 <= f < 1; exact, u being a power of two)
// the step adds I + [f > 1/2] to S, independently of S -- except for a tie,
// f == 1/2, which adds I + [(S + I) odd] and leaves S even.  So a run of terms
// acts on S as a map of S's parity alone: for each incoming parity, the total
// increment and the outgoing parity.  These maps compose associatively, so a
// workgroup scans them in index order, each thread finds its exact incoming S,
// and the one thread whose terms take S to 2^24 (or hold a term too large or
// not a number) replays them to find that term, which is added on its own as
// an ordinary fp32 add.  The scan then resumes in the new binade.  The window
// of terms scanned at once starts at one per thread, doubles after every
// window without a binade change and, after a change at term k of the sum,
// covers about k terms (alike terms double the sum again around term 2k), so
// the early changes (the sum grows quickly at first) cost little.
#pragma once
#include <stdint.h>
#include <string.h>
#if defined(__HIPCC__)
#include "nls_primitives.h"
#define NLS_SEQ_HD __host__ __device__
#else
#define NLS_SEQ_HD
#endif

namespace nls {

constexpr int kSeqSat = 1 << 26;  // increments saturate here (no binade holds 2^24 steps of u)
constexpr int kSeqMaxJ = 16;      // terms per thread in one window
// The first terms of a sum are added one at a time by one lane: while the sum
// is a few terms large it changes binade every few terms, and each change
// would end a window of the workgroup scan.
constexpr int kSeqSerial = 1024;

// A parity map, packed: a = (d0 << 1) | p0 and c = (d1 << 1) | p1, where d_p
// is the increment of S for incoming parity p (saturating at kSeqSat) and p_p
// the outgoing parity.
struct SeqMap {
  int a, c;
};

NLS_SEQ_HD inline SeqMap sm_identity() { return SeqMap{0, 1}; }

NLS_SEQ_HD inline SeqMap sm_make(int d0, int p0, int d1, int p1) {
  d0 = d0 < kSeqSat ? d0 : kSeqSat;
  d1 = d1 < kSeqSat ? d1 : kSeqSat;
  return SeqMap{(d0 << 1) | p0, (d1 << 1) | p1};
}

// map x, then map y
NLS_SEQ_HD inline SeqMap sm_then(SeqMap x, SeqMap y) {
  const int ya = (x.a & 1) ? y.c : y.a;
  const int yc = (x.c & 1) ? y.c : y.a;
  int da = (x.a >> 1) + (ya >> 1), dc = (x.c >> 1) + (yc >> 1);
  da = da < kSeqSat ? da : kSeqSat;
  dc = dc < kSeqSat ? dc : kSeqSat;
  return SeqMap{(da << 1) | (ya & 1), (dc << 1) | (yc & 1)};
}

// increment for incoming S (of that parity)
NLS_SEQ_HD inline int sm_inc(SeqMap m, int S) { return ((S & 1) ? m.c : m.a) >> 1; }

// Binade exponent E of a running sum s >= 0 (the subnormal range and 0: -126).
NLS_SEQ_HD inline int seq_binade(float s) {
  uint32_t bits;
  memcpy(&bits, &s, sizeof bits);
  const int ex = (int)((bits >> 23) & 0xffu);
  return ex == 0 ? -126 : ex - 127;
}

NLS_SEQ_HD inline float seq_ldexp(float x, int e) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_amdgcn_ldexpf(x, e);
#else
  return __builtin_ldexpf(x, e);
#endif
}

// One term's step in the binade of exponent E, packed: -1 when the term
// leaves the binade on its own (e/u >= 2^24, or e is not a number), else
// (I << 1) | tie with I = e/u rounded half up below a tie.  Branch-free.
NLS_SEQ_HD inline int seq_code(float e, int E) {
  const float q = seq_ldexp(e, 23 - E);  // exact (an underflow only loses bits far below 1/2)
  const bool big = !(q < 16777216.0f);
  const float qc = big ? 0.0f : q;
  const float fi = __builtin_truncf(qc);
  const float f = qc - fi;  // exact
  const int I = (int)fi + (f > 0.5f ? 1 : 0);
  const int code = (I << 1) | (f == 0.5f ? 1 : 0);
  return big ? -1 : code;
}

// The map of one term's code.
NLS_SEQ_HD inline SeqMap seq_code_map(int code) {
  if (code < 0) return sm_make(kSeqSat, 0, kSeqSat, 0);
  const int I = code >> 1;
  if (code & 1) {
    const int o = I & 1;
    return sm_make(I + o, 0, I + (o ^ 1), 0);
  }
  return sm_make(I, I & 1, I, (I + 1) & 1);
}

// Terms per thread of the window after a binade change at term `at` of the
// sum: with terms of similar size the sum doubles again around term 2 * at,
// so the window covers about `at` terms (per workgroup of 1024 threads).
NLS_SEQ_HD inline int seq_next_j(int at) {
  int j = 1;
  while (j < kSeqMaxJ && j * 1024 < at) j <<= 1;
  return j;
}

NLS_SEQ_HD inline float seq_fract(float q) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_amdgcn_fractf(q);
#else
  return q - __builtin_floorf(q);
#endif
}

// The map of a run of terms, accumulated term by term without branches: until
// the run's first tie the increments do not depend on the parity (A); the tie
// adds tI plus a parity bit and leaves S even; from there every step is
// determined (B, and the parity `par` after it).  `big`: a term that leaves
// the binade on its own.  A zero term leaves the run unchanged.
struct SeqRun {
  int A = 0, tI = -1, B = 0, par = 0;
  bool big = false;
  // the term e in the binade of exponent E
  NLS_SEQ_HD void add(float e, int E) {
    const float q = seq_ldexp(e, 23 - E);  // exact (an underflow only loses bits far below 1/2)
    const bool bg = !(q < 16777216.0f);
    const float qc = bg ? 0.0f : q;
    const float fr = seq_fract(qc);
    const int I = (int)qc;
    const int t = fr == 0.5f ? 1 : 0;
    const int d = I + (fr > 0.5f ? 1 : 0) + (t & ((par + I) & 1));
    const bool pre = tI < 0;
    big = big || bg;
    A += (pre && !t) ? d : 0;
    B += pre ? 0 : d;
    par = pre ? par : ((par + d) & 1);
    tI = (pre && t) ? I : tI;
  }
  NLS_SEQ_HD SeqMap map() const {
    if (big) return sm_make(kSeqSat, 0, kSeqSat, 0);
    if (tI < 0) return sm_make(A, A & 1, A, (A + 1) & 1);
    // incoming parity p: parity p ^ A at the tie, which adds tI + [(p ^ A) + tI odd]
    const int d0 = A + tI + (((A & 1) + tI) & 1) + B;
    const int d1 = A + tI + ((((A & 1) ^ 1) + tI) & 1) + B;
    return sm_make(d0, par, d1, par);
  }
};

#if defined(__HIPCC__)
constexpr int kSeqNoStop = 0x7fffffff;

struct SeqSumShared {
  SeqMap wtot[2][16];  // per window parity, per wave: the map of its terms
  int stop[2];         // the window's term that leaves the binade (kSeqNoStop: none)
  float s[2];          // the sum after that term
  float s_plain;       // the sum finished with plain adds (NaN or +inf)
};

// Call once (by every thread) before the first seq_sum_block on `sh`, followed
// by a barrier.
__device__ __forceinline__ void seq_sum_init(SeqSumShared& sh) {
  if (threadIdx.x == 0) {
    sh.stop[0] = kSeqNoStop;
    sh.stop[1] = kSeqNoStop;
  }
}

// DPP moves of a packed map (lanes without a source get the identity).
template <int CTRL, int ROWS>
__device__ __forceinline__ SeqMap sm_dpp(SeqMap m) {
  return SeqMap{__builtin_amdgcn_update_dpp(0, m.a, CTRL, ROWS, 0xf, false),
                __builtin_amdgcn_update_dpp(1, m.c, CTRL, ROWS, 0xf, false)};
}

// Inclusive scan of the wave's maps in lane order: row_shr 1, 2, 4, 8 within
// each row of 16 lanes, then row_bcast 15 and 31 across the rows.
__device__ __forceinline__ SeqMap sm_wave_scan(SeqMap m) {
  m = sm_then(sm_dpp<0x111, 0xf>(m), m);
  m = sm_then(sm_dpp<0x112, 0xf>(m), m);
  m = sm_then(sm_dpp<0x114, 0xf>(m), m);
  m = sm_then(sm_dpp<0x118, 0xf>(m), m);
  m = sm_then(sm_dpp<0x142, 0xa>(m), m);
  m = sm_then(sm_dpp<0x143, 0xc>(m), m);
  return m;
}

// Inclusive scan over lanes 0..15 (one row).
__device__ __forceinline__ SeqMap sm_row_scan(SeqMap m) {
  m = sm_then(sm_dpp<0x111, 0xf>(m), m);
  m = sm_then(sm_dpp<0x112, 0xf>(m), m);
  m = sm_then(sm_dpp<0x114, 0xf>(m), m);
  m = sm_then(sm_dpp<0x118, 0xf>(m), m);
  return m;
}

// Inclusive integer scan over lanes 0..15 (one row).
__device__ __forceinline__ int seq_row_scan_int(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, true);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, true);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, true);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, true);  // row_shr:8
  return x;
}

__device__ __forceinline__ SeqMap sm_readlane(SeqMap m, int l) {
  return SeqMap{__builtin_amdgcn_readlane(m.a, l), __builtin_amdgcn_readlane(m.c, l)};
}

// This thread's JB-term run at b (terms at or past `end` count as zeros),
// with every term read before any is used.  Ties are rare (a term whose bits
// below u are exactly 100...0), so the run is first summed as if it held
// none -- the increments are then e/u rounded to nearest and do not depend
// on S -- into A (clamped at 2^24: any run that large leaves the binade).
// When some lane of the wave met a tie or a term too large, `wodd` is set
// and m is the run's parity map, with the bookkeeping redone.
template <int JB>
__device__ __forceinline__ void seq_thread_run(const float* e, int b, int end, int len, int E, int& A,
                                               bool& wodd, SeqMap& m) {
  float v[JB];
#pragma unroll
  for (int j = 0; j < JB; ++j) v[j] = b + j < end ? e[min(b + j, len - 1)] : 0.0f;
  int a = 0;
  bool odd = false;
#pragma unroll
  for (int j = 0; j < JB; ++j) {
    const float q = seq_ldexp(v[j], 23 - E);
    const bool ok = q < 16777216.0f;
    const float qc = ok ? q : 0.0f;
    const float fr = seq_fract(qc);
    a += (int)qc + (fr > 0.5f ? 1 : 0);
    odd = odd || !ok || fr == 0.5f;
  }
  A = min(a, 1 << 24);
  wodd = __ballot(odd) != 0ull;  // wave-uniform
  if (wodd) {
    SeqRun run;
#pragma unroll
    for (int j = 0; j < JB; ++j) run.add(v[j], E);
    m = run.map();
  }
}

// A map that adds the same amount for either parity (a run without ties).
__device__ __forceinline__ bool sm_is_plain(SeqMap m) {
  return (m.a >> 1) == (m.c >> 1) && ((m.a ^ m.c) & 1) != 0;
}

// s + e[0] + ... + e[len - 1], added one at a time in fp32 as above.  Every
// thread of the workgroup calls it with the same arguments and gets the sum.
// s >= 0; the terms e[i] are >= 0 or NaN (a NaN, or an infinite sum, is
// finished with plain adds on one lane).  `e` may be LDS or global memory;
// the caller has made it visible to every thread (a barrier after its
// writes).  J (in/out, 1 .. kSeqMaxJ) is the window's terms per thread and w
// (in/out) the window count, both carried from one call to the next over the
// chunks of a row (start them at 1 and 0, after seq_sum_init and a barrier);
// `done` is the number of terms summed before e[0]; a call with done == 0 and
// w == 0 (the first of a row) adds the first kSeqSerial terms on one lane
// first.  A window scans integer increments in waves without ties (the
// general parity maps in the others) and takes one barrier, or two when a
// term of it leaves the binade; the call ends with a barrier.
template <int NT>
__device__ float seq_sum_block(const float* e, int len, float s, int& J, int& w, int done,
                               SeqSumShared& sh) {
  constexpr int NW = NT / kWave;
  static_assert(NW <= 16, "one map per wave");
  const int tid = (int)threadIdx.x;
  const int lane = lane_id();
  const int wv = tid >> 6;
  int pos = 0;
  if (done == 0 && w == 0 && len > 0) {
    const int n0 = min(len, kSeqSerial);
    if (tid == 0) {
      float t = s;
      int i = 0;
      for (; i + 8 <= n0; i += 8) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = e[i + j];
#pragma unroll
        for (int j = 0; j < 8; ++j) t = t + v[j];
      }
      for (; i < n0; ++i) t = t + e[i];
      sh.s[1] = t;
    }
    __syncthreads();
    // (the first window writes sh.s[0] only; the second writes sh.s[1] after
    // its first barrier, which every thread reaches after this read)
    s = sh.s[1];
    pos = n0;
    J = seq_next_j(n0);
  }
  while (pos < len) {  // uniform
    if (!(s <= 3.4028234663852886e38f)) {
      // NaN or +inf: plain adds
      if (tid == 0) {
        for (int i = pos; i < len; ++i) s = s + e[i];
        sh.s_plain = s;
      }
      __syncthreads();
      s = sh.s_plain;
      __syncthreads();
      return s;
    }
    const int bw = w & 1;
    const int E = seq_binade(s);
    const int S0 = (int)seq_ldexp(s, 23 - E);
    const int jn = min(J, (len - pos + NT - 1) / NT);
    const int b = pos + tid * jn;
    const int end = min(b + jn, len);
    int A = 0;
    bool wodd = false;
    SeqMap m = sm_identity();
    if (jn <= 1)
      seq_thread_run<1>(e, b, end, len, E, A, wodd, m);
    else if (jn <= 2)
      seq_thread_run<2>(e, b, end, len, E, A, wodd, m);
    else if (jn <= 4)
      seq_thread_run<4>(e, b, end, len, E, A, wodd, m);
    else if (jn <= 8)
      seq_thread_run<8>(e, b, end, len, E, A, wodd, m);
    else if (jn <= 12)
      seq_thread_run<12>(e, b, end, len, E, A, wodd, m);
    else
      seq_thread_run<16>(e, b, end, len, E, A, wodd, m);
    // in-wave inclusive scan: integers (<= 2^30) without ties, else maps
    int incA = 0;
    SeqMap incM = sm_identity();
    if (!wodd)
      incA = wave_incl_scan(A);
    else
      incM = sm_wave_scan(m);
    if (lane == kWave - 1) sh.wtot[bw][wv] = wodd ? incM : sm_make(incA, incA & 1, incA, (incA + 1) & 1);
    __syncthreads();
    // (the other buffer's readers finished before the barrier above)
    if (tid == 0) sh.stop[bw ^ 1] = kSeqNoStop;
    // the waves' maps, scanned by every wave's first row of lanes: integers
    // when no wave met a tie (increments saturate at 2^26: the sum stays
    // below 2^31), else maps
    SeqMap wt = lane < NW ? sh.wtot[bw][lane] : sm_identity();
    const bool plain = __ballot(!sm_is_plain(wt)) == 0ull;  // uniform over the workgroup
    SeqMap pre;  // the waves below this one
    int Send;    // S after the window's last term (at least 2^24 when one leaves the binade)
    if (plain) {
      const int d = seq_row_scan_int(lane < NW ? (wt.a >> 1) : 0);
      const int p = wv > 0 ? __builtin_amdgcn_readlane(d, wv - 1) : 0;
      pre = sm_make(p, p & 1, p, (p + 1) & 1);
      Send = S0 + __builtin_amdgcn_readlane(d, NW - 1);
    } else {
      wt = sm_row_scan(wt);
      pre = wv > 0 ? sm_readlane(wt, wv - 1) : sm_identity();
      Send = S0 + sm_inc(sm_readlane(wt, NW - 1), S0);
    }
    ++w;
    if (Send < (1 << 24)) {
      // no term of the window leaves the binade (uniform)
      s = seq_ldexp((float)Send, E - 23);
      pos = min(pos + NT * jn, len);
      J = min(J * 2, kSeqMaxJ);
      continue;
    }
    // this thread's incoming and outgoing S; the one thread where S reaches
    // 2^24 (or meets a term that leaves the binade by itself) has its terms
    // replayed by the first row of its wave, one term per lane
    int Sin, Sout;
    if (!wodd) {
      Sin = S0 + sm_inc(pre, S0) + (incA - A);
      Sout = Sin + A;
    } else {
      Sin = S0 + sm_inc(sm_then(pre, sm_dpp<0x138, 0xf>(incM)), S0);  // wave_shr:1 -- lanes below
      Sout = Sin < (1 << 24) ? Sin + sm_inc(m, Sin) : Sin;
    }
    const uint64_t cross = __ballot(Sin < (1 << 24) && Sout >= (1 << 24));
    if (cross) {  // wave-uniform
      const int L = __ffsll((unsigned long long)cross) - 1;
      const int rb = __builtin_amdgcn_readlane(b, L);
      const int rend = __builtin_amdgcn_readlane(end, L);
      const int rS = __builtin_amdgcn_readlane(Sin, L);
      const int i = rb + lane;
      const bool in = lane < kSeqMaxJ && i < rend;
      const float x = in ? e[i] : 0.0f;
      const int c = in ? seq_code(x, E) : 0;
      const SeqMap incl = sm_row_scan(seq_code_map(c));
      const int Sb = rS + sm_inc(sm_dpp<0x111, 0xf>(incl), rS);  // S before this lane's term
      const int Sa = rS + sm_inc(incl, rS);                         // and after it
      const uint64_t hit = __ballot(in && Sa >= (1 << 24));
      if (lane == __ffsll((unsigned long long)hit) - 1) {
        sh.stop[bw] = i;
        sh.s[bw] = seq_ldexp((float)Sb, E - 23) + x;
      }
    }
    __syncthreads();
    const int k = sh.stop[bw];
    if (k == kSeqNoStop) {
      // (not reached: a window whose sum reaches 2^24 has a thread where it does)
      s = seq_ldexp((float)Send, E - 23);
      pos = min(pos + NT * jn, len);
    } else {
      s = sh.s[bw];
      J = seq_next_j(done + k);
      pos = k + 1;
    }
  }
  __syncthreads();
  return s;
}
#endif

}  // namespace nls
