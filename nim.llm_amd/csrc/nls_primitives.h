// nls_primitives.h -- wave64 / workgroup building blocks for the sampler kernels.
//
// All code here targets gfx950 (wave64).  Workgroup sizes are multiples of 64.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nls {

constexpr int kWave = 64;

// Order-preserving map float32 -> uint32 (larger float -> larger key).
// -0.0 is folded onto +0.0 first: the reference compares with `cmp`/`<`,
// under which the two zeros are equal (sampler.nim:88-97).
__device__ __forceinline__ uint32_t f2key(float f) {
  uint32_t b = __float_as_uint(f);
  if (b == 0x80000000u) b = 0u;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key2f(uint32_t k) {
  const uint32_t b = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(b);
}

__device__ __forceinline__ int lane_id() { return __lane_id(); }

// ---- wave reductions (DPP/swizzle lowered by the compiler from shfl_xor) ----
__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// (value, index) max with the lowest index on equal values.
__device__ __forceinline__ void argmax_merge(float& v, int& i, float v2, int i2) {
  if (v2 > v || (v2 == v && i2 < i)) {
    v = v2;
    i = i2;
  }
}
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float v2 = __shfl_xor(v, o, kWave);
    const int i2 = __shfl_xor(i, o, kWave);
    argmax_merge(v, i, v2, i2);
  }
}

// Inclusive wave scan: DPP row shifts within each 16-lane row (sources
// outside the row read 0), then the row totals are carried across rows.
__device__ __forceinline__ int wave_incl_scan(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, true);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, true);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, true);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, true);  // row_shr:8
  const int r0 = __builtin_amdgcn_readlane(x, 15);
  const int r1 = __builtin_amdgcn_readlane(x, 31);
  const int r2 = __builtin_amdgcn_readlane(x, 47);
  const int row = lane_id() >> 4;
  x += (row >= 1 ? r0 : 0) + (row >= 2 ? r1 : 0) + (row >= 3 ? r2 : 0);
  return x;
}

// Maximum over the wave (every lane gets it): DPP row shifts within each
// 16-lane row, then the four row maxima.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x) {
  x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x111, 0xf, 0xf, true));  // row_shr:1
  x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x112, 0xf, 0xf, true));  // row_shr:2
  x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x114, 0xf, 0xf, true));  // row_shr:4
  x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x118, 0xf, 0xf, true));  // row_shr:8
  const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)x, 15);
  const uint32_t b = (uint32_t)__builtin_amdgcn_readlane((int)x, 31);
  const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)x, 47);
  const uint32_t d = (uint32_t)__builtin_amdgcn_readlane((int)x, 63);
  return max(max(a, b), max(c, d));
}

// The k-th largest of the lanes' values (1 <= k <= 64; lanes without a value
// hold 0): the largest r with at least k values >= r, fixed one bit at a
// time from the top.
__device__ __forceinline__ uint32_t wave_kth_largest(uint32_t x, int k) {
  uint32_t r = 0u;
#pragma unroll
  for (int b = 31; b >= 0; --b) {
    const uint32_t c = r | (1u << b);
    if (__popcll(__ballot(x >= c)) >= k) r = c;
  }
  return r;
}

// Exclusive and total wave sums of small non-negative counts (x < 2^BITS),
// from one ballot per bit: no cross-lane data movement.
template <int BITS>
__device__ __forceinline__ int wave_excl_sum_small(int x, int& total) {
  const uint64_t below = (lane_id() == 0) ? 0ull : (~0ull >> (64 - lane_id()));
  int ex = 0, tot = 0;
#pragma unroll
  for (int b = 0; b < BITS; ++b) {
    const uint64_t m = __ballot((x >> b) & 1);
    ex += __popcll(m & below) << b;
    tot += __popcll(m) << b;
  }
  total = tot;
  return ex;
}

// Exclusive workgroup scan; `smem` needs NT/64 + 1 ints.  Ends with a barrier
// so `smem` may be reused immediately.
template <int NT>
__device__ __forceinline__ int block_excl_scan(int v, int* smem, int& total) {
  const int lane = lane_id();
  const int w = threadIdx.x >> 6;
  const int x = wave_incl_scan(v);
  if (lane == kWave - 1) smem[w] = x;
  __syncthreads();
  if (threadIdx.x == 0) {
    int acc = 0;
#pragma unroll
    for (int q = 0; q < NT / kWave; ++q) {
      const int t = smem[q];
      smem[q] = acc;
      acc += t;
    }
    smem[NT / kWave] = acc;
  }
  __syncthreads();
  const int res = x - v + smem[w];
  total = smem[NT / kWave];
  __syncthreads();
  return res;
}

template <int NT>
__device__ __forceinline__ int block_sum(int v, int* smem) {
  int total;
  (void)block_excl_scan<NT>(v, smem, total);
  return total;
}

// Lanes of the wave below this one.
__device__ __forceinline__ uint64_t lanes_below() {
  const int l = lane_id();
  return l == 0 ? 0ull : (~0ull >> (64 - l));
}

// hist[d] += 1 for every lane with `in` set, for BITS-bit digits; lanes with
// the same digit are grouped with ballots so each distinct digit costs one
// LDS atomic.  Every lane of the wave must call it (the ballots are
// wave-wide).  `slot` maps a digit to its (padded) histogram word.
template <int BITS>
__device__ __forceinline__ void wave_hist_add_bits(uint32_t* hist, uint32_t d, bool in) {
  uint64_t m = __ballot(in);
  if (m == 0ull) return;  // wave-uniform
#pragma unroll
  for (int b = 0; b < BITS; ++b) {
    const bool bit = (d >> b) & 1u;
    const uint64_t bal = __ballot(bit);
    m &= bit ? bal : ~bal;
  }
  if (in && (m & lanes_below()) == 0ull) atomicAdd(&hist[d + (d >> 5)], (uint32_t)__popcll(m));
}

struct SelectResult {
  uint32_t tau;  // threshold key
  int ge;        // items with key >= tau
  int gt;        // items with key > tau (exact only when the select ran to the last digit)
};

// Histogram of the radix select: 2048 digit bins, one pad word per 32 bins
// so that wave 0 reads 32 consecutive bins per lane without bank conflicts.
constexpr int kSelBins = 2048;
constexpr int kSelWords = kSelBins + kSelBins / 32;

// MSB-first radix select over 32-bit keys with 11-, 11- and 10-bit digits.
// for_each(fn) calls fn(key, valid) for the thread's items; the number of
// calls must be the same on every lane of a wave.  Finds the kk-th largest
// valid key (1 <= kk <= valid item count).  Returns early, after any round,
// with tau = the current prefix (lower bits zero) as soon as the number of
// items >= tau is at most `fit`; that tau is a lower bound of the kk-th
// largest.  fit < 0 always runs to the exact kk-th largest.
// `hist` (kSelWords uints) must be all zero on entry and is left all zero;
// `smem` is NT/64 + 4 ints.
template <int NT, typename ForEach>
__device__ __forceinline__ SelectResult block_select(ForEach for_each, int kk, int fit,
                                                     uint32_t* hist, int* smem) {
  constexpr int NW = NT / kWave;
  uint32_t prefix = 0u, mask = 0u;
  int gt = 0;
  SelectResult r;
#pragma unroll 1
  for (int round = 0; round < 3; ++round) {
    const int shift = round == 0 ? 21 : round == 1 ? 10 : 0;
    const uint32_t dmask = round == 2 ? 1023u : 2047u;
    for_each([&](uint32_t key, bool valid) {
      wave_hist_add_bits<11>(hist, (key >> shift) & dmask, valid && ((key & mask) == prefix));
    });
    __syncthreads();
    if (threadIdx.x < kWave) {
      // lane l owns bins [2048 - 32 (l + 1), 2048 - 32 l): the largest digits first
      const int lane = threadIdx.x;
      const int base = kSelBins - 32 * (lane + 1);
      uint32_t* hb = hist + base + (base >> 5);
      int c = 0;
#pragma unroll
      for (int q = 0; q < 32; ++q) c += (int)hb[q];
      const int incl = wave_incl_scan(c);
      const int above = incl - c;  // items in larger digits
      // the lane holding the kk-th largest; then lanes 0..31 scan its 32 bins
      // (lane q takes the q-th largest digit of them)
      const uint64_t sel = __ballot(above < kk && above + c >= kk);
      const int sl = __ffsll((unsigned long long)sel) - 1;
      const int sbase = __builtin_amdgcn_readlane(base, sl);
      const int sabove = __builtin_amdgcn_readlane(above, sl);
      const int dq = sbase + 31 - (lane & 31);
      const int cq = lane < 32 ? (int)hist[dq + (dq >> 5)] : 0;
      const int iq = wave_incl_scan(cq) + sabove;  // items >= digit dq
      const uint64_t hitq = __ballot(lane < 32 && iq >= kk);
      const int fq = __ffsll((unsigned long long)hitq) - 1;
      if (lane == fq) {
        smem[NW + 1] = dq;
        smem[NW + 2] = iq - cq;
        smem[NW + 3] = cq;
      }
#pragma unroll
      for (int q = 0; q < 32; ++q) hb[q] = 0u;
    }
    __syncthreads();
    const int d = smem[NW + 1], ab = smem[NW + 2], cd = smem[NW + 3];
    kk -= ab;
    gt += ab;
    prefix |= (uint32_t)d << shift;
    mask |= dmask << shift;
    if (round == 2 || gt + cd <= fit) {
      r.tau = prefix;
      r.ge = gt + cd;
      r.gt = gt;
      break;
    }
  }
  // smem[NW + 1..3] are read above by every thread; the caller's next
  // barrier orders any reuse.
  return r;
}

// ---- wave-private radix select (no barriers) ----
// Per-wave histogram of 256 bins, all zero on entry and on return.
constexpr int kWaveBins = 256;

__device__ __forceinline__ void wave_hist_add8(uint32_t* hist, uint32_t d, bool in) {
  uint64_t m = __ballot(in);
  if (m == 0ull) return;  // wave-uniform
#pragma unroll
  for (int b = 0; b < 8; ++b) {
    const bool bit = (d >> b) & 1u;
    const uint64_t bal = __ballot(bit);
    m &= bit ? bal : ~bal;
  }
  if (in && (m & lanes_below()) == 0ull) atomicAdd(&hist[d], (uint32_t)__popcll(m));
}

// kk-th largest of the keys one wave feeds through for_each(fn): fn(key,
// valid) with a wave-uniform number of calls; 1 <= kk <= valid items.  Same
// early-exit contract as block_select (`fit`), 8-bit digits, and only this
// wave's `hist` (kWaveBins words) is touched, so no barrier is needed: LDS
// operations of one wave complete in order.
template <typename ForEach>
__device__ __forceinline__ SelectResult wave_select(ForEach for_each, int kk, int fit,
                                                    uint32_t* hist) {
  const int lane = lane_id();
  uint32_t prefix = 0u, mask = 0u;
  int gt = 0;
  SelectResult r;
#pragma unroll 1
  for (int shift = 24;; shift -= 8) {
    for_each([&](uint32_t key, bool valid) {
      wave_hist_add8(hist, (key >> shift) & 255u, valid && ((key & mask) == prefix));
    });
    // lane l owns digits 255-4l .. 252-4l (largest first)
    const int top = kWaveBins - 1 - 4 * lane;
    const int b0 = (int)hist[top], b1 = (int)hist[top - 1], b2 = (int)hist[top - 2],
              b3 = (int)hist[top - 3];
    hist[top] = 0u;
    hist[top - 1] = 0u;
    hist[top - 2] = 0u;
    hist[top - 3] = 0u;
    const int c = b0 + b1 + b2 + b3;
    const int above = wave_incl_scan(c) - c;
    const bool mine = above < kk && above + c >= kk;
    int d = top, ab = above, cd = b0;
    if (above + b0 < kk) {
      d = top - 1;
      ab = above + b0;
      cd = b1;
      if (ab + b1 < kk) {
        d = top - 2;
        ab += b1;
        cd = b2;
        if (ab + b2 < kk) {
          d = top - 3;
          ab += b2;
          cd = b3;
        }
      }
    }
    const int sl = __ffsll((unsigned long long)__ballot(mine)) - 1;
    d = __builtin_amdgcn_readlane(d, sl);
    ab = __builtin_amdgcn_readlane(ab, sl);
    cd = __builtin_amdgcn_readlane(cd, sl);
    kk -= ab;
    gt += ab;
    prefix |= (uint32_t)d << shift;
    mask |= 255u << shift;
    if (shift == 0 || gt + cd <= fit) {
      r.tau = prefix;
      r.ge = gt + cd;
      r.gt = gt;
      return r;
    }
  }
}

// Per-thread top-Q of the keys fed to it (descending, zero-filled).
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

// In-place bitonic sort of n (power of two) 64-bit keys, ascending.
template <int NT, typename Ptr>
__device__ __forceinline__ void bitonic_sort_u64(Ptr a, int n, bool descending) {
  // Bitonic network over a[0..n), n a power of two.  The stages whose
  // partners lie less than 64 apart stay inside a 64-element block: a wave
  // loads its blocks into registers (one element per lane) and runs each
  // such run of stages through lane shuffles, with one barrier after the
  // run.  Stages of larger distance go through memory, a barrier each.
  const int lane = (int)(threadIdx.x & (kWave - 1));
  const int wv = (int)(threadIdx.x / kWave);
  // stages (k, j) for k = k_lo..k_hi and j = (k == k_lo ? j_lo : k/2) .. 1
  auto wave_run = [&](int k_lo, int k_hi, int j_lo) __attribute__((always_inline)) {
    for (int b = wv * kWave; b < n; b += NT) {
      const int i = b + lane;
      uint64_t x = i < n ? a[i] : 0ull;
      for (int k = k_lo; k <= k_hi; k <<= 1) {
        const bool up = ((i & k) == 0) != descending;
        for (int j = (k == k_lo ? j_lo : (k >> 1)); j > 0; j >>= 1) {
          const uint32_t lo = __shfl_xor((uint32_t)x, j, kWave);
          const uint32_t hi = __shfl_xor((uint32_t)(x >> 32), j, kWave);
          const uint64_t y = ((uint64_t)hi << 32) | lo;
          // the lower index of a pair keeps the smaller value when ascending
          const bool keep_small = ((i & j) == 0) == up;
          x = keep_small ? (y < x ? y : x) : (y < x ? x : y);
        }
      }
      if (i < n) a[i] = x;
    }
  };
  if (n <= 1) return;
  wave_run(2, n < kWave ? n : kWave, 1);
  __syncthreads();
  for (int k = 2 * kWave; k <= n; k <<= 1) {
    for (int j = k >> 1; j >= kWave; j >>= 1) {
      for (int i = threadIdx.x; i < n; i += NT) {
        const int ixj = i ^ j;
        if (ixj > i) {
          const uint64_t x = a[i], y = a[ixj];
          const bool up = ((i & k) == 0) != descending;
          if (up ? (x > y) : (x < y)) {
            a[i] = y;
            a[ixj] = x;
          }
        }
      }
      __syncthreads();
    }
    wave_run(k, k, kWave / 2);
    __syncthreads();
  }
}

__host__ __device__ inline int next_pow2(int n) {
  int p = 1;
  while (p < n) p <<= 1;
  return p;
}

// ---- Nim std/random on the device (xoroshiro128+; rand(1.0)) ----
__device__ __forceinline__ uint64_t rotl64(uint64_t x, int k) {
  return (x << k) | (x >> (64 - k));
}
__device__ __forceinline__ double nim_rand_unit(uint64_t* st) {
  const uint64_t s0 = st[0];
  uint64_t s1 = st[1];
  const uint64_t res = s0 + s1;
  s1 ^= s0;
  st[0] = rotl64(s0, 55) ^ s1 ^ (s1 << 14);
  st[1] = rotl64(s1, 36);
  const uint64_t bits = (0x3FFull << 52) | (res >> 12);
  return __longlong_as_double((long long)bits) - 1.0;
}

}  // namespace nls
