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

// Inclusive wave scan.
__device__ __forceinline__ int wave_incl_scan(int x) {
  const int lane = lane_id();
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int y = __shfl_up(x, o, kWave);
    if (lane >= o) x += y;
  }
  return x;
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

// kk-th largest (1-based) 32-bit key among the items each thread feeds through
// `for_each(fn)` (fn(key) is called once per item).  MSB-first radix select,
// 8 bits per round, histogram in LDS.  Requires NT >= 256 and
// 1 <= kk <= item count.  `hist` is 256 uints, `smem` NT/64 + 3 ints.
template <int NT, typename ForEach>
__device__ uint32_t block_radix_select(ForEach for_each, int kk, uint32_t* hist, int* smem) {
  static_assert(NT >= 256, "radix select needs >= 256 threads");
  uint32_t prefix = 0u, mask = 0u;
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int q = threadIdx.x; q < 256; q += NT) hist[q] = 0u;
    __syncthreads();
    for_each([&](uint32_t key) {
      if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
    });
    __syncthreads();
    // reversed bins so an exclusive prefix sum is the count strictly above
    const int t = threadIdx.x;
    const int c = (t < 256) ? (int)hist[255 - t] : 0;
    int tot;
    const int above = block_excl_scan<NT>(c, smem, tot);
    if (t < 256 && above < kk && above + c >= kk) {
      smem[NT / kWave + 1] = 255 - t;
      smem[NT / kWave + 2] = above;
    }
    __syncthreads();
    const int d = smem[NT / kWave + 1];
    kk -= smem[NT / kWave + 2];
    prefix |= (uint32_t)d << shift;
    mask |= 255u << shift;
    __syncthreads();
  }
  return prefix;
}

// In-place bitonic sort of n (power of two) 64-bit keys, ascending.
template <int NT, typename Ptr>
__device__ void bitonic_sort_u64(Ptr a, int n, bool descending) {
  for (int k = 2; k <= n; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
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
