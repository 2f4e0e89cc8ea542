// nls_softmax.hip -- softmaxInPlace (sampler.nim:51-57) over whole rows on
// the device, and logProb's per-token term (nimllm-doc-en.md:1700-1707).
//
// One 1024-thread workgroup per row, three steps:
//   1. mx, the row's float32 maximum (Nim's max(mx, v) keeps mx for a NaN v,
//      as fmaxf does; the sign of a zero maximum changes no l - mx).
//   2. s, the fp32 sum of exp(l - mx) (correctly rounded: nls_expf.h's table
//      form, its table in LDS) in index order: chunks of 12288 exponentials
//      go to LDS -- the next chunk's logits are requested before the current
//      chunk is summed -- and the workgroup adds each chunk exactly as
//      one-at-a-time fp32 adds would, with the parity-map scan of
//      nls_seqsum.h.
//   3. softmax: out[i] = exp(l_i - mx) / s for the whole row (out may be the
//      logits themselves: each element is read before it is written, by the
//      same thread); logProb: p = exp(l_t - mx) / s for the row's target t,
//      and ln(float64(p)).
// The row is read three times (twice for logProb) and written once; the
// exponentials are recomputed in step 3 rather than stored.
#include "nls_device.h"
#include "nls_seqsum.h"

namespace nls {

namespace {
constexpr int kSmxNT = 1024;
constexpr int kSmxPer = 12;                 // logits per thread and chunk
constexpr int kSmxChunk = kSmxNT * kSmxPer;  // 12288: 48 KB of exponentials in LDS
constexpr int kSmxOOR = 0x7ffffff0;          // buffer offset that reads 0 without touching memory
}  // namespace

template <bool LOGP>
__global__ __launch_bounds__(kSmxNT) void softmax_kernel(const float* logits, int64_t V,
                                                         float* out, const int32_t* __restrict__ targets,
                                                         float* __restrict__ prob, double* __restrict__ logp) {
  constexpr int NT = kSmxNT;
  constexpr int NW = NT / kWave;
  static_assert(kSmxPer <= kSeqMaxJ && kSmxPer % 4 == 0, "chunk layout");
  __shared__ __align__(16) float ebuf[kSmxChunk];
  __shared__ SeqSumShared sh;
  __shared__ float s_part[NW];
  __shared__ double s_pow2[kExpfPow2Count];  // the exponential's table
  const int row = (int)blockIdx.x;
  const int tid = (int)threadIdx.x;
  const int lane = lane_id();
  const int wv = tid >> 6;
  const int n = (int)V;  // V < 2^29 (checked by the host)
  const float* x = logits + (int64_t)row * V;
  const __amdgpu_buffer_rsrc_t xr = slice_rsrc(x, n);
  // 16-byte accesses when every row start is 16-byte aligned
  const bool vec = (n % 4 == 0) && ((reinterpret_cast<uintptr_t>(logits) & 15) == 0);
  // element of slot q of this thread in the chunk at c0: float4 group
  // tid + (q / 4) * NT (vec), or element tid + q * NT
  auto elem = [&](int c0, int q) -> int {
    return vec ? c0 + 4 * (tid + (q >> 2) * NT) + (q & 3) : c0 + tid + q * NT;
  };
  auto load = [&](int c0, float (&v)[kSmxPer]) __attribute__((always_inline)) {
    if (vec) {
#pragma unroll
      for (int g = 0; g < kSmxPer / 4; ++g) {
        const int e0 = c0 + 4 * (tid + g * NT);
        const f32x4 t = __builtin_bit_cast(
            f32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, e0 < n ? e0 * 4 : kSmxOOR, 0, 0));
        v[4 * g] = t.x;
        v[4 * g + 1] = t.y;
        v[4 * g + 2] = t.z;
        v[4 * g + 3] = t.w;
      }
    } else {
#pragma unroll
      for (int q = 0; q < kSmxPer; ++q) {
        const int e = c0 + tid + q * NT;
        v[q] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(xr, e < n ? e * 4 : kSmxOOR, 0, 0));
      }
    }
  };

  // (1) mx (:52-53), the next chunk requested before the current one is reduced
  float mx = -__builtin_inff();
  {
    float a[kSmxPer], b[kSmxPer];
    load(0, a);
    // (after the first chunk's requests; the barrier after this pass orders it)
    if (tid < kExpfPow2Count) s_pow2[tid] = kExpfPow2J64[tid];
    for (int c0 = 0; c0 < n; c0 += kSmxChunk) {
      const bool more = c0 + kSmxChunk < n;
      if (more) load(c0 + kSmxChunk, b);
#pragma unroll
      for (int q = 0; q < kSmxPer; ++q)
        if (elem(c0, q) < n) mx = __builtin_fmaxf(mx, a[q]);
      if (more) {
#pragma unroll
        for (int q = 0; q < kSmxPer; ++q) a[q] = b[q];
      }
    }
  }
  for (int o = kWave / 2; o > 0; o >>= 1) mx = __builtin_fmaxf(mx, __shfl_xor(mx, o));
  if (lane == 0) s_part[wv] = mx;
  __syncthreads();
  mx = s_part[0];
  for (int w = 1; w < NW; ++w) mx = __builtin_fmaxf(mx, s_part[w]);

  // (2) s = exp(l_0 - mx) + exp(l_1 - mx) + ... in index order (:54-56)
  // (the barriers of the first chunk's staging order seq_sum_init's stores)
  seq_sum_init(sh);
  float s = 0.0f;
  int J = 1, nwin = 0;
  {
    float v[kSmxPer];
    load(0, v);
    for (int c0 = 0; c0 < n; c0 += kSmxChunk) {
#pragma unroll
      for (int q = 0; q < kSmxPer; ++q) {
        const int e = elem(c0, q);
        if (e < n) ebuf[e - c0] = expf_cr_t(v[q] - mx, s_pow2);
      }
      __syncthreads();
      if (c0 + kSmxChunk < n) load(c0 + kSmxChunk, v);
      s = seq_sum_block<NT>(ebuf, min(kSmxChunk, n - c0), s, J, nwin, c0, sh);  // ends with a barrier
    }
  }

  if constexpr (LOGP) {
    // (3) logProb: p[t] (:57) and ln(float64(p[t]))
    if (tid == 0) {
      const int t = targets[row];
      float p = __builtin_nanf("");
      if (t >= 0 && t < n) p = expf_cr_t(x[t] - mx, s_pow2) / s;
      prob[row] = p;
      logp[row] = log((double)p);
    }
  } else {
    // (3) softmax: v /= s (:57) over the row
    float* o = out + (int64_t)row * V;
    const bool ovec = vec && ((reinterpret_cast<uintptr_t>(out) & 15) == 0);
    float a[kSmxPer], b[kSmxPer];
    load(0, a);
    for (int c0 = 0; c0 < n; c0 += kSmxChunk) {
      const bool more = c0 + kSmxChunk < n;
      if (more) load(c0 + kSmxChunk, b);
      if (ovec) {
#pragma unroll
        for (int g = 0; g < kSmxPer / 4; ++g) {
          const int e0 = c0 + 4 * (tid + g * NT);
          if (e0 < n) {
            f32x4 r;
            r.x = expf_cr_t(a[4 * g] - mx, s_pow2) / s;
            r.y = expf_cr_t(a[4 * g + 1] - mx, s_pow2) / s;
            r.z = expf_cr_t(a[4 * g + 2] - mx, s_pow2) / s;
            r.w = expf_cr_t(a[4 * g + 3] - mx, s_pow2) / s;
            *reinterpret_cast<f32x4*>(o + e0) = r;
          }
        }
      } else {
#pragma unroll
        for (int q = 0; q < kSmxPer; ++q) {
          const int e = elem(c0, q);
          if (e < n) o[e] = expf_cr_t(a[q] - mx, s_pow2) / s;
        }
      }
      if (more) {
#pragma unroll
        for (int q = 0; q < kSmxPer; ++q) a[q] = b[q];
      }
    }
  }
}

hipError_t launch_softmax_rows(const float* logits, int rows, int64_t V, float* out, hipStream_t s) {
  hipLaunchKernelGGL(softmax_kernel<false>, dim3(rows), dim3(kSmxNT), 0, s, logits, V, out, nullptr, nullptr,
                     nullptr);
  return hipGetLastError();
}

hipError_t launch_log_prob(const float* logits, int rows, int64_t V, const int32_t* targets, float* prob,
                           double* logp, hipStream_t s) {
  hipLaunchKernelGGL(softmax_kernel<true>, dim3(rows), dim3(kSmxNT), 0, s, logits, V, nullptr, targets, prob,
                     logp);
  return hipGetLastError();
}

}  // namespace nls
