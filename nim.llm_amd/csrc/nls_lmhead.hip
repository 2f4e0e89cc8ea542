// nls_lmhead.hip -- the output projection (LM head) on gfx950.
//
// y[b, r] = dot(W[r, :], x[b, :]) for GGUF-quantised weight rows, computed the
// way nimllm's `matmul` computes it for `m.output` (src/nimllm/model.nim:144-200,
// called at :461-470), so the logits the sampler reads are bit-identical to
// the reference's:
//
//  * the int8 path (model.nim:150-156, taken when actBlockLen > 0, cols is a
//    multiple of it, nb <= 4 or the type is not Q8_0, and exactMatmul is off):
//    the activations are quantised per block (quantizeAct, quant.nim:646-667)
//    and each block's integer dot product is formed exactly; its float term
//    (quant.nim:669-786) is formed with the reference's fp32 operations and
//    the terms are added in block order;
//  * the float path (:157-170): the row is dequantised (dequantBlock,
//    quant.nim:164-334) and dotted with x in dotF32's eight strided chains
//    (quant.nim:362-374);
//  * an optional LoRA term (:189-200).
//
// Integer sums are exact in any grouping, so the int8 path splits a block
// across 8 lanes (32 weights each) and adds the lanes' partial sums; only the
// per-block fp32 terms must be added in order, which one lane per row does
// from LDS after the wave has formed the terms of its rows.  A dotF32 chain is
// a sequential fp32 sum, so the float path gives each chain its own lane
// (8 lanes per row) and combines the chains in the reference's order with DPP
// exchanges (fp32 addition commutes exactly).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "nls_internal.h"

namespace nls {
namespace {

constexpr int kLmNT = 256;   // threads per workgroup: 4 waves
constexpr int kLmNBC = 4;    // activation rows per pass over a row group

// ---------------------------------------------------------------- loads

__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) {
  uint16_t v;
  __builtin_memcpy(&v, p, 2);
  return v;
}
__device__ __forceinline__ uint2 ld_8(const void* p) {
  uint2 v;
  __builtin_memcpy(&v, p, 8);
  return v;
}
__device__ __forceinline__ uint4 ld_16(const void* p) {
  uint4 v;
  __builtin_memcpy(&v, p, 16);
  return v;
}
// 4-byte aligned words covering NW * 4 bytes at a 2-byte aligned address,
// funnel-shifted into place (the word past the field is read only when the
// address is not 4-byte aligned, and never past the field's last word).
template <int NW>
__device__ __forceinline__ void ld_words_a(const uint8_t* p, uint32_t (&out)[NW]) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  const uint32_t sh = (uint32_t)(a & 3) * 8;
  const uint32_t* q = reinterpret_cast<const uint32_t*>(p - (a & 3));
  uint32_t w[NW + 1];
#pragma unroll
  for (int k = 0; k < NW; k += 4) {
    uint4 v;
    __builtin_memcpy(&v, q + k, 16);
    w[k] = v.x;
    w[k + 1] = v.y;
    w[k + 2] = v.z;
    w[k + 3] = v.w;
  }
  w[NW] = sh ? q[NW] : 0u;
#pragma unroll
  for (int k = 0; k < NW; ++k) out[k] = __builtin_amdgcn_alignbit(w[k + 1], w[k], sh);
}

// IEEE half to float: exact for every finite half (subnormals included).
__device__ __forceinline__ float half_f(uint32_t bits) {
  _Float16 h;
  const uint16_t b = (uint16_t)bits;
  __builtin_memcpy(&h, &b, 2);
  return (float)h;
}
__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}
constexpr uint32_t kOnes = 0x01010101u;
constexpr uint32_t kLo4 = 0x0F0F0F0Fu;

// Sum over the aligned group of 8 lanes; the total lands on lanes 4..7 of
// the group (quad exchanges, then a row shift by 4).
__device__ __forceinline__ int group8_sum(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);  // quad_perm 1,0,3,2
  v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);  // quad_perm 2,3,0,1
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, true);  // row_shr:4
  return v;
}
template <int CTRL, bool BOUND>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, BOUND);
}
// NB per-state block sums of an aligned group of 8 lanes (lane p = 0..7 of
// the group), reduced at once: lanes exchange the halves of their states
// they do not keep (quad_perm 1,0,3,2, then 2,3,0,1), so each lane of a quad
// holds one state's quad sum, and row_shr:4 adds the other quad.  Lanes 4..7
// get the totals of states group8_state<NB>(p) (NB = 4: 0, 2, 1, 3; NB = 2:
// 0, 1, 0, 1): 4 DPP moves for four states instead of 12.
template <int NB>
__device__ __forceinline__ int group8_state(int p) {
  return NB == 4 ? (((p & 1) << 1) | ((p >> 1) & 1)) : (p & 1);
}
template <int NB>
__device__ __forceinline__ int group8_sum_states(const int (&v)[NB], int p) {
  static_assert(NB == 2 || NB == 4, "two or four states");
  const bool odd = p & 1;
  int t;
  if constexpr (NB == 2) {
    const int keep = odd ? v[1] : v[0], send = odd ? v[0] : v[1];
    t = keep + dpp_i<0xB1, false>(send);
    t += dpp_i<0x4E, false>(t);
  } else {
    const int k0 = odd ? v[2] : v[0], k1 = odd ? v[3] : v[1];
    const int x0 = odd ? v[0] : v[2], x1 = odd ? v[1] : v[3];
    const int r0 = k0 + dpp_i<0xB1, false>(x0), r1 = k1 + dpp_i<0xB1, false>(x1);
    const bool hi = (p & 2) != 0;
    t = (hi ? r1 : r0) + dpp_i<0x4E, false>(hi ? r0 : r1);
  }
  return t + dpp_i<0x114, true>(t);  // row_shr:4
}
template <int CTRL, bool BOUND>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, BOUND));
}
// dotF32's combine (quant.nim:374), `(s0 + s1) + (s2 + s3) + (s4 + s5) +
// (s6 + s7)`, which adds left to right: ((p01 + p23) + p45) + p67, of lane
// k's value s_k in an aligned group of 8.  The result lands on lane 6 of the
// group (fp32 addition commutes exactly, so a + b may be formed as b + a).
__device__ __forceinline__ float group8_dotf32_combine(float v) {
  const float pair = v + dpp_f<0xB1, false>(v);      // quad_perm 1,0,3,2: lanes 2i, 2i+1 hold p
  const float a = pair + dpp_f<0x4E, false>(pair);   // lane 0: p01 + p23
  const float c = pair + dpp_f<0x114, true>(a);      // row_shr:4 -> lane 4: p45 + (p01 + p23)
  return pair + dpp_f<0x00, false>(c);               // quad_perm 0,0,0,0 -> lane 6: p67 + that
}

// ------------------------------------------------ int8 path, per format
//
// A lane owns one 32-weight slice of a block: `p` is the slice within the
// block (0..7 for the 256-weight K formats, 0 for Q8_0 / Q4_0).  Wt holds the
// slice's weight bytes and the block's scale fields, Act the matching 32
// activation bytes and the sums the format subtracts.

template <int T>
struct Fmt;

// Q6_K (quant.nim:731-760): ql[128] qh[64] scales[16] d.  Slice p: half
// h = p / 4, positions l0 = 8 (p % 4) .. l0 + 7, all four quarters m = 0..3
// (weights 128 h + 32 m + l).
template <>
struct Fmt<14> {
  static constexpr int BL = 256, TS = 210, LPB = 8;
  struct Wt {
    uint2 ql0, ql1, qh, sc;
    uint32_t d;
  };
  struct Act {
    uint2 a[4];
    int a32[4];  // 32 * (sum of the quarter's 8 activations)
  };
  __device__ static Wt load_w(const uint8_t* blk, int p) {
    const int h = p >> 2, l0 = 8 * (p & 3);
    Wt w;
    w.ql0 = ld_8(blk + 64 * h + l0);
    w.ql1 = ld_8(blk + 64 * h + 32 + l0);
    w.qh = ld_8(blk + 128 + 32 * h + l0);
    w.sc = ld_8(blk + 192 + 8 * h);
    w.d = ld_u16(blk + 208);
    return w;
  }
  static constexpr bool HAS_MIN = false;
  // byte group gi (8 activations) of slice p: weights 128 h + 32 gi + l0 ..
  __device__ static int group_base(int p, int gi) { return 128 * (p >> 2) + 32 * gi + 8 * (p & 3); }
  __device__ static Act make_act(const uint32_t (&wd)[8]) {
    Act a;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      a.a[m] = make_uint2(wd[2 * m], wd[2 * m + 1]);
      a.a32[m] = 32 * dot4(kOnes, wd[2 * m + 1], dot4(kOnes, wd[2 * m], 0));
    }
    return a;
  }
  __device__ static void partial(const Wt& w, const Act& a, int p, int& sumi, int& summ) {
    const int g = (p >> 1) & 1;  // which 16 of the half's 32 positions
    uint32_t q[4][2];
    const uint32_t L0[2] = {w.ql0.x, w.ql0.y}, L1[2] = {w.ql1.x, w.ql1.y}, H[2] = {w.qh.x, w.qh.y};
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      q[0][k] = (L0[k] & kLo4) | ((H[k] << 4) & 0x30303030u);
      q[1][k] = (L1[k] & kLo4) | ((H[k] << 2) & 0x30303030u);
      q[2][k] = ((L0[k] >> 4) & kLo4) | (H[k] & 0x30303030u);
      q[3][k] = ((L1[k] >> 4) & kLo4) | ((H[k] >> 2) & 0x30303030u);
    }
    int s = 0;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const uint32_t scw = (m & 2) ? w.sc.y : w.sc.x;
      const int sc = __builtin_amdgcn_sbfe((int)scw, 8 * (g + (m & 1) * 2), 8);
      const int dm = dot4(q[m][1], a.a[m].y, dot4(q[m][0], a.a[m].x, 0)) - a.a32[m];
      s += __mul24(sc, dm);  // |sc| < 2^7, |dm| < 2^17: 24-bit products
    }
    sumi = s;
    summ = 0;
  }
  // acc += a.d * d * sumi  (quant.nim:759)
  __device__ static float term(const Wt& w, int sumi, int, float ad) {
    return __fmul_rn(__fmul_rn(ad, half_f(w.d)), (float)sumi);
  }
};

// Q4_K (quant.nim:669-695) and Q5_K (:697-729): d dmin scales[12] [qh[32]]
// qs[128].  Slice p: pair j = p / 2 of sub-blocks (2j, 2j + 1), positions
// l0 = 16 (p % 2) .. l0 + 15 (weights 64 j + l and 64 j + 32 + l).
template <bool FIVE>
struct FmtK45 {
  static constexpr int BL = 256, TS = FIVE ? 176 : 144, LPB = 8;
  struct Wt {
    uint4 hd;   // d, dmin, scales[12]
    uint4 qs;
    uint4 qh;   // Q5_K only
  };
  struct Act {
    uint4 lo, hi;
    int slo, shi;  // sums of the 16 activations (the reference's bsums)
  };
  __device__ static Wt load_w(const uint8_t* blk, int p) {
    const int j = p >> 1, l0 = 16 * (p & 1);
    Wt w;
    w.hd = ld_16(blk);
    w.qs = ld_16(blk + (FIVE ? 48 : 16) + 32 * j + l0);
    if (FIVE) w.qh = ld_16(blk + 16 + l0);
    return w;
  }
  static constexpr bool HAS_MIN = true;
  // byte groups 0, 1: weights 64 j + l0 ..; groups 2, 3: 64 j + 32 + l0 ..
  __device__ static int group_base(int p, int gi) {
    return 64 * (p >> 1) + 16 * (p & 1) + (gi < 2 ? 8 * gi : 32 + 8 * (gi - 2));
  }
  __device__ static Act make_act(const uint32_t (&wd)[8]) {
    Act a;
    a.lo = make_uint4(wd[0], wd[1], wd[2], wd[3]);
    a.hi = make_uint4(wd[4], wd[5], wd[6], wd[7]);
    a.slo = dot4(kOnes, wd[3], dot4(kOnes, wd[2], dot4(kOnes, wd[1], dot4(kOnes, wd[0], 0))));
    a.shi = dot4(kOnes, wd[7], dot4(kOnes, wd[6], dot4(kOnes, wd[5], dot4(kOnes, wd[4], 0))));
    return a;
  }
  // getScaleMinK4 (quant.nim:156-162) of sub-block jj from the header words
  __device__ static void scale_min(const uint4& hd, int jj, int& sc, int& mn) {
    const int k = 8 * (jj & 3);
    const uint32_t yb = (hd.y >> k) & 0xFF, zb = (hd.z >> k) & 0xFF, wb = (hd.w >> k) & 0xFF;
    if (jj < 4) {
      sc = yb & 63;
      mn = zb & 63;
    } else {
      sc = (wb & 0xF) | ((yb >> 6) << 4);
      mn = (wb >> 4) | ((zb >> 6) << 4);
    }
  }
  __device__ static void partial(const Wt& w, const Act& a, int p, int& sumi, int& summ) {
    const int j = p >> 1;
    const uint32_t Q[4] = {w.qs.x, w.qs.y, w.qs.z, w.qs.w};
    const uint32_t H[4] = {w.qh.x, w.qh.y, w.qh.z, w.qh.w};
    const uint32_t AL[4] = {a.lo.x, a.lo.y, a.lo.z, a.lo.w};
    const uint32_t AH[4] = {a.hi.x, a.hi.y, a.hi.z, a.hi.w};
    int s0 = 0, s1 = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint32_t lo = Q[k] & kLo4, hi = (Q[k] >> 4) & kLo4;
      if (FIVE) {
        lo |= ((H[k] >> (2 * j)) & kOnes) << 4;
        hi |= ((H[k] >> (2 * j + 1)) & kOnes) << 4;
      }
      s0 = dot4(lo, AL[k], s0);
      s1 = dot4(hi, AH[k], s1);
    }
    int sc0, m0, sc1, m1;
    scale_min(w.hd, 2 * j, sc0, m0);
    scale_min(w.hd, 2 * j + 1, sc1, m1);
    // scales < 2^6, |s0|, |s1| < 2^16, |slo|, |shi| < 2^11: 24-bit products
    sumi = __mul24(sc0, s0) + __mul24(sc1, s1);
    summ = __mul24(m0, a.slo) + __mul24(m1, a.shi);
  }
  // acc += a.d * (d * sumi - dmin * summ)  (quant.nim:694, :728)
  __device__ static float term(const Wt& w, int sumi, int summ, float ad) {
    const float d = half_f(w.hd.x & 0xFFFF), dmin = half_f(w.hd.x >> 16);
    return __fmul_rn(ad, __fsub_rn(__fmul_rn(d, (float)sumi), __fmul_rn(dmin, (float)summ)));
  }
};
template <>
struct Fmt<12> : FmtK45<false> {};
template <>
struct Fmt<13> : FmtK45<true> {};

// Q8_0 (quant.nim:762-772): d qs[32]; one lane per block.
template <>
struct Fmt<8> {
  static constexpr int BL = 32, TS = 34, LPB = 1;
  struct Wt {
    uint4 q0, q1;
    uint32_t d;
  };
  struct Act {
    uint4 a0, a1;
  };
  __device__ static Wt load_w(const uint8_t* blk, int) {
    Wt w;
    w.d = ld_u16(blk);
    uint32_t q[8];
    ld_words_a<8>(blk + 2, q);
    w.q0 = make_uint4(q[0], q[1], q[2], q[3]);
    w.q1 = make_uint4(q[4], q[5], q[6], q[7]);
    return w;
  }
  static constexpr bool HAS_MIN = false;
  __device__ static int group_base(int, int gi) { return 8 * gi; }
  __device__ static Act make_act(const uint32_t (&wd)[8]) {
    return Act{make_uint4(wd[0], wd[1], wd[2], wd[3]), make_uint4(wd[4], wd[5], wd[6], wd[7])};
  }
  __device__ static void partial(const Wt& w, const Act& a, int, int& sumi, int& summ) {
    int s = dot4(w.q0.x, a.a0.x, 0);
    s = dot4(w.q0.y, a.a0.y, s);
    s = dot4(w.q0.z, a.a0.z, s);
    s = dot4(w.q0.w, a.a0.w, s);
    s = dot4(w.q1.x, a.a1.x, s);
    s = dot4(w.q1.y, a.a1.y, s);
    s = dot4(w.q1.z, a.a1.z, s);
    s = dot4(w.q1.w, a.a1.w, s);
    sumi = s;
    summ = 0;
  }
  // acc += rdHalf(w, o) * a.d * s  (quant.nim:771)
  __device__ static float term(const Wt& w, int sumi, int, float ad) {
    return __fmul_rn(__fmul_rn(half_f(w.d), ad), (float)sumi);
  }
};

// Q4_0 (quant.nim:774-786): d qs[16]; one lane per block.
template <>
struct Fmt<2> {
  static constexpr int BL = 32, TS = 18, LPB = 1;
  struct Wt {
    uint4 q;
    uint32_t d;
  };
  struct Act {
    uint4 lo, hi;
    int s8;  // 8 * (sum of the block's 32 activations)
  };
  __device__ static Wt load_w(const uint8_t* blk, int) {
    Wt w;
    w.d = ld_u16(blk);
    uint32_t q[4];
    ld_words_a<4>(blk + 2, q);
    w.q = make_uint4(q[0], q[1], q[2], q[3]);
    return w;
  }
  static constexpr bool HAS_MIN = false;
  __device__ static int group_base(int, int gi) { return 8 * gi; }
  __device__ static Act make_act(const uint32_t (&wd)[8]) {
    Act a;
    a.lo = make_uint4(wd[0], wd[1], wd[2], wd[3]);
    a.hi = make_uint4(wd[4], wd[5], wd[6], wd[7]);
    int s = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) s = dot4(kOnes, wd[k], s);
    a.s8 = 8 * s;
    return a;
  }
  __device__ static void partial(const Wt& w, const Act& a, int, int& sumi, int& summ) {
    const uint32_t Q[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
    const uint32_t AL[4] = {a.lo.x, a.lo.y, a.lo.z, a.lo.w};
    const uint32_t AH[4] = {a.hi.x, a.hi.y, a.hi.z, a.hi.w};
    int s = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      s = dot4(Q[k] & kLo4, AL[k], s);
      s = dot4((Q[k] >> 4) & kLo4, AH[k], s);
    }
    sumi = s - a.s8;
    summ = 0;
  }
  __device__ static float term(const Wt& w, int sumi, int, float ad) {
    return __fmul_rn(__fmul_rn(half_f(w.d), ad), (float)sumi);
  }
};

// A lane's activation slice from the int8 activations of its block.
template <int T>
__device__ __forceinline__ typename Fmt<T>::Act load_act(const int8_t* ablk, int p) {
  uint32_t wd[8];
#pragma unroll
  for (int gi = 0; gi < 4; ++gi) {
    const uint2 v = ld_8(ablk + Fmt<T>::group_base(p, gi));
    wd[2 * gi] = v.x;
    wd[2 * gi + 1] = v.y;
  }
  return Fmt<T>::make_act(wd);
}

// ------------------------------------------------ quantizeAct

// quantizeAct (quant.nim:646-667) of nb * cols activations in blocks of BL:
// each lane owns 4 consecutive values; BL / 4 lanes share a block's maximum.
// Values i4 * 4 .. i4 * 4 + 3 of one lane; BL / 4 consecutive lanes hold a
// block and share its maximum.  Every lane of the wave calls this (the
// maximum is exchanged across lanes); `on` is false past the end.
template <int BL>
__device__ __forceinline__ void quant4(const float* __restrict__ x, int64_t i4, bool on, int8_t* qs,
                                       float* dout) {
  constexpr int G = BL / 4;
  const float4 v = on ? *reinterpret_cast<const float4*>(x + i4 * 4) : make_float4(0.f, 0.f, 0.f, 0.f);
  float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
#pragma unroll
  for (int o = 1; o < G; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
  if (!on) return;
  const float d = __fdiv_rn(amax, 127.0f);
  const float id = d > 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
  const float xv[4] = {v.x, v.y, v.z, v.w};
  uint32_t packed = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float s = __fmul_rn(xv[k], id);
    // int(v + 0.5) for v >= 0, else -int(-v + 0.5): fp32 add, then truncation
    const int t = (int)__fadd_rn(s >= 0.0f ? s : -s, 0.5f);
    const int q = s >= 0.0f ? t : -t;
    packed |= (uint32_t)(q & 0xFF) << (8 * k);
  }
  *reinterpret_cast<uint32_t*>(qs + i4 * 4) = packed;
  if ((i4 & (G - 1)) == 0) dout[(i4 * 4) / BL] = d;
}

template <int BL>
__global__ __launch_bounds__(kLmNT) void quant_act_kernel(const float* __restrict__ x, int64_t n,
                                                         int8_t* __restrict__ qs, float* __restrict__ dout) {
  const int64_t i4 = (int64_t)blockIdx.x * kLmNT + threadIdx.x;  // which 4 values
  quant4<BL>(x, i4, i4 * 4 < n, qs, dout);                       // n is a multiple of BL
}

// ------------------------------------------------ int8 path kernel

struct IntArgs {
  const uint8_t* w;
  int64_t rows, cols, row_bytes;
  const int8_t* aqs;
  const float* ad;
  int nb, nblk, passes, rw;
  float* y;
};

// One wave per group of `rw` rows.  For each row the wave's lanes form the
// integer partials of their slices (64 slices = 2048 weights per pass), the
// 8 lanes of a block add theirs, and the block's last lane writes the block's
// fp32 term to LDS.  Then one lane per row adds its row's terms in block
// order.  Up to kLmNBC activation rows share each load of a weight slice.
template <int T>
__global__ __launch_bounds__(kLmNT) void lm_int_kernel(IntArgs a) {
  using F = Fmt<T>;
  extern __shared__ float s_term[];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int64_t row0 = ((int64_t)blockIdx.x * (kLmNT / 64) + wave) * a.rw;
  if (row0 >= a.rows) return;
  const int nrow = (int)min<int64_t>(a.rw, a.rows - row0);
  const int nbc_max = min(a.nb, kLmNBC);
  float* term = s_term + (size_t)wave * nbc_max * a.rw * a.nblk;
  const int S = (int)(a.cols / 32);  // 32-weight slices per row
  for (int b0 = 0; b0 < a.nb; b0 += kLmNBC) {
    const int nbc = min(kLmNBC, a.nb - b0);
    for (int rr = 0; rr < nrow; ++rr) {
      const uint8_t* rp = a.w + (row0 + rr) * a.row_bytes;
      for (int pass = 0; pass < a.passes; ++pass) {
        const int s = pass * 64 + lane;
        const bool on = s < S;
        const int ib = s / F::LPB, p = s % F::LPB;
        typename F::Wt w{};
        if (on) w = F::load_w(rp + (int64_t)ib * F::TS, p);
        for (int bb = 0; bb < nbc; ++bb) {
          const int64_t brow = b0 + bb;
          int si = 0, sm = 0;
          if (on) {
            const typename F::Act act = load_act<T>(a.aqs + brow * a.cols + (int64_t)ib * F::BL, p);
            F::partial(w, act, p, si, sm);
          }
          if (F::LPB == 8) {
            si = group8_sum(si);
            if (F::HAS_MIN) sm = group8_sum(sm);
          }
          if (on && p == F::LPB - 1)
            term[(bb * a.rw + rr) * a.nblk + ib] = F::term(w, si, sm, a.ad[brow * a.nblk + ib]);
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    for (int idx = lane; idx < nbc * nrow; idx += 64) {
      const int bb = idx / nrow, rr = idx % nrow;
      const float* t = term + (bb * a.rw + rr) * a.nblk;
      float acc = 0.0f;
      for (int ib = 0; ib < a.nblk; ++ib) acc = __fadd_rn(acc, t[ib]);
      a.y[(b0 + bb) * a.rows + row0 + rr] = acc;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
}

struct Int1Args {
  const uint8_t* w;
  int64_t rows, cols, row_bytes;
  const float* x;
  int nb, nblk, rw;
  float* y;
};

// Up to NB hidden states (nb <= NB), cols <= P * 2048: the workgroup
// quantises x into LDS itself (quantizeAct), each lane keeps its NB x P
// activation slices in registers, and the weight slices stream through a ring
// of kRing (row, pass) units, each reloaded right after its use with the unit
// kRing on, so every wave keeps the next unit's loads in flight while it
// computes (deeper rings measured no faster: the grid's waves already cover
// the memory latency).  Each weight slice, loaded once, serves all nb rows.
// Terms and row sums as in lm_int_kernel.
template <int T, int P, int NB>
__global__ __launch_bounds__(kLmNT) void lm_int1_kernel(Int1Args a) {
  using F = Fmt<T>;
  constexpr int SPP = 64 / F::LPB;  // blocks per pass
  constexpr int kRing = P > 2 ? P : 2;  // (row, pass) units in the ring: one row or more
  constexpr int RPI = kRing / P;         // rows per turn of the ring (>= 1)
  extern __shared__ __align__(16) unsigned char s_mem[];
  const int nb = a.nb;
  int8_t* s_act = reinterpret_cast<int8_t*>(s_mem);                          // [nb][cols]
  float* s_ad = reinterpret_cast<float*>(s_mem + (size_t)nb * a.cols);       // [nb][nblk]
  float* s_term = s_ad + ((nb * a.nblk + 3) & ~3);                           // [waves][nb][rw][nblk]
  for (int base = 0; base < (int)(nb * a.cols / 4); base += kLmNT) {
    const int i4 = base + threadIdx.x;
    quant4<F::BL>(a.x, i4, i4 * 4 < nb * a.cols, s_act, s_ad);
  }
  __syncthreads();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  // the rows split evenly over the grid's waves (at most a.rw each)
  const int64_t waves = (int64_t)gridDim.x * (kLmNT / 64), g = (int64_t)blockIdx.x * (kLmNT / 64) + wave;
  const int64_t row0 = g * a.rows / waves;
  const int nrow = (int)((g + 1) * a.rows / waves - row0);
  if (nrow <= 0) return;
  float* term = s_term + (size_t)wave * nb * a.rw * a.nblk;
  const int p = lane % F::LPB;
  typename F::Act act[NB][P];
  float ad[NB][P];
  int ib[P], ibc[P];
#pragma unroll
  for (int ps = 0; ps < P; ++ps) {
    ib[ps] = ps * SPP + lane / F::LPB;
    ibc[ps] = min(ib[ps], a.nblk - 1);  // lanes past the row load a real block and write nothing
  }
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const int bc = min(b, nb - 1);  // rows past nb repeat the last and write nothing
#pragma unroll
    for (int ps = 0; ps < P; ++ps) {
      act[b][ps] = load_act<T>(s_act + (size_t)bc * a.cols + ibc[ps] * F::BL, p);
      ad[b][ps] = s_ad[bc * a.nblk + ibc[ps]];
    }
  }
  const uint8_t* wrow = a.w + row0 * a.row_bytes;  // wave-uniform
  int loff[P];                                     // the lane's block offset in a row
#pragma unroll
  for (int ps = 0; ps < P; ++ps) loff[ps] = ibc[ps] * F::TS;
  auto unit = [&](int rr, int ps) { return wrow + (int64_t)min(rr, nrow - 1) * a.row_bytes + loff[ps]; };
  typename F::Wt ring[kRing];
#pragma unroll
  for (int d = 0; d < kRing; ++d) ring[d] = F::load_w(unit(d / P, d % P), p);
  for (int rr0 = 0; rr0 < nrow; rr0 += RPI) {
#pragma unroll
    for (int d = 0; d < kRing; ++d) {
      const int rr = rr0 + d / P, ps = d % P;
      if constexpr (F::LPB == 8 && NB == 4) {  // (two states: measured faster one at a time)
        // the states' sums reduced together; lane p >= 4 writes state st's term
        int si[NB], sm[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) F::partial(ring[d], act[b][ps], p, si[b], sm[b]);
        const int ti = group8_sum_states<NB>(si, p);
        const int tm = F::HAS_MIN ? group8_sum_states<NB>(sm, p) : 0;
        const int st = group8_state<NB>(p);
        float adv = ad[0][ps];
#pragma unroll
        for (int b = 1; b < NB; ++b) adv = st == b ? ad[b][ps] : adv;
        if (p >= 4 && st < nb && rr < nrow && ib[ps] < a.nblk)
          term[(st * a.rw + rr) * a.nblk + ib[ps]] = F::term(ring[d], ti, tm, adv);
      } else {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          int si, sm;
          F::partial(ring[d], act[b][ps], p, si, sm);
          if (F::LPB == 8) {
            si = group8_sum(si);
            if (F::HAS_MIN) sm = group8_sum(sm);
          }
          if (b < nb && rr < nrow && ib[ps] < a.nblk && p == F::LPB - 1)
            term[(b * a.rw + rr) * a.nblk + ib[ps]] = F::term(ring[d], si, sm, ad[b][ps]);
        }
      }
      // the slot's next unit, kRing units on: loaded into the registers just
      // freed, so the ring needs no copies between turns
      ring[d] = F::load_w(unit(rr + RPI, ps), p);
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  for (int idx = lane; idx < nb * nrow; idx += 64) {
    const int b = idx / nrow, rr = idx - b * nrow;
    const float* t = term + (b * a.rw + rr) * a.nblk;
    float acc = 0.0f;
    for (int j = 0; j < a.nblk; ++j) acc = __fadd_rn(acc, t[j]);
    a.y[(int64_t)b * a.rows + row0 + rr] = acc;
  }
}

// ------------------------------------------------ float path

// One weight of a dequantised row (dequantBlock, quant.nim:164-334): element
// e of row `rp`, with the reference's fp32 operations.
template <int T>
__device__ __forceinline__ float deq1(const uint8_t* __restrict__ rp, int64_t e);

template <>
__device__ __forceinline__ float deq1<0>(const uint8_t* rp, int64_t e) {  // F32
  float v;
  __builtin_memcpy(&v, rp + 4 * e, 4);
  return v;
}
template <>
__device__ __forceinline__ float deq1<1>(const uint8_t* rp, int64_t e) {  // F16
  return half_f(ld_u16(rp + 2 * e));
}
template <>
__device__ __forceinline__ float deq1<30>(const uint8_t* rp, int64_t e) {  // BF16
  return __uint_as_float(ld_u16(rp + 2 * e) << 16);
}
template <>
__device__ __forceinline__ float deq1<2>(const uint8_t* rp, int64_t e) {  // Q4_0 :167-172
  const uint8_t* b = rp + 18 * (e >> 5);
  const int i = (int)(e & 31);
  const uint32_t q = b[2 + (i & 15)];
  const int v = (int)(i < 16 ? (q & 0xF) : (q >> 4)) - 8;
  return __fmul_rn((float)v, half_f(ld_u16(b)));
}
template <>
__device__ __forceinline__ float deq1<3>(const uint8_t* rp, int64_t e) {  // Q4_1 :173-179
  const uint8_t* b = rp + 20 * (e >> 5);
  const int i = (int)(e & 31);
  const uint32_t q = b[4 + (i & 15)];
  const uint32_t v = i < 16 ? (q & 0xF) : (q >> 4);
  return __fadd_rn(__fmul_rn((float)v, half_f(ld_u16(b))), half_f(ld_u16(b + 2)));
}
template <>
__device__ __forceinline__ float deq1<6>(const uint8_t* rp, int64_t e) {  // Q5_0 :180-188
  const uint8_t* b = rp + 22 * (e >> 5);
  const int i = (int)(e & 31), j = i & 15;
  uint32_t qh;
  __builtin_memcpy(&qh, b + 2, 4);
  const uint32_t q = b[6 + j];
  const uint32_t v = i < 16 ? ((q & 0xF) | (((qh >> j) << 4) & 0x10)) : ((q >> 4) | ((qh >> (j + 12)) & 0x10));
  return __fmul_rn((float)((int)v - 16), half_f(ld_u16(b)));
}
template <>
__device__ __forceinline__ float deq1<7>(const uint8_t* rp, int64_t e) {  // Q5_1 :189-198
  const uint8_t* b = rp + 24 * (e >> 5);
  const int i = (int)(e & 31), j = i & 15;
  uint32_t qh;
  __builtin_memcpy(&qh, b + 4, 4);
  const uint32_t q = b[8 + j];
  const uint32_t v = i < 16 ? ((q & 0xF) | (((qh >> j) << 4) & 0x10)) : ((q >> 4) | ((qh >> (j + 12)) & 0x10));
  return __fadd_rn(__fmul_rn((float)v, half_f(ld_u16(b))), half_f(ld_u16(b + 2)));
}
template <>
__device__ __forceinline__ float deq1<8>(const uint8_t* rp, int64_t e) {  // Q8_0 :199-202
  const uint8_t* b = rp + 34 * (e >> 5);
  return __fmul_rn((float)(int8_t)b[2 + (e & 31)], half_f(ld_u16(b)));
}
template <>
__device__ __forceinline__ float deq1<10>(const uint8_t* rp, int64_t e) {  // Q2_K :207-228
  const uint8_t* b = rp + 84 * (e >> 8);
  const int i = (int)(e & 255), n = i >> 7, j = (i >> 5) & 3, l = i & 31;
  const uint32_t sc = b[i >> 4];
  const float dl = __fmul_rn(half_f(ld_u16(b + 80)), (float)(sc & 0xF));
  const float ml = __fmul_rn(half_f(ld_u16(b + 82)), (float)(sc >> 4));
  const uint32_t q = (b[16 + 32 * n + l] >> (2 * j)) & 3;
  return __fsub_rn(__fmul_rn(dl, (float)q), ml);
}
template <>
__device__ __forceinline__ float deq1<11>(const uint8_t* rp, int64_t e) {  // Q3_K :229-260
  const uint8_t* b = rp + 110 * (e >> 8);
  const int i = (int)(e & 255), n = i >> 7, j = (i >> 5) & 3, l = i & 31, s = i >> 4;
  // the 6-bit scale s: low 4 bits from byte s % 8 (low nibble for s < 8),
  // high 2 bits from byte 8 + s % 4 at bit 2 (s / 4)
  const uint32_t lo = s < 8 ? (b[96 + s] & 0xF) : (b[96 + s - 8] >> 4);
  const uint32_t hi = (b[104 + (s & 3)] >> (2 * (s >> 2))) & 3;
  const int scale = (int)(lo | (hi << 4));
  const float dl = __fmul_rn(half_f(ld_u16(b + 108)), (float)(scale - 32));
  const int hv = (b[l] & (1u << (4 * n + j))) != 0 ? 0 : 4;
  const int q = (int)((b[32 + 32 * n + l] >> (2 * j)) & 3) - hv;
  return __fmul_rn(dl, (float)q);
}
template <bool FIVE>
__device__ __forceinline__ float deq1_k45(const uint8_t* rp, int64_t e) {  // :261-302
  const uint8_t* b = rp + (FIVE ? 176 : 144) * (e >> 8);
  const int i = (int)(e & 255), jj = i >> 6, hi = (i >> 5) & 1, l = i & 31;
  int sc, mn;
  const uint4 hd = ld_16(b);
  FmtK45<FIVE>::scale_min(hd, 2 * jj + hi, sc, mn);
  const float d1 = __fmul_rn(half_f(hd.x & 0xFFFF), (float)sc);
  const float m1 = __fmul_rn(half_f(hd.x >> 16), (float)mn);
  const uint32_t byte = b[(FIVE ? 48 : 16) + 32 * jj + l];
  int q = (int)(hi ? (byte >> 4) : (byte & 0xF));
  if (FIVE) q += ((b[16 + l] >> (2 * jj + hi)) & 1) ? 16 : 0;
  return __fsub_rn(__fmul_rn(d1, (float)q), m1);
}
template <>
__device__ __forceinline__ float deq1<12>(const uint8_t* rp, int64_t e) {
  return deq1_k45<false>(rp, e);
}
template <>
__device__ __forceinline__ float deq1<13>(const uint8_t* rp, int64_t e) {
  return deq1_k45<true>(rp, e);
}
template <>
__device__ __forceinline__ float deq1<14>(const uint8_t* rp, int64_t e) {  // Q6_K :303-320
  const uint8_t* b = rp + 210 * (e >> 8);
  const int i = (int)(e & 255), n = i >> 7, m = (i >> 5) & 3, l = i & 31;
  const uint32_t qlb = b[64 * n + l + 32 * (m & 1)];
  const uint32_t nib = (m & 2) ? (qlb >> 4) : (qlb & 0xF);
  const uint32_t hb = (b[128 + 32 * n + l] >> (2 * m)) & 3;
  const int q = (int)(nib | (hb << 4)) - 32;
  const int sc = (int8_t)b[192 + 8 * n + (l >> 4) + 2 * m];
  return __fmul_rn(__fmul_rn(half_f(ld_u16(b + 208)), (float)sc), (float)q);
}
template <>
__device__ __forceinline__ float deq1<15>(const uint8_t* rp, int64_t e) {  // Q8_K :321-324
  const uint8_t* b = rp + 292 * (e >> 8);
  float d;
  __builtin_memcpy(&d, b, 4);
  return __fmul_rn((float)(int8_t)b[4 + (e & 255)], d);
}

struct FloatArgs {
  const uint8_t* w;
  int64_t rows, cols, row_bytes;
  const float* x;
  int nb;
  float* y;
};

// Eight consecutive weights e0 .. e0 + 7 of a dequantised row (e0 a multiple
// of 8; past `cols` they read 0 without touching memory).
template <int T>
__device__ __forceinline__ void deq8(const uint8_t* __restrict__ rp, int64_t e0, int64_t cols, float (&w)[8]) {
  if (e0 + 8 <= cols) {
    if constexpr (T == 0) {  // F32: two 16-byte loads
      const uint4 a = ld_16(rp + 4 * e0), b = ld_16(rp + 4 * e0 + 16);
      const uint32_t u[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int j = 0; j < 8; ++j) w[j] = __uint_as_float(u[j]);
    } else if constexpr (T == 1 || T == 30) {  // F16, BF16: one 16-byte load
      const uint4 a = ld_16(rp + 2 * e0);
      const uint32_t u[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr (T == 1) {
          w[2 * j] = half_f(u[j] & 0xFFFF);
          w[2 * j + 1] = half_f(u[j] >> 16);
        } else {
          w[2 * j] = __uint_as_float(u[j] << 16);
          w[2 * j + 1] = __uint_as_float(u[j] & 0xFFFF0000u);
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) w[j] = deq1<T>(rp, e0 + j);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) w[j] = e0 + j < cols ? deq1<T>(rp, e0 + j) : 0.0f;
  }
}

// The 2- and 4-byte types' eight weights as loaded (F32: both pieces; F16,
// BF16: `a`), so that a segment's load can go out one segment ahead.
struct Raw8 {
  uint4 a, b;
};
template <int T>
__device__ __forceinline__ Raw8 raw8(const uint8_t* __restrict__ rp, int64_t e0, int64_t cols) {
  Raw8 r{make_uint4(0u, 0u, 0u, 0u), make_uint4(0u, 0u, 0u, 0u)};
  if (e0 + 8 <= cols) {
    if constexpr (T == 0) {
      r.a = ld_16(rp + 4 * e0);
      r.b = ld_16(rp + 4 * e0 + 16);
    } else {
      r.a = ld_16(rp + 2 * e0);
    }
  }
  return r;
}
template <int T>
__device__ __forceinline__ void cvt8(const Raw8& r, float (&w)[8]) {
  if constexpr (T == 0) {
    const uint32_t u[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) w[j] = __uint_as_float(u[j]);
  } else {
    const uint32_t u[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (T == 1) {
        w[2 * j] = half_f(u[j] & 0xFFFF);
        w[2 * j + 1] = half_f(u[j] >> 16);
      } else {
        w[2 * j] = __uint_as_float(u[j] << 16);
        w[2 * j + 1] = __uint_as_float(u[j] & 0xFFFF0000u);
      }
    }
  }
}

// dotF32 (quant.nim:362-374) of each dequantised row with each x row: lane
// k of an aligned group of 8 runs chain k (weights k, k + 8, ...), lane 0
// takes the cols % 8 tail, and the chains combine as the reference adds them.
// The row is read in 16-byte pieces: the 8 lanes of a row dequantise 64
// consecutive weights (8 each) and pass them through LDS so that lane k holds
// chain k's 8 of them; for the 2- and 4-byte types the next 64 are requested
// before these are used.  32 rows per workgroup; up to kLmNBC activation rows
// per pass over the row.
template <int T, bool XLDS>
__global__ __launch_bounds__(kLmNT) void lm_float_kernel(FloatArgs a) {
  __shared__ float s_t[kLmNT / 8][8][9];  // per row group: [lane][its 8 weights], padded
  // XLDS: the activations of the pass, chain-major: xt[bb][k][j] = x[bb][8 j + k]
  extern __shared__ __align__(16) float xt[];
  const int k = threadIdx.x & 7, grp = threadIdx.x >> 3;
  const int64_t r = (int64_t)blockIdx.x * (kLmNT / 8) + grp;
  const bool live = r < a.rows;  // (groups past the last row still take part in the exchanges)
  const uint8_t* rp = a.w + min(r, a.rows - 1) * a.row_bytes;
  const int64_t c8 = a.cols & ~(int64_t)7;
  const int s8 = (int)(c8 / 8);  // steps of a chain
  for (int b0 = 0; b0 < a.nb; b0 += kLmNBC) {
    const int nbc = min(kLmNBC, a.nb - b0);
    float acc[kLmNBC] = {0.0f, 0.0f, 0.0f, 0.0f};
    const float* xb = a.x + (int64_t)b0 * a.cols;
    if constexpr (XLDS) {
      __syncthreads();  // the previous pass is done with xt
      for (int i = threadIdx.x; i < nbc * (int)c8; i += kLmNT) {
        const int bb = i / (int)c8, e = i - bb * (int)c8;
        xt[(bb * 8 + (e & 7)) * s8 + (e >> 3)] = xb[(int64_t)bb * a.cols + e];
      }
      __syncthreads();
    }
    // F32, F16, BF16: the next segment's 16-byte pieces are requested before
    // this segment is used
    constexpr bool kPre = T == 0 || T == 1 || T == 30;
    Raw8 nxt{};
    if constexpr (kPre) nxt = raw8<T>(rp, 8 * k, c8);
    for (int64_t seg = 0; seg < c8; seg += 64) {
      float w[8];
      if constexpr (kPre) {
        const Raw8 cur = nxt;
        if (seg + 64 < c8) nxt = raw8<T>(rp, seg + 64 + 8 * k, c8);
        cvt8<T>(cur, w);
      } else {
        deq8<T>(rp, seg + 8 * k, c8, w);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) s_t[grp][k][j] = w[j];
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      // chain k's weights of this segment: element seg + 8 j + k sits at
      // lane j's slot k
      float cw[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) cw[j] = s_t[grp][j][k];
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const int j0 = (int)(seg >> 3);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int64_t e = seg + 8 * j + k;
        if (e < c8) {
#pragma unroll
          for (int bb = 0; bb < kLmNBC; ++bb)
            if (bb < nbc) {
              const float xv = XLDS ? xt[(bb * 8 + k) * s8 + j0 + j] : xb[bb * a.cols + e];
              acc[bb] = __fadd_rn(acc[bb], __fmul_rn(cw[j], xv));
            }
        }
      }
    }
    if (k == 0) {
      for (int64_t e = c8; e < a.cols; ++e) {
        const float w = deq1<T>(rp, e);
#pragma unroll
        for (int bb = 0; bb < kLmNBC; ++bb)
          if (bb < nbc) acc[bb] = __fadd_rn(acc[bb], __fmul_rn(w, xb[bb * a.cols + e]));
      }
    }
#pragma unroll
    for (int bb = 0; bb < kLmNBC; ++bb) {
      const float t = group8_dotf32_combine(acc[bb]);
      if (live && bb < nbc && k == 6) a.y[(int64_t)(b0 + bb) * a.rows + r] = t;
    }
  }
}

// ------------------------------------------------ LoRA (model.nim:189-200)

// tmp[b, i] = dotF32(A[i, :], x[b, :]): one group of 8 lanes per (b, i).
__global__ __launch_bounds__(kLmNT) void lora_tmp_kernel(const float* __restrict__ A, const float* __restrict__ x,
                                                        int64_t cols, int nb, int rank, float* __restrict__ tmp) {
  const int k = threadIdx.x & 7;
  const int64_t pair = (int64_t)blockIdx.x * (kLmNT / 8) + (threadIdx.x >> 3);
  if (pair >= (int64_t)nb * rank) return;
  const int b = (int)(pair / rank), i = (int)(pair % rank);
  const float* ar = A + (int64_t)i * cols;
  const float* xr = x + (int64_t)b * cols;
  const int64_t c8 = cols & ~(int64_t)7;
  float acc = 0.0f;
  for (int64_t e = k; e < c8; e += 8) acc = __fadd_rn(acc, __fmul_rn(ar[e], xr[e]));
  if (k == 0)
    for (int64_t e = c8; e < cols; ++e) acc = __fadd_rn(acc, __fmul_rn(ar[e], xr[e]));
  const float t = group8_dotf32_combine(acc);
  if (k == 6) tmp[pair] = t;
}

// y[b, r] += scale * (sum over i, in order, of B[r, i] * tmp[b, i])
__global__ __launch_bounds__(kLmNT) void lora_apply_kernel(const float* __restrict__ Bm, const float* __restrict__ tmp,
                                                          int64_t rows, int nb, int rank, float scale,
                                                          float* __restrict__ y) {
  const int64_t idx = (int64_t)blockIdx.x * kLmNT + threadIdx.x;
  if (idx >= (int64_t)nb * rows) return;
  const int b = (int)(idx / rows);
  const int64_t r = idx % rows;
  float s = 0.0f;
  for (int i = 0; i < rank; ++i) s = __fadd_rn(s, __fmul_rn(Bm[r * rank + i], tmp[(int64_t)b * rank + i]));
  y[idx] = __fadd_rn(y[idx], __fmul_rn(scale, s));
}

// ------------------------------------------------ launch helpers

// Compute units of the current device and resident workgroups of a kernel
// per CU, looked up once per process (one device's shape is assumed).
int device_cus() {
  static int n = 0;
  if (n == 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) !=
                                                 hipSuccess || n <= 0)
      n = 256;
  }
  return n;
}

template <int T, int P, int NB>
hipError_t launch_int1(const LmHeadCall& c, int nblk, hipStream_t s) {
  Int1Args a{static_cast<const uint8_t*>(c.w), c.rows, c.cols, c.row_bytes, c.x, c.nb, nblk, 0, c.y};
  // rows per wave: at most what a 4 KiB term buffer holds (and 32)
  int cap = 32;
  while (cap > 1 && (int64_t)cap * NB * nblk * 4 > 4096) cap >>= 1;
  const size_t lds = (size_t)c.nb * c.cols + 4 * (size_t)((c.nb * nblk + 3) & ~3) +
                     (size_t)(kLmNT / 64) * c.nb * cap * nblk * 4;
  static int occ = 0;  // resident workgroups per CU at the largest LDS size of this instance
  if (occ == 0) {
    const size_t lds_max = (size_t)NB * c.cols + 4 * (size_t)((NB * nblk + 3) & ~3) +
                           (size_t)(kLmNT / 64) * NB * cap * nblk * 4;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, lm_int1_kernel<T, P, NB>, kLmNT, lds_max) !=
            hipSuccess || occ <= 0)
      occ = 4;
  }
  // one resident round of workgroups with the rows split evenly over their
  // waves, unless that gives a wave more rows than the term buffer holds
  const int64_t waves_min = (c.rows + cap - 1) / cap;
  int64_t waves = std::max<int64_t>((int64_t)device_cus() * occ * (kLmNT / 64), waves_min);
  waves = std::min<int64_t>(waves, c.rows);
  const int64_t grid = (waves + kLmNT / 64 - 1) / (kLmNT / 64);
  a.rw = (int)((c.rows + grid * (kLmNT / 64) - 1) / (grid * (kLmNT / 64)));
  hipLaunchKernelGGL((lm_int1_kernel<T, P, NB>), dim3((unsigned)grid), dim3(kLmNT), lds, s, a);
  return hipGetLastError();
}

template <int T>
hipError_t launch_int(const LmHeadCall& c, hipStream_t s) {
  using F = Fmt<T>;
  const int nblk = (int)(c.cols / F::BL);
  const int passes = (int)((c.cols / 32 + 63) / 64);
  // up to four hidden states with each weight slice loaded once for all;
  // activation slices held in registers for nb x passes <= 4
  if (c.nb == 1 && passes <= 4) {
    if (passes == 1) return launch_int1<T, 1, 1>(c, nblk, s);
    if (passes == 2) return launch_int1<T, 2, 1>(c, nblk, s);
    return launch_int1<T, 4, 1>(c, nblk, s);
  }
  if (c.nb == 2 && passes <= 2) return passes == 1 ? launch_int1<T, 1, 2>(c, nblk, s) : launch_int1<T, 2, 2>(c, nblk, s);
  if (c.nb <= 4 && passes == 1) return launch_int1<T, 1, 4>(c, nblk, s);
  const int64_t n = (int64_t)c.nb * c.cols;
  const int64_t qgrid = (n / 4 + kLmNT - 1) / kLmNT;
  hipLaunchKernelGGL(quant_act_kernel<F::BL>, dim3((unsigned)qgrid), dim3(kLmNT), 0, s, c.x, n, c.act_qs, c.act_d);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  IntArgs a;
  a.w = static_cast<const uint8_t*>(c.w);
  a.rows = c.rows;
  a.cols = c.cols;
  a.row_bytes = c.row_bytes;
  a.aqs = c.act_qs;
  a.ad = c.act_d;
  a.nb = c.nb;
  a.nblk = nblk;
  a.passes = passes;
  a.y = c.y;
  const int nbc = std::min(c.nb, kLmNBC);
  // rows per wave: 16, fewer when the per-wave term buffer would pass 4 KiB
  int rw = 16;
  while (rw > 1 && (int64_t)nbc * rw * a.nblk * 4 > 4096) rw >>= 1;
  a.rw = rw;
  const size_t lds = (size_t)(kLmNT / 64) * nbc * rw * a.nblk * sizeof(float);
  const int64_t grid = (c.rows + (int64_t)rw * (kLmNT / 64) - 1) / ((int64_t)rw * (kLmNT / 64));
  hipLaunchKernelGGL(lm_int_kernel<T>, dim3((unsigned)grid), dim3(kLmNT), lds, s, a);
  return hipGetLastError();
}

template <int T>
hipError_t launch_float(const LmHeadCall& c, hipStream_t s) {
  FloatArgs a{static_cast<const uint8_t*>(c.w), c.rows, c.cols, c.row_bytes, c.x, c.nb, c.y};
  const int64_t grid = (c.rows + kLmNT / 8 - 1) / (kLmNT / 8);
  // the activations of a pass in LDS when they fit in 32 KiB
  const size_t xbytes = (size_t)std::min(c.nb, kLmNBC) * (size_t)(c.cols & ~(int64_t)7) * 4;
  if (xbytes <= 32768)
    hipLaunchKernelGGL((lm_float_kernel<T, true>), dim3((unsigned)grid), dim3(kLmNT), xbytes, s, a);
  else
    hipLaunchKernelGGL((lm_float_kernel<T, false>), dim3((unsigned)grid), dim3(kLmNT), 0, s, a);
  return hipGetLastError();
}

}  // namespace

int lm_act_block_len(int type) {
  switch (type) {
    case 12: case 13: case 14: return 256;
    case 8: case 2: return 32;
    default: return 0;
  }
}

bool lm_type_supported(int type) {
  switch (type) {
    case 0: case 1: case 2: case 3: case 6: case 7: case 8: case 10: case 11: case 12: case 13: case 14:
    case 15: case 30:
      return true;
    default:
      return false;
  }
}

hipError_t launch_lm_head(const LmHeadCall& c, hipStream_t s) {
  hipError_t e = hipSuccess;
  if (c.use_act) {
    switch (c.type) {
      case 14: e = launch_int<14>(c, s); break;
      case 12: e = launch_int<12>(c, s); break;
      case 13: e = launch_int<13>(c, s); break;
      case 8: e = launch_int<8>(c, s); break;
      case 2: e = launch_int<2>(c, s); break;
      default: return hipErrorInvalidValue;
    }
  } else {
    switch (c.type) {
      case 0: e = launch_float<0>(c, s); break;
      case 1: e = launch_float<1>(c, s); break;
      case 30: e = launch_float<30>(c, s); break;
      case 2: e = launch_float<2>(c, s); break;
      case 3: e = launch_float<3>(c, s); break;
      case 6: e = launch_float<6>(c, s); break;
      case 7: e = launch_float<7>(c, s); break;
      case 8: e = launch_float<8>(c, s); break;
      case 10: e = launch_float<10>(c, s); break;
      case 11: e = launch_float<11>(c, s); break;
      case 12: e = launch_float<12>(c, s); break;
      case 13: e = launch_float<13>(c, s); break;
      case 14: e = launch_float<14>(c, s); break;
      case 15: e = launch_float<15>(c, s); break;
      default: return hipErrorInvalidValue;
    }
  }
  if (e != hipSuccess) return e;
  if (c.lora_rank > 0) {
    const int64_t pairs = (int64_t)c.nb * c.lora_rank;
    hipLaunchKernelGGL(lora_tmp_kernel, dim3((unsigned)((pairs + kLmNT / 8 - 1) / (kLmNT / 8))), dim3(kLmNT), 0, s,
                       c.lora_a, c.x, c.cols, c.nb, c.lora_rank, c.lora_tmp);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    const int64_t outs = (int64_t)c.nb * c.rows;
    hipLaunchKernelGGL(lora_apply_kernel, dim3((unsigned)((outs + kLmNT - 1) / kLmNT)), dim3(kLmNT), 0, s, c.lora_b,
                       c.lora_tmp, c.rows, c.nb, c.lora_rank, c.lora_scale, c.y);
    e = hipGetLastError();
  }
  return e;
}

}  // namespace nls
