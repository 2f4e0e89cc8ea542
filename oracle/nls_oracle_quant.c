/*
 * nls_oracle_quant.c -- CPU restatement of nimllm's output projection.
 * TEST INFRASTRUCTURE ONLY (see nls_oracle_quant.h for what it follows).
 */
#include "nls_oracle_quant.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

typedef const uint8_t* bytes;

/* quant.nim:38-63 */
int32_t nlo_block_size(int32_t t) {
  switch (t) {
    case NLO_F32: case NLO_F16: case NLO_BF16: return 1;
    case NLO_Q4_0: case NLO_Q4_1: case NLO_Q5_0: case NLO_Q5_1: case NLO_Q8_0: return 32;
    case NLO_Q2_K: case NLO_Q3_K: case NLO_Q4_K: case NLO_Q5_K: case NLO_Q6_K: case NLO_Q8_K:
      return 256;
    default: return 0;
  }
}

int32_t nlo_type_size(int32_t t) {
  switch (t) {
    case NLO_F32: return 4;
    case NLO_F16: case NLO_BF16: return 2;
    case NLO_Q4_0: return 18;
    case NLO_Q4_1: return 20;
    case NLO_Q5_0: return 22;
    case NLO_Q5_1: return 24;
    case NLO_Q8_0: return 34;
    case NLO_Q2_K: return 84;
    case NLO_Q3_K: return 110;
    case NLO_Q4_K: return 144;
    case NLO_Q5_K: return 176;
    case NLO_Q6_K: return 210;
    case NLO_Q8_K: return 292;
    default: return 0;
  }
}

/* quant.nim:65-70 */
int64_t nlo_row_bytes(int32_t t, int64_t n) {
  const int32_t bs = nlo_block_size(t);
  if (bs == 0 || n % bs != 0) return -1;
  return (n / bs) * nlo_type_size(t);
}

/* halfToFloatSlow (quant.nim:83-98); the reference reads halves through a
 * table built from it (:100-110). */
float nlo_half_to_float(uint16_t h) {
  const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  const uint32_t ex = ((uint32_t)h >> 10) & 0x1F;
  const uint32_t mant = (uint32_t)h & 0x3FF;
  uint32_t bits;
  if (ex == 0) {
    const float v = (float)((double)mant * pow(2.0, -24.0));
    return sign != 0 ? -v : v;
  } else if (ex == 31) {
    bits = sign | 0x7F800000u | (mant << 13);
  } else {
    bits = sign | ((ex + 127 - 15) << 23) | (mant << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

/* bf16ToFloat (quant.nim:138) */
static float bf16_to_float(uint16_t h) {
  const uint32_t bits = (uint32_t)h << 16;
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

/* rd16 / rdHalf (quant.nim:144-147) */
static uint16_t rd16(bytes p, int o) { return (uint16_t)(p[o] | (p[o + 1] << 8)); }
static float rd_half(bytes p, int o) { return nlo_half_to_float(rd16(p, o)); }

/* getScaleMinK4 (quant.nim:156-162) */
static void scale_min_k4(int j, bytes q, int o, uint8_t* d, uint8_t* m) {
  if (j < 4) {
    *d = q[o + j] & 63;
    *m = q[o + j + 4] & 63;
  } else {
    *d = (uint8_t)((q[o + j + 4] & 0xF) | ((q[o + j - 4] >> 6) << 4));
    *m = (uint8_t)((q[o + j + 4] >> 4) | ((q[o + j] >> 6) << 4));
  }
}

/* dequantBlock (quant.nim:164-334): one block at b into y. */
static void dequant_block(int32_t t, bytes b, float* y) {
  switch (t) {
    case NLO_Q4_0: { /* :167-172 */
      const float d = rd_half(b, 0);
      for (int j = 0; j < 16; ++j) {
        const uint8_t q = b[2 + j];
        y[j] = (float)((int)(q & 0xF) - 8) * d;
        y[j + 16] = (float)((int)(q >> 4) - 8) * d;
      }
      break;
    }
    case NLO_Q4_1: { /* :173-179 */
      const float d = rd_half(b, 0);
      const float m = rd_half(b, 2);
      for (int j = 0; j < 16; ++j) {
        const uint8_t q = b[4 + j];
        y[j] = (float)(q & 0xF) * d + m;
        y[j + 16] = (float)(q >> 4) * d + m;
      }
      break;
    }
    case NLO_Q5_0: { /* :180-188 */
      const float d = rd_half(b, 0);
      const uint32_t qh = (uint32_t)b[2] | ((uint32_t)b[3] << 8) | ((uint32_t)b[4] << 16) |
                          ((uint32_t)b[5] << 24);
      for (int j = 0; j < 16; ++j) {
        const uint32_t xh0 = ((qh >> j) << 4) & 0x10;
        const uint32_t xh1 = (qh >> (j + 12)) & 0x10;
        const uint8_t q = b[6 + j];
        y[j] = (float)((int)((uint32_t)(q & 0xF) | xh0) - 16) * d;
        y[j + 16] = (float)((int)((uint32_t)(q >> 4) | xh1) - 16) * d;
      }
      break;
    }
    case NLO_Q5_1: { /* :189-198 */
      const float d = rd_half(b, 0);
      const float m = rd_half(b, 2);
      const uint32_t qh = (uint32_t)b[4] | ((uint32_t)b[5] << 8) | ((uint32_t)b[6] << 16) |
                          ((uint32_t)b[7] << 24);
      for (int j = 0; j < 16; ++j) {
        const uint32_t xh0 = ((qh >> j) << 4) & 0x10;
        const uint32_t xh1 = (qh >> (j + 12)) & 0x10;
        const uint8_t q = b[8 + j];
        y[j] = (float)((uint32_t)(q & 0xF) | xh0) * d + m;
        y[j + 16] = (float)((uint32_t)(q >> 4) | xh1) * d + m;
      }
      break;
    }
    case NLO_Q8_0: { /* :199-202 */
      const float d = rd_half(b, 0);
      for (int j = 0; j < 32; ++j) y[j] = (float)(int8_t)b[2 + j] * d;
      break;
    }
    case NLO_Q2_K: { /* :207-228: scales[16] qs[64] d dmin */
      const float d = rd_half(b, 80);
      const float mn = rd_half(b, 82);
      int isc = 0, yo = 0, qo = 16;
      for (int n = 0; n < 2; ++n) {
        int shift = 0;
        for (int j = 0; j < 4; ++j) {
          uint8_t sc = b[isc++];
          float dl = d * (float)(sc & 0xF);
          float ml = mn * (float)(sc >> 4);
          for (int l = 0; l < 16; ++l) y[yo++] = dl * (float)((b[qo + l] >> shift) & 3) - ml;
          sc = b[isc++];
          dl = d * (float)(sc & 0xF);
          ml = mn * (float)(sc >> 4);
          for (int l = 0; l < 16; ++l) y[yo++] = dl * (float)((b[qo + l + 16] >> shift) & 3) - ml;
          shift += 2;
        }
        qo += 32;
      }
      break;
    }
    case NLO_Q3_K: { /* :229-260: hmask[32] qs[64] scales[12] d */
      const float dAll = rd_half(b, 108);
      uint32_t aux[4] = {0, 0, 0, 0};
      memcpy(aux, b + 96, 12);
      const uint32_t kmask1 = 0x03030303u, kmask2 = 0x0f0f0f0fu;
      const uint32_t tmp = aux[2];
      aux[2] = ((aux[0] >> 4) & kmask2) | (((tmp >> 4) & kmask1) << 4);
      aux[3] = ((aux[1] >> 4) & kmask2) | (((tmp >> 6) & kmask1) << 4);
      aux[0] = (aux[0] & kmask2) | (((tmp >> 0) & kmask1) << 4);
      aux[1] = (aux[1] & kmask2) | (((tmp >> 2) & kmask1) << 4);
      int8_t scales[16];
      memcpy(scales, aux, 16);
      uint8_t m = 1;
      int isc = 0, yo = 0, qo = 32;
      for (int n = 0; n < 2; ++n) {
        int shift = 0;
        for (int j = 0; j < 4; ++j) {
          float dl = dAll * (float)((int)scales[isc] - 32);
          ++isc;
          for (int l = 0; l < 16; ++l) {
            const int hv = (b[l] & m) != 0 ? 0 : 4;
            y[yo++] = dl * (float)((int)((b[qo + l] >> shift) & 3) - hv);
          }
          dl = dAll * (float)((int)scales[isc] - 32);
          ++isc;
          for (int l = 0; l < 16; ++l) {
            const int hv = (b[l + 16] & m) != 0 ? 0 : 4;
            y[yo++] = dl * (float)((int)((b[qo + l + 16] >> shift) & 3) - hv);
          }
          shift += 2;
          m = (uint8_t)(m << 1);
        }
        qo += 32;
      }
      break;
    }
    case NLO_Q4_K: { /* :261-278: d dmin scales[12] qs[128] */
      const float d = rd_half(b, 0);
      const float mn = rd_half(b, 2);
      int isc = 0, qo = 16, yo = 0;
      for (int jj = 0; jj < 4; ++jj) {
        uint8_t sc, mm;
        scale_min_k4(isc, b, 4, &sc, &mm);
        const float d1 = d * (float)sc;
        const float m1 = mn * (float)mm;
        scale_min_k4(isc + 1, b, 4, &sc, &mm);
        const float d2 = d * (float)sc;
        const float m2 = mn * (float)mm;
        for (int l = 0; l < 32; ++l) y[yo + l] = d1 * (float)(b[qo + l] & 0xF) - m1;
        for (int l = 0; l < 32; ++l) y[yo + 32 + l] = d2 * (float)(b[qo + l] >> 4) - m2;
        qo += 32;
        yo += 64;
        isc += 2;
      }
      break;
    }
    case NLO_Q5_K: { /* :279-302: d dmin scales[12] qh[32] qs[128] */
      const float d = rd_half(b, 0);
      const float mn = rd_half(b, 2);
      int isc = 0, qo = 48, yo = 0;
      uint8_t u1 = 1, u2 = 2;
      for (int jj = 0; jj < 4; ++jj) {
        uint8_t sc, mm;
        scale_min_k4(isc, b, 4, &sc, &mm);
        const float d1 = d * (float)sc;
        const float m1 = mn * (float)mm;
        scale_min_k4(isc + 1, b, 4, &sc, &mm);
        const float d2 = d * (float)sc;
        const float m2 = mn * (float)mm;
        for (int l = 0; l < 32; ++l) {
          const int h = (b[16 + l] & u1) != 0 ? 16 : 0;
          y[yo + l] = d1 * (float)((int)(b[qo + l] & 0xF) + h) - m1;
        }
        for (int l = 0; l < 32; ++l) {
          const int h = (b[16 + l] & u2) != 0 ? 16 : 0;
          y[yo + 32 + l] = d2 * (float)((int)(b[qo + l] >> 4) + h) - m2;
        }
        qo += 32;
        yo += 64;
        isc += 2;
        u1 = (uint8_t)(u1 << 2);
        u2 = (uint8_t)(u2 << 2);
      }
      break;
    }
    case NLO_Q6_K: { /* :303-320: ql[128] qh[64] scales[16] d */
      const float d = rd_half(b, 208);
      int qlo = 0, qho = 128, sco = 192, yo = 0;
      for (int n = 0; n < 2; ++n) {
        for (int l = 0; l < 32; ++l) {
          const int isc = l / 16;
          const uint8_t qh = b[qho + l];
          const int q1 = (int)((b[qlo + l] & 0xF) | (((qh >> 0) & 3) << 4)) - 32;
          const int q2 = (int)((b[qlo + l + 32] & 0xF) | (((qh >> 2) & 3) << 4)) - 32;
          const int q3 = (int)((b[qlo + l] >> 4) | (((qh >> 4) & 3) << 4)) - 32;
          const int q4 = (int)((b[qlo + l + 32] >> 4) | (((qh >> 6) & 3) << 4)) - 32;
          y[yo + l] = d * (float)(int8_t)b[sco + isc] * (float)q1;
          y[yo + l + 32] = d * (float)(int8_t)b[sco + isc + 2] * (float)q2;
          y[yo + l + 64] = d * (float)(int8_t)b[sco + isc + 4] * (float)q3;
          y[yo + l + 96] = d * (float)(int8_t)b[sco + isc + 6] * (float)q4;
        }
        yo += 128;
        qlo += 64;
        qho += 32;
        sco += 8;
      }
      break;
    }
    case NLO_Q8_K: { /* :321-324 */
      float d;
      memcpy(&d, b, 4);
      for (int j = 0; j < 256; ++j) y[j] = (float)(int8_t)b[4 + j] * d;
      break;
    }
    case NLO_F32: memcpy(y, b, 4); break;           /* :325-326 */
    case NLO_F16: y[0] = rd_half(b, 0); break;      /* :327-328 */
    case NLO_BF16: y[0] = bf16_to_float(rd16(b, 0)); break; /* :329-330 */
    default: break;
  }
}

/* dequantRow (quant.nim:336-352) */
int32_t nlo_dequant_row(int32_t t, const void* src, float* dst, int64_t n) {
  const int32_t bs = nlo_block_size(t), ts = nlo_type_size(t);
  if (bs == 0) return -1;
  bytes s = (bytes)src;
  if (t == NLO_F32) {
    memcpy(dst, src, (size_t)n * 4);
  } else if (t == NLO_F16) {
    for (int64_t i = 0; i < n; ++i) dst[i] = nlo_half_to_float(rd16(s + 2 * i, 0));
  } else if (t == NLO_BF16) {
    for (int64_t i = 0; i < n; ++i) dst[i] = bf16_to_float(rd16(s + 2 * i, 0));
  } else {
    const int64_t nb = n / bs;
    for (int64_t i = 0; i < nb; ++i) dequant_block(t, s + i * ts, dst + i * bs);
  }
  return 0;
}

/* dotF32 (quant.nim:362-374) */
float nlo_dot_f32(const float* x, const float* y, int64_t n) {
  float s0 = 0, s1 = 0, s2 = 0, s3 = 0, s4 = 0, s5 = 0, s6 = 0, s7 = 0;
  int64_t i = 0;
  while (i + 8 <= n) {
    s0 += x[i] * y[i];
    s1 += x[i + 1] * y[i + 1];
    s2 += x[i + 2] * y[i + 2];
    s3 += x[i + 3] * y[i + 3];
    s4 += x[i + 4] * y[i + 4];
    s5 += x[i + 5] * y[i + 5];
    s6 += x[i + 6] * y[i + 6];
    s7 += x[i + 7] * y[i + 7];
    i += 8;
  }
  while (i < n) {
    s0 += x[i] * y[i];
    ++i;
  }
  return (s0 + s1) + (s2 + s3) + (s4 + s5) + (s6 + s7);
}

/* actBlockLen (quant.nim:639-644) */
int32_t nlo_act_block_len(int32_t t) {
  switch (t) {
    case NLO_Q4_K: case NLO_Q5_K: case NLO_Q6_K: return 256;
    case NLO_Q8_0: case NLO_Q4_0: return 32;
    default: return 0;
  }
}

/* Nim's float32 max for the non-NaN values the restatement is checked on:
 * the larger of the two (a NaN activation is outside what is pinned). */
static float nim_max(float x, float y) { return y <= x ? x : y; }

/* quantizeAct (quant.nim:646-667) */
void nlo_quantize_act(const float* x, int64_t n, int32_t bl, float* d_out, int8_t* qs,
                      int32_t* bsums) {
  const int64_t nb = n / bl;
  for (int64_t b = 0; b < nb; ++b) {
    float amax = 0.0f;
    for (int i = 0; i < bl; ++i) amax = nim_max(amax, fabsf(x[b * bl + i]));
    const float d = amax / 127.0f;
    const float id = d > 0 ? 1.0f / d : 0.0f;
    d_out[b] = d;
    for (int i = 0; i < bl; ++i) {
      const float v = x[b * bl + i] * id;
      const float r = v >= 0 ? v + 0.5f : -v + 0.5f;
      const int64_t t = (int64_t)r;
      qs[b * bl + i] = (int8_t)(v >= 0 ? t : -t);
    }
    if (bl == 256) {
      for (int g = 0; g < 16; ++g) {
        int32_t s = 0;
        for (int i = 0; i < 16; ++i) s += qs[b * 256 + g * 16 + i];
        bsums[b * 16 + g] = s;
      }
    }
  }
}

/* dotQ4K (quant.nim:669-695) */
static float dot_q4k(bytes w, const float* ad, const int8_t* aqs, const int32_t* abs_,
                     int64_t off, int64_t n) {
  const int64_t nb = n / 256;
  float acc = 0.0f;
  for (int64_t ib = 0; ib < nb; ++ib) {
    bytes b = w + ib * 144;
    const int64_t ab = off / 256 + ib;
    const int8_t* q8 = aqs + ab * 256;
    const float d = rd_half(b, 0);
    const float dmin = rd_half(b, 2);
    int32_t sumi = 0, summ = 0;
    for (int j = 0; j < 4; ++j) {
      uint8_t sc0, m0, sc1, m1;
      scale_min_k4(2 * j, b, 4, &sc0, &m0);
      scale_min_k4(2 * j + 1, b, 4, &sc1, &m1);
      int32_t s0 = 0, s1 = 0;
      const int qo = 16 + 32 * j;
      for (int l = 0; l < 32; ++l) {
        const uint8_t q = b[qo + l];
        s0 += (int32_t)(q & 0xF) * q8[64 * j + l];
        s1 += (int32_t)(q >> 4) * q8[64 * j + 32 + l];
      }
      sumi += (int32_t)sc0 * s0 + (int32_t)sc1 * s1;
      const int32_t* bs = abs_ + ab * 16 + 4 * j;
      summ += (int32_t)m0 * (bs[0] + bs[1]) + (int32_t)m1 * (bs[2] + bs[3]);
    }
    acc += ad[ab] * (d * (float)sumi - dmin * (float)summ);
  }
  return acc;
}

/* dotQ5K (quant.nim:697-729) */
static float dot_q5k(bytes w, const float* ad, const int8_t* aqs, const int32_t* abs_,
                     int64_t off, int64_t n) {
  const int64_t nb = n / 256;
  float acc = 0.0f;
  for (int64_t ib = 0; ib < nb; ++ib) {
    bytes b = w + ib * 176;
    const int64_t ab = off / 256 + ib;
    const int8_t* q8 = aqs + ab * 256;
    const float d = rd_half(b, 0);
    const float dmin = rd_half(b, 2);
    int32_t sumi = 0, summ = 0;
    uint8_t u1 = 1, u2 = 2;
    for (int j = 0; j < 4; ++j) {
      uint8_t sc0, m0, sc1, m1;
      scale_min_k4(2 * j, b, 4, &sc0, &m0);
      scale_min_k4(2 * j + 1, b, 4, &sc1, &m1);
      int32_t s0 = 0, s1 = 0;
      const int qo = 48 + 32 * j;
      for (int l = 0; l < 32; ++l) {
        const uint8_t q = b[qo + l];
        const uint8_t h = b[16 + l];
        const int32_t v0 = (int32_t)(q & 0xF) + ((h & u1) != 0 ? 16 : 0);
        const int32_t v1 = (int32_t)(q >> 4) + ((h & u2) != 0 ? 16 : 0);
        s0 += v0 * q8[64 * j + l];
        s1 += v1 * q8[64 * j + 32 + l];
      }
      sumi += (int32_t)sc0 * s0 + (int32_t)sc1 * s1;
      const int32_t* bs = abs_ + ab * 16 + 4 * j;
      summ += (int32_t)m0 * (bs[0] + bs[1]) + (int32_t)m1 * (bs[2] + bs[3]);
      u1 = (uint8_t)(u1 << 2);
      u2 = (uint8_t)(u2 << 2);
    }
    acc += ad[ab] * (d * (float)sumi - dmin * (float)summ);
  }
  return acc;
}

/* dotQ6K (quant.nim:731-760) */
static float dot_q6k(bytes w, const float* ad, const int8_t* aqs, int64_t off, int64_t n) {
  const int64_t nb = n / 256;
  float acc = 0.0f;
  for (int64_t ib = 0; ib < nb; ++ib) {
    bytes b = w + ib * 210;
    const int64_t ab = off / 256 + ib;
    const int8_t* q8 = aqs + ab * 256;
    const float d = rd_half(b, 208);
    const int8_t* sc = (const int8_t*)(b + 192);
    int32_t sumi = 0;
    for (int h = 0; h < 2; ++h) {
      const int ql = 64 * h, qh = 128 + 32 * h;
      for (int half = 0; half < 2; ++half) {
        int32_t s0 = 0, s1 = 0, s2 = 0, s3 = 0;
        for (int l = 16 * half; l < 16 * half + 16; ++l) {
          const uint8_t hb = b[qh + l];
          const int32_t q1 = (int32_t)((b[ql + l] & 0xF) | ((hb & 3) << 4)) - 32;
          const int32_t q2 = (int32_t)((b[ql + l + 32] & 0xF) | (((hb >> 2) & 3) << 4)) - 32;
          const int32_t q3 = (int32_t)((b[ql + l] >> 4) | (((hb >> 4) & 3) << 4)) - 32;
          const int32_t q4 = (int32_t)((b[ql + l + 32] >> 4) | (((hb >> 6) & 3) << 4)) - 32;
          const int base = 128 * h + l;
          s0 += q1 * q8[base];
          s1 += q2 * q8[base + 32];
          s2 += q3 * q8[base + 64];
          s3 += q4 * q8[base + 96];
        }
        const int so = 8 * h + half;
        sumi += (int32_t)sc[so] * s0 + (int32_t)sc[so + 2] * s1 + (int32_t)sc[so + 4] * s2 +
                (int32_t)sc[so + 6] * s3;
      }
    }
    acc += ad[ab] * d * (float)sumi;
  }
  return acc;
}

/* dotQ8_0i (quant.nim:762-772) */
static float dot_q8_0i(bytes w, const float* ad, const int8_t* aqs, int64_t off, int64_t n) {
  const int64_t nb = n / 32;
  float acc = 0.0f;
  for (int64_t ib = 0; ib < nb; ++ib) {
    const int64_t o = ib * 34;
    const int64_t ab = off / 32 + ib;
    const int8_t* q8 = aqs + ab * 32;
    int32_t s = 0;
    for (int l = 0; l < 32; ++l) s += (int32_t)(int8_t)w[o + 2 + l] * q8[l];
    acc += rd_half(w + o, 0) * ad[ab] * (float)s;
  }
  return acc;
}

/* dotQ4_0i (quant.nim:774-786) */
static float dot_q4_0i(bytes w, const float* ad, const int8_t* aqs, int64_t off, int64_t n) {
  const int64_t nb = n / 32;
  float acc = 0.0f;
  for (int64_t ib = 0; ib < nb; ++ib) {
    const int64_t o = ib * 18;
    const int64_t ab = off / 32 + ib;
    const int8_t* q8 = aqs + ab * 32;
    int32_t s = 0;
    for (int l = 0; l < 16; ++l) {
      const uint8_t q = w[o + 2 + l];
      s += ((int32_t)(q & 0xF) - 8) * q8[l] + ((int32_t)(q >> 4) - 8) * q8[l + 16];
    }
    acc += rd_half(w + o, 0) * ad[ab] * (float)s;
  }
  return acc;
}

/* dotRowAct (quant.nim:788-798) */
float nlo_dot_row_act(int32_t t, const void* row, const float* ad, const int8_t* aqs,
                      const int32_t* abs_, int64_t off, int64_t n) {
  bytes w = (bytes)row;
  switch (t) {
    case NLO_Q4_K: return dot_q4k(w, ad, aqs, abs_, off, n);
    case NLO_Q5_K: return dot_q5k(w, ad, aqs, abs_, off, n);
    case NLO_Q6_K: return dot_q6k(w, ad, aqs, off, n);
    case NLO_Q8_0: return dot_q8_0i(w, ad, aqs, off, n);
    case NLO_Q4_0: return dot_q4_0i(w, ad, aqs, off, n);
    default: return 0.0f;
  }
}

/* model.nim:184-185 */
int32_t nlo_matmul_uses_act(int32_t t, int64_t cols, int32_t nb, int32_t exact) {
  const int32_t bl = nlo_act_block_len(t);
  return !exact && bl > 0 && cols % bl == 0 && (nb <= 4 || t != NLO_Q8_0);
}

/* matmul (model.nim:179-200) with matmulTask (:144-170) over rows first..last-1 */
int32_t nlo_matmul(int32_t t, const void* w, int64_t rows, int64_t cols, const float* x,
                   int32_t nb, float* y, int32_t exact, const float* lora_a,
                   const float* lora_b, int32_t rank, float scale, int64_t first, int64_t last) {
  const int64_t rb = nlo_row_bytes(t, cols);
  if (rb < 0) return -1;
  bytes data = (bytes)w;
  if (nlo_matmul_uses_act(t, cols, nb, exact)) {
    const int32_t bl = nlo_act_block_len(t);
    const int64_t n = (int64_t)nb * cols;
    float* ad = (float*)malloc(sizeof(float) * (size_t)(n / bl));
    int8_t* aqs = (int8_t*)malloc((size_t)n);
    int32_t* abs_ = (int32_t*)malloc(sizeof(int32_t) * (size_t)(n / 16 + 1));
    nlo_quantize_act(x, n, bl, ad, aqs, abs_);
    for (int64_t r = first; r < last; ++r)
      for (int32_t b = 0; b < nb; ++b)
        y[b * rows + r] = nlo_dot_row_act(t, data + r * rb, ad, aqs, abs_, b * cols, cols);
    free(ad);
    free(aqs);
    free(abs_);
  } else if (nb == 1 && t == NLO_F32) {
    for (int64_t r = first; r < last; ++r)
      y[r] = nlo_dot_f32((const float*)(data + r * rb), x, cols);
  } else {
    float* tmp = (float*)malloc(sizeof(float) * (size_t)cols);
    for (int64_t r = first; r < last; ++r) {
      nlo_dequant_row(t, data + r * rb, tmp, cols);
      for (int32_t b = 0; b < nb; ++b) y[b * rows + r] = nlo_dot_f32(tmp, x + b * cols, cols);
    }
    free(tmp);
  }
  if (rank > 0 && lora_a != NULL && lora_b != NULL) {
    float* tmp = (float*)malloc(sizeof(float) * (size_t)rank);
    for (int32_t b = 0; b < nb; ++b) {
      for (int32_t i = 0; i < rank; ++i) tmp[i] = nlo_dot_f32(lora_a + (int64_t)i * cols, x + b * cols, cols);
      for (int64_t r = first; r < last; ++r) {
        float s = 0.0f;
        for (int32_t i = 0; i < rank; ++i) s += lora_b[r * rank + i] * tmp[i];
        y[b * rows + r] += scale * s;
      }
    }
    free(tmp);
  }
  return 0;
}
