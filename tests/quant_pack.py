"""Writers of the GGML weight blocks, for tests: they pack given integer levels
and scales into the byte layout, the way the quantisers do.

Q8_0, Q4_0, Q4_1, Q5_0, Q5_1, Q4_K, Q5_K and Q6_K follow the packing steps of
the reference's own writer, quantizeBlock (src/nimllm/quant.nim:424-580);
Q2_K, Q3_K and Q8_K, which the reference only reads, follow ggml's published
reference quantisers (quantize_row_q2_K_ref, quantize_row_q3_K_ref,
quantize_row_q8_K_ref in ggml-quants.c).  Each writer also returns the values
the format stands for, computed from the levels and scales in float32 in the
order the dequantiser's formula states, so a round trip through a reader
checks the reader's byte and bit layout against an independent writer.

Every writer takes a numpy Generator and draws its own levels and scales.
"""
from __future__ import annotations

import numpy as np

F32 = np.float32


def f16_bits(v: float) -> int:
    return int(np.array([v], dtype=np.float16).view(np.uint16)[0])


def f16_val(bits: int) -> np.float32:
    return F32(np.array([bits], dtype=np.uint16).view(np.float16)[0])


def rand_half(rng, lo=-12, hi=-2, positive=False) -> int:
    """A finite, normal half with a random mantissa and exponent in [lo, hi]."""
    m = rng.integers(0, 1024)
    e = rng.integers(lo, hi + 1)
    s = 0 if positive or rng.integers(0, 2) == 0 else 0x8000
    return int(s | ((e + 15) << 10) | m)


def _wr16(b, o, v):
    b[o] = v & 0xFF
    b[o + 1] = v >> 8


def pack_q8_0(rng):
    b = np.zeros(34, np.uint8)
    dh = rand_half(rng)
    _wr16(b, 0, dh)
    q = rng.integers(-127, 128, 32).astype(np.int8)
    b[2:34] = q.view(np.uint8)
    d = f16_val(dh)
    return b, (q.astype(F32) * d).astype(F32)


def pack_q4_0(rng):
    b = np.zeros(18, np.uint8)
    dh = rand_half(rng)
    _wr16(b, 0, dh)
    L = rng.integers(0, 16, 32)
    for j in range(16):
        b[2 + j] = L[j] | (L[16 + j] << 4)
    d = f16_val(dh)
    return b, ((L - 8).astype(F32) * d).astype(F32)


def pack_q4_1(rng):
    b = np.zeros(20, np.uint8)
    dh, mh = rand_half(rng), rand_half(rng)
    _wr16(b, 0, dh)
    _wr16(b, 2, mh)
    L = rng.integers(0, 16, 32)
    for j in range(16):
        b[4 + j] = L[j] | (L[16 + j] << 4)
    d, m = f16_val(dh), f16_val(mh)
    return b, (L.astype(F32) * d + m).astype(F32)


def _pack_q5(rng, with_min):
    n = 24 if with_min else 22
    b = np.zeros(n, np.uint8)
    dh = rand_half(rng)
    mh = rand_half(rng)
    _wr16(b, 0, dh)
    o = 2
    if with_min:
        _wr16(b, 2, mh)
        o = 4
    L = rng.integers(0, 32, 32)
    qh = 0
    for j in range(16):
        q0, q1 = int(L[j]), int(L[16 + j])
        b[o + 4 + j] = (q0 & 0xF) | ((q1 & 0xF) << 4)
        qh |= ((q0 & 0x10) >> 4) << j
        qh |= ((q1 & 0x10) >> 4) << (j + 16)
    for k in range(4):
        b[o + k] = (qh >> (8 * k)) & 0xFF
    d, m = f16_val(dh), f16_val(mh)
    if with_min:
        return b, (L.astype(F32) * d + m).astype(F32)
    return b, ((L - 16).astype(F32) * d).astype(F32)


def pack_q5_0(rng):
    return _pack_q5(rng, False)


def pack_q5_1(rng):
    return _pack_q5(rng, True)


def _pack_k_scales(b, ls, lm):
    # quant.nim:529-537
    for j in range(8):
        if j < 4:
            b[4 + j] = ls[j]
            b[4 + j + 4] = lm[j]
        else:
            b[4 + j + 4] = (ls[j] & 0xF) | ((lm[j] & 0xF) << 4)
            b[4 + j - 4] |= (ls[j] >> 4) << 6
            b[4 + j] |= (lm[j] >> 4) << 6


def _pack_q45k(rng, five):
    b = np.zeros(176 if five else 144, np.uint8)
    dh, mh = rand_half(rng, positive=True), rand_half(rng, positive=True)
    _wr16(b, 0, dh)
    _wr16(b, 2, mh)
    ls = rng.integers(0, 64, 8)
    lm = rng.integers(0, 64, 8)
    _pack_k_scales(b, ls, lm)
    L = rng.integers(0, 32 if five else 16, 256)
    if not five:  # quant.nim:549-552
        for j in range(4):
            for l in range(32):
                b[16 + 32 * j + l] = L[64 * j + l] | (L[64 * j + 32 + l] << 4)
    else:  # quant.nim:553-564
        m1, m2 = 1, 2
        for j in range(4):
            for l in range(32):
                l1 = int(L[64 * j + l])
                if l1 > 15:
                    l1 -= 16
                    b[16 + l] |= m1
                l2 = int(L[64 * j + 32 + l])
                if l2 > 15:
                    l2 -= 16
                    b[16 + l] |= m2
                b[48 + 32 * j + l] = l1 | (l2 << 4)
            m1 <<= 2
            m2 <<= 2
    d, mn = f16_val(dh), f16_val(mh)
    y = np.zeros(256, F32)
    for s in range(8):
        d1 = F32(d * F32(ls[s]))
        m1_ = F32(mn * F32(lm[s]))
        y[32 * s:32 * s + 32] = (d1 * L[32 * s:32 * s + 32].astype(F32)).astype(F32) - m1_
    return b, y


def pack_q4_k(rng):
    return _pack_q45k(rng, False)


def pack_q5_k(rng):
    return _pack_q45k(rng, True)


def pack_q6_k(rng):
    b = np.zeros(210, np.uint8)
    dh = rand_half(rng)
    _wr16(b, 208, dh)
    sc = rng.integers(-128, 128, 16).astype(np.int8)
    b[192:208] = sc.view(np.uint8)
    L = rng.integers(0, 64, 256)
    for j in range(2):  # quant.nim:568-577
        for l in range(32):
            q1 = L[128 * j + l] & 0xF
            q2 = L[128 * j + l + 32] & 0xF
            q3 = L[128 * j + l + 64] & 0xF
            q4 = L[128 * j + l + 96] & 0xF
            b[64 * j + l] = q1 | (q3 << 4)
            b[64 * j + l + 32] = q2 | (q4 << 4)
            b[128 + 32 * j + l] = ((L[128 * j + l] >> 4) | ((L[128 * j + l + 32] >> 4) << 2)
                                   | ((L[128 * j + l + 64] >> 4) << 4)
                                   | ((L[128 * j + l + 96] >> 4) << 6))
    d = f16_val(dh)
    y = np.zeros(256, F32)
    for e in range(256):
        y[e] = F32(F32(d * F32(sc[e // 16])) * F32(L[e] - 32))
    return b, y


def pack_q2_k(rng):
    # ggml block_q2_K: scales[16] qs[64] d dmin (quantize_row_q2_K_ref)
    b = np.zeros(84, np.uint8)
    dh, mh = rand_half(rng, positive=True), rand_half(rng, positive=True)
    Lsc = rng.integers(0, 16, 16)
    Lm = rng.integers(0, 16, 16)
    for j in range(16):
        b[j] = Lsc[j] | (Lm[j] << 4)
    L = rng.integers(0, 4, 256)
    for j in (0, 128):
        for l in range(32):
            b[16 + j // 4 + l] = (L[j + l] | (L[j + l + 32] << 2) | (L[j + l + 64] << 4)
                                  | (L[j + l + 96] << 6))
    _wr16(b, 80, dh)
    _wr16(b, 82, mh)
    d, mn = f16_val(dh), f16_val(mh)
    y = np.zeros(256, F32)
    for e in range(256):
        dl = F32(d * F32(Lsc[e // 16]))
        ml = F32(mn * F32(Lm[e // 16]))
        y[e] = F32(F32(dl * F32(L[e])) - ml)
    return b, y


def pack_q3_k(rng):
    # ggml block_q3_K: hmask[32] qs[64] scales[12] d (quantize_row_q3_K_ref)
    b = np.zeros(110, np.uint8)
    dh = rand_half(rng)
    Ls = rng.integers(0, 64, 16)
    sc = np.zeros(12, np.int64)
    for j in range(16):
        l = int(Ls[j])
        if j < 8:
            sc[j] = l & 0xF
        else:
            sc[j - 8] |= (l & 0xF) << 4
        l >>= 4
        sc[j % 4 + 8] |= l << (2 * (j // 4))
    b[96:108] = sc.astype(np.uint8)
    Lf = rng.integers(0, 8, 256)
    L = Lf.copy()
    for j in range(256):
        if L[j] > 3:
            b[j % 32] |= 1 << (j // 32)
            L[j] -= 4
    for j in (0, 128):
        for l in range(32):
            b[32 + j // 4 + l] = (L[j + l] | (L[j + l + 32] << 2) | (L[j + l + 64] << 4)
                                  | (L[j + l + 96] << 6))
    _wr16(b, 108, dh)
    d = f16_val(dh)
    y = np.zeros(256, F32)
    for e in range(256):
        dl = F32(d * F32(int(Ls[e // 16]) - 32))
        y[e] = F32(dl * F32(int(Lf[e]) - 4))
    return b, y


def pack_q8_k(rng):
    # ggml block_q8_K: float d, int8 qs[256], int16 bsums[16]
    b = np.zeros(292, np.uint8)
    d = F32(rng.uniform(0.001, 0.1))
    b[0:4] = np.array([d], F32).view(np.uint8)
    q = rng.integers(-127, 128, 256).astype(np.int8)
    b[4:260] = q.view(np.uint8)
    bs = q.astype(np.int16).reshape(16, 16).sum(axis=1).astype(np.int16)
    b[260:292] = bs.view(np.uint8)
    return b, (q.astype(F32) * d).astype(F32)


def pack_f16(rng):
    h = np.array([rand_half(rng, -8, 3)], np.uint16)
    return h.view(np.uint8), h.view(np.float16).astype(F32)


def pack_bf16(rng):
    v = F32(rng.normal())
    bits = np.array([v], F32).view(np.uint32)[0] >> 16
    h = np.array([bits], np.uint16)
    return h.view(np.uint8), (h.astype(np.uint32) << 16).view(F32)


def pack_f32(rng):
    v = np.array([rng.normal()], F32)
    return v.view(np.uint8), v


PACKERS = {
    0: pack_f32, 1: pack_f16, 2: pack_q4_0, 3: pack_q4_1, 6: pack_q5_0, 7: pack_q5_1,
    8: pack_q8_0, 10: pack_q2_k, 11: pack_q3_k, 12: pack_q4_k, 13: pack_q5_k, 14: pack_q6_k,
    15: pack_q8_k, 30: pack_bf16,
}


def pack_row(t: int, n_blocks: int, rng):
    """n_blocks packed blocks of type t: (raw bytes, the values they stand for)."""
    raws, vals = [], []
    for _ in range(n_blocks):
        b, y = PACKERS[t](rng)
        raws.append(np.asarray(b, np.uint8))
        vals.append(np.asarray(y, F32))
    return np.concatenate(raws), np.concatenate(vals)
