"""Pins of the CPU restatement of nimllm's output projection (oracle/
nls_oracle_quant.c) -- the checker the device LM head is compared with.

What pins what:
* dequantRow (quant.nim:164-352): for every type the reference reads, blocks
  packed by an independent writer (tests/quant_pack.py: the reference's own
  quantizeBlock packing, quant.nim:424-580, and ggml's reference quantisers
  for Q2_K / Q3_K / Q8_K) read back to the values the writer encoded.
* halfToFloat (quant.nim:83-110): all 65536 halves against numpy's float16.
* quantizeAct (quant.nim:646-667): the round-half-away rule, |q| <= 127 with
  the block maximum at +-127, the error bound |q d - x| <= d / 2, bsums as the
  sums of 16, and the float32 reading of `int(v + 0.5)` (an add in double
  would round 0.49999997 down).
* dotRowAct (quant.nim:669-798): against the float64 dot product of the
  dequantised weights (pinned above) with the dequantised activations, to the
  rounding bound of its few fp32 operations per block; plus a Q8_0 case whose
  result is an exact integer.
* dotF32 (quant.nim:362-374): its eight strided chains, tail into chain 0 and
  the left-to-right combine of the four pair sums, from hand-computed sums
  where the order shows, and the float64 error bound on random data.
* matmul (model.nim:179-200): the dispatch rule (:185), the float path as
  dequantRow then dotF32, and the LoRA term on a case with exact integers.
"""
import numpy as np
import pytest

import oracle as o
import quant_pack as qp

F32 = np.float32
TYPES = [0, 1, 2, 3, 6, 7, 8, 10, 11, 12, 13, 14, 15, 30]


def test_type_table():
    want = {0: (1, 4), 1: (1, 2), 30: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22),
            7: (32, 24), 8: (32, 34), 10: (256, 84), 11: (256, 110), 12: (256, 144),
            13: (256, 176), 14: (256, 210), 15: (256, 292)}
    for t, (bs, ts) in want.items():
        assert (o.block_size(t), o.type_size(t)) == (bs, ts)
    assert o.row_bytes(14, 2048) == 1680
    assert o.row_bytes(12, 100) == -1
    assert o.block_size(9) == 0  # Q8_1: not readable by the reference


def test_half_to_float_all_halves():
    h = np.arange(65536, dtype=np.uint16)
    want = h.view(np.float16).astype(F32)
    got = np.array([o.half_to_float(int(v)) for v in h], dtype=F32)
    fin = np.isfinite(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))
    # infinities and NaNs keep sign and payload (mantissa << 13); the float to
    # double step of the ctypes return quiets a signalling NaN, so the quiet
    # bit is left out of the comparison
    for v in h[~fin]:
        bits = (int(v) & 0x8000) << 16 | 0x7F800000 | (int(v) & 0x3FF) << 13
        got = int(np.array([o.half_to_float(int(v))], F32).view(np.uint32)[0])
        assert got | 0x400000 == bits | 0x400000


@pytest.mark.parametrize("t", TYPES)
def test_dequant_round_trip(t):
    rng = np.random.default_rng(100 + t)
    bs = o.block_size(t)
    nblk = 64 if bs == 1 else 6
    raw, want = qp.pack_row(t, nblk, rng)
    got = o.dequant_row(t, raw, nblk * bs)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), t


def test_quantize_act_rules():
    rng = np.random.default_rng(7)
    for bl in (32, 256):
        x = (rng.normal(size=8 * bl) * rng.uniform(0.01, 30)).astype(F32)
        x[3] = 0.0
        d, qs, bs = o.quantize_act(x, bl)
        xb = x.reshape(-1, bl)
        amax = np.abs(xb).max(axis=1)
        assert np.array_equal(d, (amax / F32(127)).astype(F32))
        q = qs.reshape(-1, bl).astype(np.int64)
        assert np.abs(q).max() <= 127
        for b in range(xb.shape[0]):
            i = np.argmax(np.abs(xb[b]))
            assert abs(q[b, i]) == 127 and np.sign(q[b, i]) == np.sign(xb[b, i])
        err = np.abs(q * d[:, None].astype(np.float64) - xb)
        assert (err <= d[:, None] * 0.5 * (1 + 1e-5)).all()
        assert qs[3] == 0
        if bl == 256:
            assert np.array_equal(bs, qs.astype(np.int32).reshape(-1, 16).sum(axis=1))
    # round half away from zero, on exact halves: amax 127 makes d = id = 1
    x = np.zeros(32, F32)
    x[0] = 127
    x[1:9] = [0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 126.5, -0.49]
    d, qs, _ = o.quantize_act(x, 32)
    assert d[0] == 1.0
    assert list(qs[:9]) == [127, 1, -1, 2, -2, 3, -3, 127, 0]
    # int(v + 0.5) adds in float32: 0.49999997 + 0.5 rounds to 1.0
    x[1] = np.nextafter(F32(0.5), F32(0))
    x[2] = -x[1]
    d, qs, _ = o.quantize_act(x, 32)
    assert qs[1] == 1 and qs[2] == -1


@pytest.mark.parametrize("t", [2, 8, 12, 13, 14])
def test_dot_row_act_against_dequantised(t):
    rng = np.random.default_rng(300 + t)
    bs = o.block_size(t)
    bl = o.act_block_len(t)
    n = 2048
    raw, wv = qp.pack_row(t, n // bs, rng)
    for trial in range(4):
        x = (rng.normal(size=n) * 3).astype(F32)
        act = o.quantize_act(x, bl)
        d, qs, _ = act
        a = qs.astype(np.float64) * np.repeat(d.astype(np.float64), bl)
        terms = wv.astype(np.float64) * a
        exact = terms.sum()
        got = float(o.dot_row_act(t, raw, act, 0, n))
        nblk = n // bl
        bound = (nblk + 4) * 2.0 ** -23 * np.abs(terms).sum() * 2 + 1e-30
        assert abs(got - exact) <= bound, (t, trial, got, exact, bound)
    # a second activation row: off selects its blocks
    x2 = (rng.normal(size=2 * n)).astype(F32)
    act2 = o.quantize_act(x2, bl)
    one = o.quantize_act(x2[n:], bl)
    assert o.dot_row_act(t, raw, act2, n, n) == o.dot_row_act(t, raw, one, 0, n)


def test_dot_row_act_exact_q8_0():
    # weights d = 1 (half 0x3c00), activations with amax 127 per block: d = 1,
    # so the result is the integer dot product itself
    rng = np.random.default_rng(5)
    nblk = 8
    raw = np.zeros(34 * nblk, np.uint8)
    w = rng.integers(-127, 128, (nblk, 32)).astype(np.int8)
    for b in range(nblk):
        raw[34 * b] = 0x00
        raw[34 * b + 1] = 0x3C
        raw[34 * b + 2:34 * b + 34] = w[b].view(np.uint8)
    x = rng.integers(-126, 127, (nblk, 32)).astype(F32)
    x[:, 0] = 127
    act = o.quantize_act(x.ravel(), 32)
    assert (act[0] == 1).all()
    want = int((w.astype(np.int64) * x.astype(np.int64)).sum())
    assert o.dot_row_act(8, raw, act, 0, 32 * nblk) == F32(want)


def test_dot_f32_order():
    # n < 8: one chain, in order: (2^24 + 1) + 1 stays 2^24 twice over
    a = np.array([2 ** 24, 1, 1], F32)
    assert o.dot_f32(a, np.ones(3, F32)) == F32(2 ** 24)
    # n = 16: chain 0 gets x0 and x8, chain 1 gets x1 and x9 ...
    a = np.zeros(16, F32)
    a[0], a[8] = 2 ** 24, 1        # s0 = 2^24 (the 1 is lost)
    a[1], a[9] = 1, 2 ** 24        # s1 = 2^24 + 1 -> 2^24 (tie to even)
    a[2], a[10] = 3, 2 ** 24       # s2 = 2^24 + 3 -> 2^24 + 4
    a[3], a[11] = -2 ** 24, -2 ** 24  # s3 = -2^25
    a[4] = 5                       # s4 = 5 ... ((s0+s1)+(s2+s3)) + ((s4+s5)+(s6+s7))
    got = o.dot_f32(a, np.ones(16, F32))
    s01 = F32(2 ** 25)
    s23 = F32(F32(2 ** 24 + 4) + F32(-2 ** 25))
    assert got == F32(F32(s01 + s23) + F32(5))
    # the combine adds the four pair sums left to right, ((p01 + p23) + p45)
    # + p67: p01 = 2^24 absorbs each 1 in turn, where a tree would give
    # 2^24 + (1 + 1)
    a = np.zeros(8, F32)
    a[0], a[2], a[4], a[6] = 2 ** 24, 1, 1, 1
    assert o.dot_f32(a, np.ones(8, F32)) == F32(2 ** 24)
    # a tail of n % 8 terms goes to chain 0 after the strided part: s0 =
    # 2^24 absorbs both tail ones, s1 = 1, and 2^24 + 1 ties to 2^24 (tails
    # dealt to chains 0 and 1 would give 2^24 + 2)
    a = np.zeros(10, F32)
    a[0], a[1], a[8], a[9] = 2 ** 24, 1, 1, 1
    assert o.dot_f32(a, np.ones(10, F32)) == F32(2 ** 24)
    # random data: within the float64 bound of a sum of n/8 + 3 roundings
    rng = np.random.default_rng(9)
    for n in (1, 7, 8, 100, 2048, 4099):
        x = rng.normal(size=n).astype(F32)
        y = rng.normal(size=n).astype(F32)
        got = float(o.dot_f32(x, y))
        p = x.astype(np.float64) * y.astype(np.float64)
        assert abs(got - p.sum()) <= (n / 8 + 4) * 2.0 ** -23 * np.abs(p).sum() + 1e-30


def _rand_weights(t, rows, cols, rng):
    bs = o.block_size(t)
    raws, vals = [], []
    for _ in range(rows):
        r, v = qp.pack_row(t, cols // bs, rng)
        raws.append(r)
        vals.append(v)
    return np.stack(raws), np.stack(vals)


def test_matmul_dispatch_and_paths():
    rng = np.random.default_rng(11)
    cols, rows = 256, 6
    assert o.matmul_uses_act(8, cols, 4) and not o.matmul_uses_act(8, cols, 5)
    assert o.matmul_uses_act(14, cols, 64) and not o.matmul_uses_act(14, cols, 1, exact=True)
    assert not o.matmul_uses_act(3, cols, 1) and not o.matmul_uses_act(0, cols, 1)
    for t in (8, 14, 3, 0, 1):
        w, wv = _rand_weights(t, rows, cols, rng)
        for nb in (1, 4, 5):
            x = rng.normal(size=(nb, cols)).astype(F32)
            for exact in (False, True):
                y = o.matmul(t, w, rows, cols, x, exact=exact)
                if o.matmul_uses_act(t, cols, nb, exact):
                    act = o.quantize_act(x.ravel(), o.act_block_len(t))
                    want = np.array([[o.dot_row_act(t, w[r], act, b * cols, cols)
                                      for r in range(rows)] for b in range(nb)], F32)
                else:
                    want = np.array([[o.dot_f32(wv[r], x[b]) for r in range(rows)]
                                     for b in range(nb)], F32)
                assert np.array_equal(y.view(np.uint32), want.view(np.uint32)), (t, nb, exact)
    # rows first..last only
    w, _ = _rand_weights(14, rows, cols, rng)
    x = rng.normal(size=(1, cols)).astype(F32)
    full = o.matmul(14, w, rows, cols, x)
    part = o.matmul(14, w, rows, cols, x, first=2, last=4)
    assert np.array_equal(part[:, 2:4], full[:, 2:4]) and (part[:, :2] == 0).all()


def test_matmul_lora_exact_integers():
    # F32 weights and LoRA factors of small integers: every product and sum is
    # exact, so y = W x + scale * B (A x) holds to the bit
    rng = np.random.default_rng(12)
    rows, cols, rank, nb = 5, 64, 3, 2
    W = rng.integers(-4, 5, (rows, cols)).astype(F32)
    A = rng.integers(-3, 4, (rank, cols)).astype(F32)
    B = rng.integers(-3, 4, (rows, rank)).astype(F32)
    x = rng.integers(-5, 6, (nb, cols)).astype(F32)
    y = o.matmul(0, W.view(np.uint8), rows, cols, x, lora=(A, B, 0.5))
    want = x @ W.T + 0.5 * ((x @ A.T) @ B.T)
    assert np.array_equal(y, want.astype(F32))
