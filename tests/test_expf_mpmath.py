"""The correctly rounded exp of a binary32 input, checked against mpmath.

The reference evaluates exp(float32) with the C library's expf
(src/nimllm/sampler.nim:56); this sampler uses the correctly rounded value
instead (nim.llm_amd/csrc/nls_expf.h, the same header on host and device), and
the oracle's exact mode computes it as (float)expl(x) (oracle/nls_oracle.c).
Each value below is rounded by hand from a 256-bit mpmath evaluation, so
neither the header, its hard-case table nor the oracle is used as its own
check:

* every entry of the hard-case table (inputs and stored results);
* the 64 float64 powers 2^(j/64) of the table form;
* about 300,000 binary32 inputs (random bit patterns, uniform reals over the
  whole domain and the softmax range, and the ends of the range) through the
  host build of expf_cr and expf_cr_t and through the oracle's nlo_expf_cr;
* the relative error of both float64 evaluations against the bound that the
  header's rounding test assumes.
"""
import ctypes
import math
import os
import subprocess

import numpy as np
import pytest

mpmath = pytest.importorskip("mpmath")
from mpmath import mp, mpf  # noqa: E402

import oracle as O  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
FLAGS = ["-O2", "-ffp-contract=off", "-fno-fast-math", "-std=c++17", "-Wall"]
if os.environ.get("NLS_SANITIZE") == "1":  # the sanitizer run (tests/test_runs_cpu.py)
    FLAGS = FLAGS + ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-g"]
PREC = 256


def _round_binary(y, mant_bits: int, emin: int) -> float:
    """The positive mpf y rounded to nearest, ties to even, to a binary format
    with mant_bits significand bits and smallest ulp 2^emin (no overflow
    handling).  Returned as a float64, which holds it exactly."""
    sign, man, exp, bc = y._mpf_
    assert sign == 0 and man > 0
    top = exp + bc - 1
    e = max(top - (mant_bits - 1), emin)
    shift = e - exp
    if shift <= 0:
        q = man << -shift
    else:
        q = man >> shift
        rem = man & ((1 << shift) - 1)
        half = 1 << (shift - 1)
        # an exact midpoint would mean PREC bits are not enough to decide
        assert rem != half, "midpoint at %d bits" % PREC
        if rem > half:
            q += 1
    return math.ldexp(q, e)


def _cr_expf(x: np.float32) -> np.float32:
    """Correctly rounded binary32 e^x from a PREC-bit evaluation."""
    xf = float(x)
    if math.isnan(xf):
        return np.float32(np.nan)
    if xf == 0.0:
        return np.float32(1.0)
    with mp.workprec(PREC):
        y = mp.exp(mpf(xf))
    if y < mpf(2) ** -150:  # below half the smallest subnormal
        return np.float32(0.0)
    v = _round_binary(y, 24, -149)
    if v >= 2.0 ** 128:
        return np.float32(np.inf)
    return np.float32(v)


def _rel_err(x: np.float32, got: float) -> float:
    with mp.workprec(PREC):
        y = mp.exp(mpf(float(x)))
        return float(abs(mpf(got) - y) / y)


@pytest.fixture(scope="module")
def lib(tmp_path_factory):
    d = tmp_path_factory.mktemp("expf")
    so = str(d / "expf_cr_check.so")
    subprocess.run(["g++", *FLAGS, "-shared", "-fPIC", "-o", so,
                    os.path.join(HERE, "expf_cr_check.cpp")], check=True)
    L = ctypes.CDLL(so)
    P = ctypes.POINTER
    L.expf_batch.argtypes = [P(ctypes.c_float), ctypes.c_int64, P(ctypes.c_float),
                             P(ctypes.c_float), P(ctypes.c_double), P(ctypes.c_double)]
    L.expf_batch.restype = None
    L.pow2_table.argtypes = [P(ctypes.c_double)]
    L.pow2_table.restype = ctypes.c_int64
    L.hard_table.argtypes = [P(ctypes.c_uint32), P(ctypes.c_uint32)]
    L.hard_table.restype = ctypes.c_int64
    L.rel_err_bound.restype = ctypes.c_double
    return L


def _batch(L, x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = len(x)
    cr = np.empty(n, np.float32)
    t = np.empty(n, np.float32)
    rd = np.empty(n, np.float64)
    rt = np.empty(n, np.float64)
    P = ctypes.POINTER
    L.expf_batch(x.ctypes.data_as(P(ctypes.c_float)), n, cr.ctypes.data_as(P(ctypes.c_float)),
                 t.ctypes.data_as(P(ctypes.c_float)), rd.ctypes.data_as(P(ctypes.c_double)),
                 rt.ctypes.data_as(P(ctypes.c_double)))
    return cr, t, rd, rt


def _bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


def test_pow2_table_is_correctly_rounded(lib):
    t = np.zeros(64, np.float64)
    n = lib.pow2_table(t.ctypes.data_as(ctypes.POINTER(ctypes.c_double)))
    assert n == 64
    for j in range(64):
        with mp.workprec(PREC):
            want = _round_binary(mp.power(2, mpf(j) / 64), 53, -1074)
        assert t[j] == want, (j, float.hex(float(t[j])), float.hex(want))


def test_hard_table_is_correctly_rounded(lib):
    n = lib.hard_table(None, None)
    assert n > 0
    ins = np.zeros(n, np.uint32)
    outs = np.zeros(n, np.uint32)
    P = ctypes.POINTER
    lib.hard_table(ins.ctypes.data_as(P(ctypes.c_uint32)), outs.ctypes.data_as(P(ctypes.c_uint32)))
    assert np.all(np.diff(ins.astype(np.int64)) > 0), "the binary search needs sorted inputs"
    xs = ins.view(np.float32)
    want = np.array([_cr_expf(x) for x in xs], np.float32)
    assert np.array_equal(outs, _bits(want)), [
        (hex(int(i)), hex(int(o)), hex(int(w))) for i, o, w in zip(ins, outs, _bits(want)) if o != w]
    # each table input is one the float64 evaluations cannot decide, and both
    # public functions return the table's value for it
    cr, t, rd, rt = _batch(lib, xs)
    assert np.array_equal(_bits(cr), outs) and np.array_equal(_bits(t), outs)
    undecided = [not (lib.expf_decided(ctypes.c_double(a)) and lib.expf_decided(ctypes.c_double(b)))
                 for a, b in zip(rd, rt)]
    assert all(undecided)


def _inputs(rng):
    lo, hi = np.float32(-104.0), np.float32(89.0)
    # random bit patterns inside the domain (dense near zero, as the format is)
    u = rng.integers(0, 2 ** 32, size=400_000, dtype=np.uint64).astype(np.uint32)
    f = u.view(np.float32)
    f = f[np.isfinite(f) & (f > lo) & (f <= hi)][:110_000]
    uni = rng.uniform(-104.0, 89.0, size=110_000).astype(np.float32)
    soft = rng.uniform(-30.0, 0.0, size=70_000).astype(np.float32)
    edges = []
    for e in (-104.0, -103.97208, -103.27893, -87.33654, -0.0, 0.0, 88.72283, 88.7228394, 89.0,
              2.0 ** -24, -2.0 ** -25, 2.0 ** -149, -2.0 ** -149):
        up = dn = np.float32(e)
        edges.append(up)
        for _ in range(4):  # four neighbours on each side
            up = np.nextafter(up, np.float32(np.inf))
            dn = np.nextafter(dn, np.float32(-np.inf))
            edges += [up, dn]
    x = np.concatenate([f, uni, soft, np.array(edges, np.float32)])
    return x[(x > lo) & (x <= hi)]


def test_random_inputs_against_mpmath(lib):
    rng = np.random.default_rng(20240611)
    x = _inputs(rng)
    assert len(x) > 280_000
    want = np.array([_cr_expf(v) for v in x], np.float32)
    cr, t, rd, rt = _batch(lib, x)
    bad = np.nonzero(_bits(cr) != _bits(want))[0]
    assert len(bad) == 0, [(float.hex(float(x[i])), cr[i], want[i]) for i in bad[:10]]
    bad = np.nonzero(_bits(t) != _bits(want))[0]
    assert len(bad) == 0, [(float.hex(float(x[i])), t[i], want[i]) for i in bad[:10]]
    ol = O.lib()
    orc = np.array([ol.nlo_expf_cr(float(v)) for v in x], np.float32)
    bad = np.nonzero(_bits(orc) != _bits(want))[0]
    assert len(bad) == 0, [(float.hex(float(x[i])), orc[i], want[i]) for i in bad[:10]]


def test_float64_evaluations_within_the_rounding_bound(lib):
    """Both float64 evaluations stay inside NLS_EXPF_REL_ERR (the rounding
    test's interval) with room to spare: the measured maxima over every
    binary32 input are 2^-52.65 (Taylor form) and 2^-51.96 (table form)."""
    rng = np.random.default_rng(7)
    x = np.concatenate([rng.uniform(-104.0, 89.0, 20_000), rng.uniform(-1.0, 1.0, 10_000),
                        rng.uniform(-30.0, 0.0, 10_000)]).astype(np.float32)
    _, _, rd, rt = _batch(lib, x)
    bound = lib.rel_err_bound()
    assert bound == 2.0 ** -47
    wd = max(_rel_err(v, a) for v, a in zip(x, rd) if a > 0)
    wt = max(_rel_err(v, b) for v, b in zip(x, rt) if b > 0)
    assert wd <= 2.0 ** -52.0, math.log2(wd)
    assert wt <= 2.0 ** -51.5, math.log2(wt)
    assert max(wd, wt) * 2 ** 4 < bound


def test_outside_the_domain(lib):
    x = np.array([-np.inf, -1e30, -200.0, -104.0, np.nextafter(np.float32(-104.0), np.float32(-1e9)),
                  89.00001, 100.0, 1e30, np.inf, np.nan], np.float32)
    cr, t, _, _ = _batch(lib, x)
    ol = O.lib()
    orc = np.array([ol.nlo_expf_cr(float(v)) for v in x], np.float32)
    for got in (cr, t, orc):
        assert np.all(got[:5] == 0.0) and not np.any(np.signbit(got[:5]))
        assert np.all(np.isposinf(got[5:9]))
        assert np.isnan(got[9])
