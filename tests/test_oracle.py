"""Pins the CPU oracle (oracle/nls_oracle.c) against independent checks.

The reference (src/nimllm/sampler.nim) ships no sampler tests or golden
vectors, and no Nim toolchain exists here, so each restated function is pinned
by something that does not retype its formula: the GF(2) algebra of the RNG,
library routines (heapq, stable sorted, numpy.argmax, libm expf through an
independent Python restatement), closed forms and invariants.
"""
import math
import random

import numpy as np
import pytest

import oracle as O
import pyref_sampler as R

M64 = (1 << 64) - 1


# --------------------------------------------------------------------------
# Nim std/random
# --------------------------------------------------------------------------

def _gf2_matrix_of_next():
    """Columns of the 128x128 GF(2) matrix of one `next` state update."""
    cols = []
    L = O.lib()
    for bit in range(128):
        st = O.Rand(1 << bit if bit < 64 else 0, (1 << (bit - 64)) if bit >= 64 else 0)
        L.nlo_next(st)
        cols.append(st.a0 | (st.a1 << 64))
    return cols


def _mat_vec(cols, v):
    out = 0
    b = 0
    while v:
        if v & 1:
            out ^= cols[b]
        v >>= 1
        b += 1
    return out


def _mat_mul(a, b):
    # (a*b) column j = a * (b column j)
    return [_mat_vec(a, c) for c in b]


def test_rng_jump_is_2_pow_64_steps():
    """skipRandomNumbers must equal 2^64 applications of `next` (GF(2) power).

    A wrong rotation/shift constant in `next` or a wrong jump polynomial word
    makes the two sides differ."""
    M = _gf2_matrix_of_next()
    P = M
    for _ in range(64):
        P = _mat_mul(P, P)
    L = O.lib()
    rng = random.Random(7)
    for _ in range(4):
        a0, a1 = rng.getrandbits(64), rng.getrandbits(64)
        st = O.Rand(a0, a1)
        L.nlo_skip_random_numbers(st)
        want = _mat_vec(P, a0 | (a1 << 64))
        assert st.a0 == want & M64 and st.a1 == want >> 64


def test_rng_next_matches_python_restatement():
    L = O.lib()
    rng = random.Random(3)
    for _ in range(8):
        a0, a1 = rng.getrandbits(64), rng.getrandbits(64)
        st = O.Rand(a0, a1)
        py = [a0, a1]
        for _ in range(50):
            assert L.nlo_next(st) == R.nim_rand_next(py)
        assert (st.a0, st.a1) == tuple(py)


def test_rand_float_closed_form():
    """rand(1.0) == (x >> 12) / 2^52 exactly, for the raw `next` output x."""
    L = O.lib()
    st = O.Rand(0x0123456789ABCDEF, 0xFEDCBA9876543210)
    st2 = O.Rand(st.a0, st.a1)
    for _ in range(1000):
        x = L.nlo_next(st2)
        f = L.nlo_rand_float(st, 1.0)
        assert f == R.float_from_next(x)
        assert 0.0 <= f < 1.0


def test_init_rand_seed_zero_is_int32_high():
    """initRand(0) is documented to fall back to int32.high (seed 0 is a fixed
    point of the generator).  Parity of the seed split itself is unpinned."""
    assert np.array_equal(O.uniforms(0, 16), O.uniforms(2147483647, 16))
    u = O.uniforms(1234, 10000)
    assert u.min() >= 0 and u.max() < 1
    assert abs(u.mean() - 0.5) < 0.02


# --------------------------------------------------------------------------
# Sampler: oracle vs independent restatement
# --------------------------------------------------------------------------

def _rand_case(rng, V, grid=None):
    x = rng.standard_normal(V).astype(np.float32) * np.float32(rng.uniform(0.5, 3))
    if grid:
        x = (np.round(x * grid) / grid).astype(np.float32)
    return x


def _rand_params(rng, V):
    mode = rng.integers(0, 5)
    p = dict(temperature=float(rng.choice([0.0, 0.5, 0.7, 1.0, 1.3])),
             topK=int(rng.choice([0, 1, 2, 5, 20, V - 1, V, V + 3])),
             topP=float(rng.choice([0.0, 0.5, 0.9, 0.95, 1.0])),
             minP=float(rng.choice([0.0, 0.05, 0.1, 0.3])),
             repeatPenalty=float(rng.choice([1.0, 1.1, 0.9, 1.3])),
             repeatLastN=int(rng.choice([0, 4, 16, 64])),
             presencePenalty=float(rng.choice([0.0, 0.3, -0.2])),
             frequencyPenalty=float(rng.choice([0.0, 0.5, 0.25])),
             seed=0)
    if mode == 0:
        p["temperature"] = 0.0
    return p


@pytest.mark.parametrize("seed", range(6))
def test_oracle_matches_python_restatement(seed):
    rng = np.random.default_rng(seed)
    for case in range(40):
        V = int(rng.integers(1, 120))
        grid = [None, 4, 1][case % 3]
        x = _rand_case(rng, V, grid)
        pd = _rand_params(rng, V)
        hist = [int(t) for t in rng.integers(-3, V + 3, size=int(rng.integers(0, 40)))]
        bias = {}
        for t in rng.choice(V + 4, size=min(V, int(rng.integers(0, 6))), replace=False):
            bias[int(t) - 2] = float(rng.choice([-np.inf, -1.5, 0.0, 2.25, 7.0]))
        u = float(rng.choice([0.0, rng.random(), 0.999999, 0.5]))
        for cr in (False, True):
            pr = R.sample(R.Params(logitBias=bias, **pd), x, hist, u, cr=cr)
            res, cand, probs, fl = O.sample(O.make_params(**pd), x, hist, bias, u,
                                            O.EXPF_CR if cr else O.EXPF_LIBM)
            assert res.id == pr.id, (seed, case, pd)
            assert np.array_equal(fl.view(np.uint32), pr.final_logits.view(np.uint32))
            if not pr.greedy:
                assert list(cand) == list(pr.cand)
                assert np.array_equal(probs.view(np.uint32),
                                      np.array(pr.probs, dtype=np.float32).view(np.uint32))
                assert res.n == pr.n


def test_heap_path_matches_closed_form_rule():
    """Heap membership/order (sampler.nim:85-95) == the closed-form tie rule,
    on tie-heavy rows."""
    rng = np.random.default_rng(11)
    for _ in range(300):
        V = int(rng.integers(2, 80))
        x = rng.integers(-3, 4, size=V).astype(np.float32) * np.float32(0.5)
        if rng.random() < 0.2:
            x[rng.integers(0, V)] = -0.0
        k = int(rng.integers(1, V))
        res, cand, _, _ = O.sample(O.make_params(temperature=1.0, topK=k, repeatPenalty=1.0),
                                   x, u=0.3)
        assert res.heap == 1
        assert list(cand) == R.heap_rule(x, k)


def test_documented_tie_example():
    # values [1, 2, 2, 2, 0.5], k = 2 -> order [2, 1]; index 3 is excluded
    x = np.array([1, 2, 2, 2, 0.5], dtype=np.float32)
    res, cand, _, _ = O.sample(O.make_params(temperature=1.0, topK=2, repeatPenalty=1.0), x)
    assert list(cand) == [2, 1]


def test_sort_path_is_stable_descending():
    rng = np.random.default_rng(5)
    for _ in range(50):
        V = int(rng.integers(2, 200))
        x = (rng.integers(-4, 5, size=V) * 0.25).astype(np.float32)
        x[x == 0] = np.where(rng.random((x == 0).sum()) < 0.5, -0.0, 0.0)
        res, cand, _, _ = O.sample(O.make_params(temperature=1.0, topK=0, repeatPenalty=1.0), x)
        assert res.heap == 0
        want = sorted(range(V), key=lambda i: -float(x[i]))
        assert list(cand) == want


def test_greedy_is_numpy_argmax_first_max():
    rng = np.random.default_rng(2)
    for _ in range(100):
        V = int(rng.integers(1, 300))
        x = rng.integers(-2, 3, size=V).astype(np.float32)
        res, _, _, fl = O.sample(O.make_params(temperature=0.0, repeatPenalty=1.0), x)
        assert res.greedy == 1 and res.id == int(np.argmax(x))
        assert O.lib().nlo_argmax(x.ctypes.data_as(O.ctypes.POINTER(O.ctypes.c_float)), V) == int(np.argmax(x))


def test_invariants():
    rng = np.random.default_rng(9)
    for _ in range(200):
        V = int(rng.integers(2, 300))
        x = rng.standard_normal(V).astype(np.float32) * 2
        k = int(rng.integers(0, V + 2))
        topP = float(rng.choice([1.0, 0.9, 0.5]))
        minP = float(rng.choice([0.0, 0.1]))
        p = O.make_params(temperature=0.8, topK=k, topP=topP, minP=minP, repeatPenalty=1.0)
        # u = 0 -> the first candidate (r = 0 <= 0 after the first step)
        res0, cand, probs, fl = O.sample(p, x, u=0.0)
        assert res0.id == cand[0] and res0.pos == 0
        assert 1 <= res0.n <= res0.ncand
        # the post-filter distribution sums to one (up to fp32 rounding)
        post = probs[:res0.n].astype(np.float64) / float(res0.total)
        assert abs(post.sum() - 1) < 1e-5
        # the candidates are the top of fl, in non-increasing order
        assert np.all(np.diff(fl[cand].astype(np.float64)) <= 0)
        # u -> 1 picks a candidate inside the kept prefix
        res1, _, _, _ = O.sample(p, x, u=0.9999999)
        assert res1.pos <= res1.n - 1
    # k = 1 is the argmax of the scaled logits
    for _ in range(50):
        V = int(rng.integers(2, 100))
        x = rng.standard_normal(V).astype(np.float32)
        res, _, _, _ = O.sample(O.make_params(temperature=0.7, topK=1, repeatPenalty=1.0), x, u=0.77)
        assert res.id == int(np.argmax(x))


def test_batch_candidates_match_single_rows():
    """The threaded batch call's first-cap candidates, results and ids equal
    one nlo_sample call per row (greedy, top-k and full-sort rows, penalties,
    bias, rows with fewer candidates than the cap)."""
    rng = np.random.default_rng(12)
    B, V, H, NB, cap = 24, 700, 16, 3, 64
    x = (rng.standard_normal((B, V)) * 2).astype(np.float32)
    x[3, :] = 0.5  # one flat row: every candidate tied
    plist, rows = [], []
    for b in range(B):
        kw = dict(temperature=[0.0, 0.8, 1.2][b % 3], topK=[0, 5, 40, 1000, V][b % 5],
                  topP=[1.0, 0.9][b % 2], minP=[0.0, 0.05][(b // 2) % 2], repeatPenalty=1.1,
                  repeatLastN=8, presencePenalty=0.2, frequencyPenalty=0.1, seed=b)
        plist.append(O.make_params(**kw))
        rows.append(kw)
    hist = rng.integers(0, V, (B, H)).astype(np.int64)
    hl = np.full(B, H, dtype=np.int64)
    bid = np.stack([rng.choice(V, NB, replace=False) for _ in range(B)]).astype(np.int64)
    bval = rng.standard_normal((B, NB))
    nb = np.full(B, NB, dtype=np.int64)
    u = rng.random(B)
    ids, res, ci, cp = O.sample_batch(plist, x, hist, hl, bid, bval, nb, u, O.EXPF_CR,
                                      nthreads=4, want_res=True, cand_cap=cap)
    for b in range(B):
        bias = {int(i): float(v) for i, v in zip(bid[b], bval[b])}
        r1, cand, probs, _ = O.sample(plist[b], x[b], hist[b], bias, u[b], O.EXPF_CR)
        assert ids[b] == r1.id and res[b].id == r1.id and res[b].n == r1.n
        m = min(len(cand), cap)
        assert np.array_equal(ci[b, :m], cand[:m]) and np.all(ci[b, m:] == -1)
        assert np.array_equal(cp[b, :m].view(np.uint32), probs[:m].view(np.uint32))


def test_penalty_identity_and_brute_force():
    rng = np.random.default_rng(4)
    V = 50
    x = rng.standard_normal(V).astype(np.float32)
    hist = list(rng.integers(0, V, size=30))
    # rp = 1, freq = pres = 0 leaves the logits untouched
    _, _, _, fl = O.sample(O.make_params(temperature=1.0, repeatPenalty=1.0), x, hist, u=0.1)
    assert np.array_equal(fl, x)
    # brute force over a hand-built history: one id seen 3 times, one id 1 time
    hist = [7, 7, 3, 7]
    p = O.make_params(temperature=1.0, repeatPenalty=2.0, frequencyPenalty=0.5,
                      presencePenalty=0.25, repeatLastN=0)
    x2 = np.zeros(V, dtype=np.float32)
    x2[7], x2[3] = 3.0, -1.0
    _, _, _, fl = O.sample(p, x2, hist, u=0.1)
    assert fl[7] == np.float32(3.0 / 2.0 - (3 * 0.5 + 0.25))
    assert fl[3] == np.float32(-1.0 * 2.0 - (1 * 0.5 + 0.25))
    # window: repeatLastN = 1 keeps only the last id
    p.repeatLastN = 1
    _, _, _, fl = O.sample(p, x2, hist, u=0.1)
    assert fl[3] == np.float32(-1.0) and fl[7] == np.float32(3.0 / 2.0 - 0.75)
    # bias -inf forbids a token even when it is the maximum
    res, _, _, _ = O.sample(O.make_params(temperature=0.0, repeatPenalty=1.0), x2, [],
                            {7: -math.inf})
    assert res.id != 7


def test_draw_inverts_the_cdf_on_a_u_grid():
    """For a tiny row, each u picks the candidate whose CDF interval holds u."""
    x = np.array([2.0, 1.0, 0.0, -1.0, 0.5], dtype=np.float32)
    p = O.make_params(temperature=1.0, topK=0, repeatPenalty=1.0)
    res, cand, probs, _ = O.sample(p, x, u=0.0)
    cdf = np.cumsum(probs.astype(np.float64))
    for u in np.linspace(0, 0.999, 400):
        if np.min(np.abs(cdf - u * cdf[-1])) < 1e-5:
            continue
        r, _, _, _ = O.sample(p, x, u=float(u))
        want = cand[int(np.searchsorted(cdf, u * cdf[-1]))]
        assert r.id == want


def test_top_tokens_and_softmax():
    x = np.array([0.5, 3.0, 3.0, -1.0], dtype=np.float32)
    ids = np.zeros(3, dtype=np.int64)
    pr = np.zeros(3, dtype=np.float32)
    m = O.lib().nlo_top_tokens(x.ctypes.data_as(O.ctypes.POINTER(O.ctypes.c_float)), 4, 3, 0,
                               ids.ctypes.data_as(O.ctypes.POINTER(O.ctypes.c_int64)),
                               pr.ctypes.data_as(O.ctypes.POINTER(O.ctypes.c_float)))
    assert m == 3 and list(ids) == [1, 2, 0]
    e = np.exp(x.astype(np.float64) - 3.0)
    assert np.allclose(pr, (e / e.sum())[[1, 2, 0]], rtol=1e-6)


def _oracle_top_tokens(x, n, mode=None):
    mode = O.EXPF_CR if mode is None else mode
    x = np.ascontiguousarray(x, dtype=np.float32)
    m = min(n, x.size)
    ids = np.zeros(max(m, 1), dtype=np.int64)
    pr = np.zeros(max(m, 1), dtype=np.float32)
    got = O.lib().nlo_top_tokens(x.ctypes.data_as(O.ctypes.POINTER(O.ctypes.c_float)), x.size, n, mode,
                                 ids.ctypes.data_as(O.ctypes.POINTER(O.ctypes.c_int64)),
                                 pr.ctypes.data_as(O.ctypes.POINTER(O.ctypes.c_float)))
    return ids[:got], pr[:got]


def _numpy_softmax(x):
    """softmaxInPlace (:51-57) from numpy parts: Nim's max (a NaN never
    replaces mx), exp per element through the oracle's correctly rounded expf,
    the fp32 sum accumulated strictly in index order (np.add.accumulate) and
    numpy's fp32 division."""
    x = np.asarray(x, dtype=np.float32)
    mx = np.float32(-np.inf)
    for v in x:
        if mx <= v:
            mx = v
    e = np.array([O.lib().nlo_expf_cr(float(np.float32(v - mx))) for v in x], dtype=np.float32)
    s = np.add.accumulate(e, dtype=np.float32)[-1]
    return (e / s).astype(np.float32)


def _numpy_top_tokens(x, n):
    """softmaxInPlace (:51-57) and the stable descending sort (:127-128) from
    numpy parts: _numpy_softmax, then numpy's stable argsort."""
    p = _numpy_softmax(x)
    order = np.argsort(-p, kind="stable")[:min(n, p.size)]
    return order, p[order]


def test_softmax_and_log_prob_oracle_pins():
    """softmaxInPlace (sampler.nim:51-57) and logProb's per-token term
    (nimllm-doc-en.md:1700-1707: ln of the float32 probability, widened)
    against the numpy restatement and math.log; equal logits over a power of
    two give exactly 1/V."""
    rng = np.random.default_rng(17)
    rows = [rng.normal(0, 2.5, 3000).astype(np.float32),
            (np.round(rng.normal(0, 2, 2000) * 4) / 4).astype(np.float32),
            np.full(50, 1.25, np.float32), np.array([0.5], np.float32),
            np.array([-np.inf, 1.0, np.nan, 2.0], np.float32)]
    for x in rows:
        want = _numpy_softmax(x)
        got = O.softmax(x)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        for t in (0, len(x) // 2, len(x) - 1):
            p, lp = O.log_prob(x, t)
            assert p.view(np.uint32) == want[t].view(np.uint32)
            if want[t] == want[t]:
                assert lp == math.log(float(want[t])) if want[t] > 0 else lp == -math.inf
            else:
                assert math.isnan(lp)
    p, lp = O.log_prob(np.full(1024, -3.0, np.float32), 5)
    assert p == np.float32(1.0 / 1024) and lp == math.log(1.0 / 1024)
    assert math.isnan(O.log_prob(rows[0], -1)[1]) and math.isnan(O.log_prob(rows[0], 3000)[1])


def test_top_tokens_oracle_pins():
    """The oracle's topTokens against a numpy restatement built from library
    parts, on rows where probabilities tie although the logits differ (the
    order must follow the probability, then the index, not the logit)."""
    rng = np.random.default_rng(7)
    rows = [rng.normal(0, 2.5, 3000).astype(np.float32),
            (np.round(rng.normal(0, 2, 2000) * 4) / 4).astype(np.float32),
            np.full(50, 1.25, np.float32)]
    col = rng.normal(-6, 1, 1000).astype(np.float32)
    # four logits within 2.9e-8 below the maximum: exp rounds them to 1.0, so
    # their probabilities equal the maximum's and they follow in index order
    col[[3, 10, 400, 999]] = np.array([-2.5e-8, -1e-8, 0.0, -2e-8], np.float32)
    rows.append(col)
    for x in rows:
        for n in (1, 5, 37, 4000):
            ids, pr = _oracle_top_tokens(x, n)
            want_ids, want_p = _numpy_top_tokens(x, n)
            assert np.array_equal(ids, want_ids)
            assert np.array_equal(pr.view(np.uint32), want_p.view(np.uint32))
    ids, _ = _oracle_top_tokens(col, 4)
    assert list(ids) == [3, 10, 400, 999]


def test_row_nll_oracle_pins():
    """perplexity's per-position term (src/nimllm/model.nim:578-583) in the
    oracle, pinned by closed forms and a float64 library evaluation."""
    import math

    # all logits equal: s = V exactly, nll = ln(V)
    for V in (1, 7, 1000, 32000):
        assert O.row_nll(np.full(V, 2.5, np.float32), V // 2) == math.log(V)
    # two values a > b with counts: nll of a = ln(ca + cb e^(b - a))
    x = np.array([1.0, -2.0, 1.0, -2.0, -2.0], np.float32)
    want = math.log(2.0 + 3.0 * math.exp(-3.0))
    assert abs(O.row_nll(x, 0) - want) <= 1e-15 * want
    assert abs(O.row_nll(x, 1) - (want + 3.0)) <= 1e-15 * (want + 3.0)
    # random rows against a float64 evaluation of the same terms (numpy's
    # exp and pairwise sum): equal to rounding
    rng = np.random.default_rng(11)
    for V in (10, 5000, 128256):
        x = (rng.standard_normal(V) * 2.5).astype(np.float32)
        t = int(rng.integers(0, V))
        mx = np.float32(np.max(x))
        d = (x - mx).astype(np.float32).astype(np.float64)
        ref = -(float(d[t]) - math.log(float(np.sum(np.exp(d)))))
        got = O.row_nll(x, t)
        assert abs(got - ref) <= 1e-12 * max(1.0, abs(ref)), (V, got, ref)
    # NaN: max skips it (Nim's max keeps mx), the sum does not: NaN
    x = np.array([0.5, np.nan, 1.5], np.float32)
    assert math.isnan(O.row_nll(x, 0))
    # -inf entries add exp(-inf) = 0
    x = np.array([0.0, -np.inf, 0.0], np.float32)
    assert O.row_nll(x, 2) == math.log(2.0)
