"""GPU parity: the HIP sampler (through the C ABI) against the CPU oracle.

The bar: sampled ids, candidate lists, n and post-softmax probabilities are
bit-identical to the oracle run with the correctly rounded exp (the sampler's
exp).  Against the oracle run with the C library's expf (what the reference's
exp(float32) binds to on Linux), ids may differ only on rows where the two
oracle variants themselves disagree (exception class "libm exp", counted).
"""
import math
import sys

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def torch():
    import torch as t

    assert t.cuda.is_available(), "no GPU"
    return t


def run_gpu(pkg, torch, logits, params, hist=None, u=None, debug_cap=0, accept_rows=None):
    B, V = logits.shape
    s = pkg.BatchSampler(params, V)
    try:
        if hist is not None and hist.shape[1] > 0:
            if accept_rows is None:
                s.accept(hist)
            else:
                for b in range(B):
                    s.accept(hist[b, :accept_rows[b]], row=b)
        d = torch.from_numpy(np.ascontiguousarray(logits)).cuda()
        du = None if u is None else torch.from_numpy(np.ascontiguousarray(u, dtype=np.float64)).cuda()
        res = s.sample(d, du, debug_cap=debug_cap)
        torch.cuda.synchronize()
        if debug_cap:
            ids, dbg = res
            return ids.cpu().numpy(), {k: v.cpu().numpy() for k, v in dbg.items()}
        return res.cpu().numpy(), None
    finally:
        s.close()


def oracle_row(x, p, hist, bias, u, mode):
    return O.sample(O.make_params(**p), x, hist, bias, u, mode)


def rand_params(rng, V):
    mode = int(rng.integers(0, 6))
    p = dict(temperature=float(rng.choice([0.5, 0.7, 1.0, 1.3])),
             topK=int(rng.choice([0, 1, 3, 20, 50, 300, V - 1, V, V + 5])),
             topP=float(rng.choice([0.0, 0.5, 0.9, 0.95, 1.0])),
             minP=float(rng.choice([0.0, 0.0, 0.05, 0.1])),
             repeatPenalty=float(rng.choice([1.0, 1.0, 1.1, 0.8])),
             repeatLastN=int(rng.choice([0, 8, 64])),
             presencePenalty=float(rng.choice([0.0, 0.3])),
             frequencyPenalty=float(rng.choice([0.0, 0.5])),
             seed=1)
    if mode == 0:
        p["temperature"] = 0.0
    if p["topK"] > 0 and p["topK"] >= V:
        p["topK"] = V
    return p


def to_pkg_params(pkg, p, bias):
    sp = pkg.SamplerParams(**p)
    sp.logitBias = dict(bias)
    return sp


def compare_rows(x, plist, hists, biases, u, ids, dbg, tag):
    """Exact comparison of every row against the oracle (CR exp)."""
    for b in range(x.shape[0]):
        res, cand, probs, _ = oracle_row(x[b], plist[b], hists[b], biases[b], float(u[b]), O.EXPF_CR)
        assert ids[b] == res.id, (tag, b, plist[b], int(ids[b]), res.id)
        if dbg is not None and not res.greedy:
            n = int(dbg["n"][b])
            assert n == res.n, (tag, b, n, res.n)
            cap = dbg["cand_ids"].shape[1]
            m = min(n, cap)
            assert list(dbg["cand_ids"][b][:m]) == [int(c) for c in cand[:m]], (tag, b)
            assert np.array_equal(dbg["cand_probs"][b][:m].view(np.uint32),
                                  probs[:m].view(np.uint32)), (tag, b)
            assert dbg["total"][b].view(np.uint32) == np.float32(res.total).view(np.uint32)


@pytest.mark.parametrize("V", [1, 2, 7, 100, 1000, 5000, 16384, 16385, 40000])
def test_small_random_rows(pkg, torch, V):
    rng = np.random.default_rng(V)
    B = 24
    say(f"[small_random_rows] V={V} B={B}")
    grid = [None, 4.0][V % 2]
    x = rng.standard_normal((B, V)).astype(np.float32) * np.float32(2.0)
    if grid:
        x = (np.round(x * grid) / grid).astype(np.float32)
    plist = [rand_params(rng, V) for _ in range(B)]
    H = 40
    hist = rng.integers(-2, V + 2, size=(B, H)).astype(np.int64)
    biases = []
    for b in range(B):
        nb = int(rng.integers(0, min(V, 6) + 1))
        ids = rng.choice(V, size=nb, replace=False) if nb else []
        biases.append({int(i): float(rng.choice([-math.inf, -2.0, 1.5, 6.0])) for i in ids})
    u = rng.random(B)
    u[0] = 0.0
    params = [to_pkg_params(pkg, plist[b], biases[b]) for b in range(B)]
    ids, dbg = run_gpu(pkg, torch, x, params, hist, u, debug_cap=V + 8)
    compare_rows(x, plist, [list(h) for h in hist], biases, u, ids, dbg, f"V={V}")


SWEEP = {
    # name: (B, V, top-k choices, offset of the logits in floats)
    "k64_rows": (300, 50000, (0, 1, 20, 64), 0),
    "k64_rows_odd_vocab": (300, 50001, (0, 1, 20, 64), 0),
    "k64_rows_unaligned": (280, 40000, (0, 5, 40), 1),
    "k64_k_is_64_all_tied": (260, 20000, (64, 63, 62), 0),
    "split_rows": (40, 100000, (0, 1, 20, 50), 0),
    "split_rows_unaligned": (40, 100000, (0, 3, 64), 3),
    "block_path_two_per_cu": (600, 30000, (65, 100, 300, 600), 0),
    "whole_row_mix": (24, 70000, (0, 20, 1000, 3000), 0),
    "small_rows_every_k": (16, 3000, (0, 1, 2999, 3000, 4000), 2),
    "split_rows_tied": (40, 100000, (64, 63, 33), 0),
    "block_path_tied": (600, 30000, (65, 128, 1000), 0),
    "whole_row_tied": (24, 70000, (0, 1024, 2048, 2049), 1),
    "one_row_tied": (1, 32000, (64,), 0),
    "one_row_large_tied": (1, 151936, (50,), 2),
    "few_rows_tied": (3, 128256, (0, 64, 2000), 0),
    # bias lists longer than the fixed stride (256) and than a workgroup (1024)
    "long_bias_lists": (300, 50000, (0, 20, 64), 0, 1500),
    "long_bias_lists_split": (24, 100000, (0, 1, 50, 300), 1, 600),
}


def _drawn_config(i):
    """Random sweep configuration i: (B, V, top-k choices, offset), drawn from
    a fixed seed with B x V at most 40 M logits."""
    r = np.random.default_rng(1000 + i)
    while True:
        B = int(r.choice([1, 2, 5, 33, 200, 257, 520]))
        V = int(r.choice([1000, 4097, 32000, 50001, 128256, 151936]))
        if B * V <= 40_000_000:
            break
    ks = tuple(int(k) for k in r.choice([0, 1, 2, 17, 63, 64, 65, 200, 1024, 2048, V - 1, V], size=4))
    return B, V, ks, int(r.integers(0, 4))


for _i in range(12):
    SWEEP[f"drawn_{_i}" + ("_tied" if _i % 3 == 0 else "")] = _drawn_config(_i)


@pytest.mark.parametrize("name", list(SWEEP))
def test_random_batches_every_path(pkg, torch, name):
    """Random batches over the planner's paths -- one workgroup per row
    (k64_kernel), rows split over workgroups, the k > 64 block path with two
    workgroups per CU, whole-row rows mixed in -- with vocabularies that are
    not a multiple of 4 and logits that are not 16-byte aligned (4-byte
    loads), random temperatures, top-k, top-p, min-p, penalties over
    histories with out-of-range ids, and bias lists with -inf: every row's
    id, n, total, candidates and probabilities against the oracle
    (sampler.nim:59-121)."""
    B, V, ks, off = SWEEP[name][:4]
    max_bias = SWEEP[name][4] if len(SWEEP[name]) > 4 else 8
    rng = np.random.default_rng(abs(sum(map(ord, name))))
    say(f"[random_sweep] {name}: B={B} V={V} offset={off}")
    x = (rng.standard_normal((B, V)) * rng.choice([1.0, 2.5, 4.0])).astype(np.float32)
    nt = B if "tied" in name else B // 4  # rows on a 0.25 grid: ties at every cut
    x[:nt] = (np.round(x[:nt] * 4.0) / 4.0).astype(np.float32)
    plist, biases = [], []
    for b in range(B):
        p = rand_params(rng, V)
        if p["temperature"] > 0:
            p["topK"] = int(rng.choice(ks))
        plist.append(p)
        nb = int(rng.integers(0, min(V, max_bias) + 1))
        ids = rng.choice(V, size=nb, replace=False) if nb else []
        biases.append({int(i): float(rng.choice([-math.inf, -3.0, 0.5, 4.0])) for i in ids})
    H = 96
    hist = rng.integers(-3, V + 3, size=(B, H)).astype(np.int64)
    u = rng.random(B)
    u[: min(3, B)] = [0.0, 1.0 - 2.0 ** -53, 0.5][: min(3, B)]
    params = [to_pkg_params(pkg, plist[b], biases[b]) for b in range(B)]
    s = pkg.BatchSampler(params, V)
    try:
        s.accept(hist)
        flat = torch.zeros(B * V + off, dtype=torch.float32, device="cuda")
        flat[off:] = torch.from_numpy(x.reshape(-1)).cuda()
        d = flat[off:].view(B, V)
        assert (d.data_ptr() % 16 == 0) == (off % 4 == 0)
        ids, dbg = s.sample(d, torch.from_numpy(u).cuda(), debug_cap=64)
        torch.cuda.synchronize()
        ids = ids.cpu().numpy()
        dbg = {k: v.cpu().numpy() for k, v in dbg.items()}
    finally:
        s.close()
    compare_rows(x, plist, [list(h) for h in hist], biases, u, ids, dbg, name)
    # the same batch on a fresh sampler without candidate lists (a caller's
    # launches: full-sort rows in a grouped launch, then the rows it leaves)
    s = pkg.BatchSampler(params, V)
    try:
        s.accept(hist)
        ids_plain = s.sample(d, torch.from_numpy(u).cuda()).cpu().numpy()
    finally:
        s.close()
    assert np.array_equal(ids_plain, ids), (name, np.nonzero(ids_plain != ids)[0][:10].tolist())


def patch_designs(rng, x):
    """Rows whose penalised or biased ids fall below the threshold, rise above
    it, or sit on it (sampler.nim:64-76): one design per row, cycling."""
    B, V = x.shape
    plist, hists, biases = [], [], []
    base = dict(temperature=1.0, topK=50, topP=1.0, minP=0.0, repeatPenalty=1.0, repeatLastN=0,
                presencePenalty=0.0, frequencyPenalty=0.0, seed=3)
    for b in range(B):
        order = np.argsort(-x[b], kind="stable")
        top, low = [int(i) for i in order[:200]], [int(i) for i in order[-200:]]
        d, h, bias = dict(base), [], {}
        kind = b % 16
        if kind == 0:    # the top ids penalised: met above the threshold, then fall
            d.update(repeatPenalty=1.5); h = top[:30]
        elif kind == 1:  # negative presence: penalised ids rise
            d.update(temperature=0.7, presencePenalty=-3.0); h = list(rng.choice(V, 20, replace=False))
        elif kind == 2:  # negative frequency on repeated ids
            d.update(frequencyPenalty=-1.0); h = [int(i) for i in rng.choice(V, 5, replace=False)] * 8
        elif kind == 3:  # rp < 1 lifts negative logits towards 0
            d.update(repeatPenalty=0.5); h = low[:30]
        elif kind == 4:  # a large positive bias on the lowest id
            bias = {low[0]: 30.0}
        elif kind == 5:  # greedy: a low id lifted to the top
            d.update(temperature=0.0, presencePenalty=-50.0); h = [low[3]]
        elif kind == 6:  # greedy: the top ids pushed down
            d.update(temperature=0.0, repeatPenalty=2.0, presencePenalty=5.0); h = top[:3]
        elif kind == 7:  # greedy with a NaN bias: skipped by argmax, except at index 0
            d.update(temperature=0.0)
            bias = {top[0]: math.nan} if (b // 16) % 2 == 0 else {0: math.nan, top[1]: 5.0}
        elif kind == 8:  # the top ten banned
            bias = {i: -math.inf for i in top[:10]}
        elif kind == 9:  # the common mixture
            d.update(topK=20, topP=0.9, minP=0.05, repeatPenalty=1.3, presencePenalty=0.5,
                     frequencyPenalty=0.5)
            h = top[:10] + [int(i) for i in rng.choice(V, 40)]
        elif kind == 10:  # a tiny penalty on the whole top 64
            d.update(topK=64, presencePenalty=0.01); h = top[:64]
        elif kind == 11:  # positive bias on random ids at a high temperature
            d.update(temperature=2.0); bias = {int(i): 2.0 for i in rng.choice(V, 30, replace=False)}
        elif kind == 12:  # greedy with both
            d.update(temperature=0.0, presencePenalty=1.0); h = top[:5]
            bias = {int(i): 1.0 for i in rng.choice(V, 10, replace=False)}
        elif kind == 13:  # k = 1 with the top penalised
            d.update(topK=1, frequencyPenalty=2.0); h = top[:2] * 3
        elif kind == 14:  # k > 64 with the top penalised
            d.update(topK=300, repeatPenalty=1.5); h = top[:100]
        else:            # k > 64 with a raising presence penalty
            d.update(topK=300, presencePenalty=-2.0); h = list(rng.choice(V, 50, replace=False))
        plist.append(d)
        hists.append([int(i) for i in h])
        biases.append(bias)
    return plist, hists, biases


@pytest.mark.parametrize("B,V", [(16, 70000), (16, 70001), (256, 50000)])
def test_patched_ids_that_fall_or_rise(pkg, torch, B, V):
    rng = np.random.default_rng(B * 7 + V)
    say(f"[patched_fall_rise] B={B} V={V}")
    x = (rng.standard_normal((B, V)) * 2.5).astype(np.float32)
    plist, hists, biases = patch_designs(rng, x)
    u = rng.random(B)
    H = max(len(h) for h in hists)
    hist = np.full((B, H), -1, dtype=np.int64)
    for b, h in enumerate(hists):
        hist[b, :len(h)] = h
    params = [to_pkg_params(pkg, plist[b], biases[b]) for b in range(B)]
    ids, dbg = run_gpu(pkg, torch, x, params, hist, u, debug_cap=64,
                       accept_rows=[len(h) for h in hists])
    compare_rows(x, plist, hists, biases, u, ids, dbg, f"B={B} V={V}")


NAN_POS = np.uint32(0x7FC00000).view(np.float32)  # sign bit clear: orders above +inf
NAN_NEG = np.uint32(0xFFC00000).view(np.float32)  # sign bit set: orders below -inf


@pytest.mark.parametrize("case", ["k64_topk40", "k64_small_topk50", "split_topk40", "full_sort",
                                  "topk300"])
def test_nan_rows_flagged_others_bit_exact(pkg, torch, case):
    """Sampling rows with a NaN final logit are outside the parity claim (the
    reference's heap and sort comparisons, sampler.nim:88-97, make them
    order-dependent).  The debug path code carries NLS_PATH_NAN (0x100) on
    every row whose candidates hold a NaN: always for a NaN with the sign bit
    clear (above +inf in the key order), and for one with it set (below
    -inf) on full-sort rows.  The batch's other rows stay bit-exact against
    the oracle and unflagged, and a greedy row with a NaN logit follows
    argmax (sampler.nim:45-49)."""
    V, k, B, seed = {"k64_topk40": (128256, 40, 256, 1), "k64_small_topk50": (32000, 50, 8, 2),
                     "split_topk40": (128256, 40, 12, 3), "full_sort": (50000, 0, 8, 4),
                     "topk300": (100000, 300, 8, 5)}[case]
    rng = np.random.default_rng(seed)
    say(f"[nan_rows] {case} B={B} V={V} k={k}")
    x = (rng.standard_normal((B, V)) * 2.0).astype(np.float32)
    base = dict(temperature=0.9, topK=k, topP=0.95, minP=0.0, repeatPenalty=1.0, repeatLastN=0,
                presencePenalty=0.0, frequencyPenalty=0.0, seed=3)
    plist = [dict(base) for _ in range(B)]
    biases = [{} for _ in range(B)]
    expect = {}  # row -> flagged?
    x[1, int(rng.integers(0, V))] = NAN_POS
    expect[1] = True
    x[2, rng.choice(V, 3 * max(k, 64), replace=False)] = NAN_POS  # more NaNs than candidates
    expect[2] = True
    biases[3] = {int(rng.integers(0, V)): math.nan}  # a NaN bias makes the final logit NaN
    expect[3] = True
    x[4, int(rng.integers(0, V))] = NAN_NEG
    expect[4] = k == 0  # a candidate only on a full-sort row
    x[5, 7] = NAN_POS  # greedy: argmax skips it
    plist[5]["temperature"] = 0.0
    clean = [b for b in range(B) if b not in expect and b != 5]
    params = [to_pkg_params(pkg, plist[b], biases[b]) for b in range(B)]
    u = rng.random(B)
    s = pkg.BatchSampler(params, V)
    try:
        plan, streamed = s.plan()
        say(f"[nan_rows] {case}: k64={plan.k64} streamed={sum(streamed)}")
        if case.startswith("k64"):
            assert plan.k64 and all(streamed)
        if case == "split_topk40":  # rows split over several workgroups
            assert not plan.k64 and all(streamed)
        d = torch.from_numpy(np.ascontiguousarray(x)).cuda()
        du = torch.from_numpy(u).cuda()
        ids, dbg = s.sample(d, du, debug_cap=64)
        torch.cuda.synchronize()
        ids = ids.cpu().numpy()
        dbg = {kk: vv.cpu().numpy() for kk, vv in dbg.items()}
    finally:
        s.close()
    assert ids.min() >= 0 and ids.max() < V
    path = dbg["path"]
    for b, flagged in expect.items():
        assert bool(path[b] & 0x100) == flagged, (case, b, hex(int(path[b])))
    assert not (path[5] & 0x100) and path[5] == 1
    res = O.sample(O.make_params(**plist[5]), x[5], (), {}, 0.5, O.EXPF_CR, want_cand=False)[0]
    assert ids[5] == res.id == int(np.argmax(np.where(np.isnan(x[5]), -np.inf, x[5])))
    for b in clean:
        assert not (path[b] & 0x100), (case, b, hex(int(path[b])))
    cd = {kk: vv[clean] for kk, vv in dbg.items()}
    compare_rows(x[clean], [plist[b] for b in clean], [()] * len(clean), [biases[b] for b in clean],
                 u[clean], ids[clean], cd, f"nan_rows {case}")


def test_mixed_batch_consecutive_calls(pkg, torch):
    """One sampler over a batch mixing greedy, top-k and full-sort rows
    (sampler.nim:77-97), called three times in a row on fresh logits and
    uniforms: every row of every call against the oracle.  Such a batch runs
    the streamed rows alone in the streaming grid and the full-sort rows from
    a fixed list, with the whole-row kernel's workgroups claiming rows from a
    counter that each call resets for the next."""
    B, V = 320, 30000
    rng = np.random.default_rng(77)
    plist, hists, biases = [], [], []
    for b in range(B):
        kind = b % 5
        d = dict(temperature=1.0, topK=0, topP=1.0, minP=0.0, repeatPenalty=1.0, repeatLastN=0,
                 presencePenalty=0.0, frequencyPenalty=0.0, seed=2)
        if kind == 0:
            d.update(temperature=0.0)
        elif kind == 1:
            d.update(topK=20)
        elif kind == 2:
            d.update(minP=0.1)
        elif kind == 3:
            d.update(topP=0.8)
        else:
            d.update(topK=50, presencePenalty=0.5, repeatLastN=16)
        plist.append(d)
        hists.append([int(i) for i in rng.integers(0, V, 24)])
        biases.append({int(rng.integers(0, V)): 1.5} if b % 7 == 0 else {})
    params = [to_pkg_params(pkg, plist[b], biases[b]) for b in range(B)]
    s = pkg.BatchSampler(params, V)
    try:
        plan, streamed = s.plan()
        say(f"[mixed_batch_calls] B={B} V={V} k64={plan.k64} streamed={sum(streamed)}")
        assert plan.k64 and 0 < sum(streamed) < B
        s.accept(np.array(hists, dtype=np.int64))
        for call in range(3):
            x = (np.round(rng.standard_normal((B, V)) * 8.0) / 4.0).astype(np.float32)
            u = rng.random(B)
            d = torch.from_numpy(x).cuda()
            du = torch.from_numpy(u).cuda()
            ids = s.sample(d, du).cpu().numpy()
            torch.cuda.synchronize()
            compare_rows(x, plist, hists, biases, u, ids, None, f"call {call}")
    finally:
        s.close()


def _walk_split_batch(B, V, rng):
    """A batch with more full-sort rows than an MI355X has CUs: rows on a 0.25
    grid (heavy ties: drawn groups of many members), some with distinct values
    (groups of one, or more distinct values than the group table holds), and
    cutoffs that need candidates below the grouped path's floor."""
    plist, hists, biases = [], [], []
    for b in range(B):
        kind = b % 10
        d = dict(temperature=1.0, topK=0, topP=1.0, minP=0.0, repeatPenalty=1.0, repeatLastN=0,
                 presencePenalty=0.0, frequencyPenalty=0.0, seed=4)
        h, bias = [], {}
        if kind == 0:
            d.update(temperature=0.0)
        elif kind == 1:
            d.update(topK=20)
        elif kind == 2:
            d.update(topP=0.9)
        elif kind == 3:
            d.update(temperature=0.7, minP=0.05)
        elif kind == 4:
            d.update(repeatPenalty=1.3, presencePenalty=0.5, repeatLastN=16)
            h = [int(i) for i in rng.integers(0, V, 24)]
            bias = {int(rng.integers(0, V)): 2.5, int(rng.integers(0, V)): -math.inf}
        elif kind == 5:  # top-p just below 1 at a low temperature: the cut may need every candidate
            d.update(temperature=0.5, topP=1.0 - 1e-9)
        elif kind == 7:
            d.update(topP=0.5, minP=0.1)
        elif kind == 8:
            d.update(temperature=2.0, topP=0.95)
        plist.append(d)
        hists.append(h)
        biases.append(bias)
    return plist, hists, biases


def test_grouped_walk_split_consecutive_calls(pkg, torch, monkeypatch):
    """More full-sort rows than CUs: the grouped launch stores each row's
    groups, a launch of one-wave workgroups walks them (softmax sum, top-p,
    min-p, total, draw; sampler.nim:101-121) and a third searches the drawn
    member; rows any step cannot finish go to the whole-row launch with their
    uniform.  One sampler, five calls in a row, alternating between calls
    without candidate lists (the split launches) and calls with them (one
    launch): every row of every call against the oracle.  The same batch with
    the split switched off (NLS_WALK_SPLIT=0) gives the same ids."""
    B, V = 640, 32000
    rng = np.random.default_rng(91)
    plist, hists, biases = _walk_split_batch(B, V, rng)
    params = [to_pkg_params(pkg, plist[b], biases[b]) for b in range(B)]
    calls = []
    for call in range(5):
        x = (np.round(rng.standard_normal((B, V)) * 8.0) / 4.0).astype(np.float32)
        x[9::10] = (rng.standard_normal((len(range(9, B, 10)), V)) * 3.0).astype(np.float32)
        calls.append((x, rng.random(B)))
    s = pkg.BatchSampler(params, V)
    try:
        plan, _ = s.plan()
        say(f"[walk_split_calls] B={B} V={V} walk_split={plan.walk_split}")
        assert plan.walk_split == 1
        for b in range(B):
            if hists[b]:
                s.accept(hists[b], row=b)
        first = None
        for call, (x, u) in enumerate(calls):
            d = torch.from_numpy(x).cuda()
            du = torch.from_numpy(u).cuda()
            if call % 2:
                ids, dbg = s.sample(d, du, debug_cap=64)
                dbg = {k: v.cpu().numpy() for k, v in dbg.items()}
            else:
                ids, dbg = s.sample(d, du), None
            ids = ids.cpu().numpy()
            torch.cuda.synchronize()
            say(f"[walk_split_calls] call {call} debug={dbg is not None}")
            compare_rows(x, plist, hists, biases, u, ids, dbg, f"call {call}")
            if call == 0:
                first = ids
    finally:
        s.close()
    monkeypatch.setenv("NLS_WALK_SPLIT", "0")
    s = pkg.BatchSampler(params, V)
    try:
        plan, _ = s.plan()
        assert plan.walk_split == 0
        for b in range(B):
            if hists[b]:
                s.accept(hists[b], row=b)
        x, u = calls[0]
        ids = s.sample(torch.from_numpy(x).cuda(), torch.from_numpy(u).cuda()).cpu().numpy()
    finally:
        s.close()
    assert np.array_equal(ids, first)


def _floor_batch(B, V, rng):
    """Full-sort rows only: peaked rows (a Zipf head over noise, few values
    near the maximum), flat rows (every value near it: more than a slice
    keeps), rows on a 0.25 grid (ties), a NaN row and an all -inf row but one
    id; top-p, min-p, both or neither; penalties over windows and biases."""
    x = rng.standard_normal((B, V)).astype(np.float32)
    plist, hists, biases = [], [], []
    for b in range(B):
        kind = b % 8
        if kind in (0, 1, 2, 3):  # peaked
            x[b] += (-4.4 * np.log(1 + rng.permutation(V))).astype(np.float32)
        elif kind == 4:  # ties
            x[b] = (np.round(x[b] * 8.0) / 4.0).astype(np.float32)
        elif kind == 5:  # flat
            x[b] *= np.float32(0.5)
        d = dict(temperature=float(rng.choice([0.5, 0.7, 1.0, 1.5])), topK=0,
                 topP=float(rng.choice([1.0, 0.9, 0.5, 0.999])), minP=float(rng.choice([0.0, 0.05, 0.2])),
                 repeatPenalty=float(rng.choice([1.0, 1.1])), repeatLastN=int(rng.choice([0, 16])),
                 presencePenalty=float(rng.choice([0.0, -2.0, 0.5])), frequencyPenalty=0.0, seed=5)
        if b % 16 == 6:
            d.update(topP=1.0, minP=0.0)  # neither cut: every candidate kept
        h = [int(i) for i in rng.integers(0, V, 40)] if b % 3 else []
        top = int(np.argmax(x[b]))
        if b % 5 == 0:
            h += [top] * 3  # the maximum penalised
        bias = {}
        if b % 4 == 1:
            bias = {int(rng.integers(0, V)): 6.0, top: -math.inf}
        plist.append(d)
        hists.append(h)
        biases.append(bias)
    if B > 7:
        x[7, V // 2] = np.nan
    if B > 15:
        x[15, :] = -np.inf
        x[15, V - 1] = 0.0
    return x, plist, hists, biases


@pytest.mark.parametrize("B,V", [(8, 1000), (33, 16384), (16, 16385), (40, 50001), (64, 128256),
                                 (24, 151936), (256, 32000), (51, 151936), (16, 200000), (96, 128256)])
def test_full_sort_rows_split_over_slices(pkg, torch, monkeypatch, B, V):
    """A batch of full-sort rows only (sampler.nim:96-121) whose slices of
    16384 values fit the GPU at once (two workgroups per CU): each row split
    over slices whose workgroups keep the values within the floor of their
    maximum, the last one merging and running
    the tail; rows it cannot finish (flat rows, NaN, a chain past the kept
    values, candidate lists longer than them) go to the whole-row kernel.  Two
    calls on one sampler (with and without candidate lists) against the
    oracle, then the same batch with the split switched off (NLS_FLOOR=0).
    (51 x 151936: 510 slice workgroups, about all the GPU holds at once;
    16 x 200000: a vocabulary past the grouped path's tables, so the rows
    handed on take the whole-row sort; 96 x 128256: too many slices for one
    round, so the grouped path takes the batch.)"""
    rng = np.random.default_rng(B * 7 + V)
    x, plist, hists, biases = _floor_batch(B, V, rng)
    params = [to_pkg_params(pkg, plist[b], biases[b]) for b in range(B)]
    say(f"[floor_rows] B={B} V={V}")
    u = rng.random(B)
    u[: min(3, B)] = [0.0, 1.0 - 2.0 ** -53, 0.5][: min(3, B)]
    d = torch.from_numpy(x).cuda()
    du = torch.from_numpy(u).cuda()
    s = pkg.BatchSampler(params, V)
    try:
        plan, _ = s.plan()
        S = (V + 16383) // 16384
        ncu = torch.cuda.get_device_properties(0).multi_processor_count
        assert plan.floor_slices == (S if B * S <= 2 * ncu else 0), (plan.floor_slices, ncu)
        for b in range(B):
            if hists[b]:
                s.accept(hists[b], row=b)
        ids, dbg = s.sample(d, du, debug_cap=64)
        torch.cuda.synchronize()
        ids = ids.cpu().numpy()
        dbg = {k: v.cpu().numpy() for k, v in dbg.items()}
        ok = np.array([not (np.isnan(x[b]).any()) for b in range(B)])
        compare_rows(x[ok], [p for p, o in zip(plist, ok) if o], [h for h, o in zip(hists, ok) if o],
                     [c for c, o in zip(biases, ok) if o], u[ok], ids[ok],
                     {k: v[ok] for k, v in dbg.items()}, f"floor B={B} V={V} lists")
        ids2 = s.sample(d, du).cpu().numpy()
        torch.cuda.synchronize()
        assert np.array_equal(ids2, ids), np.nonzero(ids2 != ids)[0][:10].tolist()
    finally:
        s.close()
    monkeypatch.setenv("NLS_FLOOR", "0")
    s = pkg.BatchSampler(params, V)
    try:
        assert s.plan()[0].floor_slices == 0
        for b in range(B):
            if hists[b]:
                s.accept(hists[b], row=b)
        ids3 = s.sample(d, du).cpu().numpy()
    finally:
        s.close()
    assert np.array_equal(ids3, ids), np.nonzero(ids3 != ids)[0][:10].tolist()


@pytest.mark.parametrize("B", [12, 264])
def test_greedy_rows_resting_on_patched_ids_or_neg_inf(pkg, torch, B):
    """Greedy rows (sampler.nim:45-49, :77-78) whose argmax rests on -inf or
    on a patched id: rows of -inf with index 0 penalised or banned (answer
    0), a biased id tying the maximum at a smaller index than an unpatched
    one in the same lane, the same tie at a larger index (a later chunk of
    the same lane), and an all -inf row but for its last id.  (B = 12 splits
    rows over the CUs; B = 264 gives every row a workgroup.)"""
    V = 70000
    base = dict(temperature=0.0, topK=0, topP=1.0, minP=0.0, repeatPenalty=1.0, repeatLastN=0,
                presencePenalty=0.0, frequencyPenalty=0.0, seed=5)
    x = np.full((B, V), -1.0, dtype=np.float32)
    plist, hists, biases = [], [], []
    for b in range(B):
        d, h, bias = dict(base), [], {}
        kind = b % 6
        if kind == 0:    # all -inf, index 0 penalised
            x[b] = -np.inf; d.update(repeatPenalty=1.5); h = [0, 0, 17]
        elif kind == 1:  # all -inf, index 0 banned
            x[b] = -np.inf; bias = {0: -math.inf, 9: -2.0}
        elif kind == 2:  # the biased (unchanged) id at 5 ties the unpatched 7 and 16389
            x[b, [5, 7, 16389]] = 2.0; bias = {5: 0.0}
        elif kind == 3:  # an unchanged id at 16389 ties 7, met later in the same lane
            x[b, [7, 16389, 40000]] = 2.0; bias = {16389: 0.0}
        elif kind == 4:  # all -inf but the last id, penalised to 0.0
            x[b] = -np.inf; x[b, V - 1] = 0.0; d.update(repeatPenalty=2.0); h = [V - 1]
        else:            # all -inf, penalised ids around index 0
            x[b] = -np.inf; d.update(presencePenalty=1.0); h = [3, 0]
        if (b // 6) % 2:  # the same rows with a top id that its presence penalty takes to -950
            x[b, 60000] = 50.0; h = h + [60000]; d.update(presencePenalty=1000.0)
        plist.append(d)
        hists.append([int(i) for i in h])
        biases.append(bias)
    say(f"[greedy_edge_rows] B={B} V={V}")
    u = np.zeros(B)
    H = max(len(h) for h in hists)
    hist = np.full((B, H), -1, dtype=np.int64)
    for b, h in enumerate(hists):
        hist[b, :len(h)] = h
    params = [to_pkg_params(pkg, plist[b], biases[b]) for b in range(B)]
    ids, dbg = run_gpu(pkg, torch, x, params, hist, u, debug_cap=64,
                       accept_rows=[len(h) for h in hists])
    compare_rows(x, plist, hists, biases, u, ids, dbg, f"B={B} V={V}")


@pytest.mark.parametrize("B", [8, 300, 600])
def test_topk_rows_in_sorted_order(pkg, torch, B):
    """Top-k rows (64 < k <= 2048) whose first tile is not typical of the row:
    logits in descending order (the first tile holds the row's largest values,
    so a threshold taken from it admits fewer than k), ascending order, and
    shuffled, with ties.  Every id, candidate list and probability must match
    the oracle."""
    rng = np.random.default_rng(4242 + B)
    V = 60000
    say(f"[topk_sorted] B={B} V={V}")
    base = (rng.standard_normal((B, V)) * 2.0).astype(np.float32)
    x = np.empty_like(base)
    for b in range(B):
        r = np.sort(base[b])
        if b % 4 == 0:
            x[b] = r[::-1]
        elif b % 4 == 1:
            x[b] = r
        elif b % 4 == 2:
            x[b] = np.round(r[::-1] * 4.0) / 4.0
        else:
            x[b] = base[b]
    ks = [65, 200, 1000, 2048]
    plist = [dict(temperature=1.0, topK=ks[b % len(ks)], topP=0.95, minP=0.0, repeatPenalty=1.0,
                  repeatLastN=0, presencePenalty=0.0, frequencyPenalty=0.0, seed=1) for b in range(B)]
    u = rng.random(B)
    params = [to_pkg_params(pkg, plist[b], {}) for b in range(B)]
    ids, dbg = run_gpu(pkg, torch, x, params, None, u, debug_cap=64)
    compare_rows(x, plist, [[] for _ in range(B)], [{} for _ in range(B)], u, ids, dbg, f"B={B}")


def test_topk_rows_with_window_and_bias_two_per_cu(pkg, torch):
    """A batch of top-k rows (64 < k <= 2048) large enough for two streaming
    workgroups per CU, with repetition/frequency/presence penalties over a
    bounded window and logit bias, so the patch table is in use on that
    path; ids, candidates and probabilities against the oracle."""
    rng = np.random.default_rng(777)
    B, V, H = 560, 24000, 48
    say(f"[topk_two_per_cu] B={B} V={V}")
    x = (rng.standard_normal((B, V)) * 2.0).astype(np.float32)
    x[::7] = np.round(x[::7] * 4.0) / 4.0  # ties on some rows
    hist = rng.integers(0, V, size=(B, H)).astype(np.int64)
    hist[:, H // 2:] = hist[:, :H // 2]  # repeated ids: counts above one
    ks = [65, 130, 700, 2048]
    plist, biases = [], []
    for b in range(B):
        plist.append(dict(temperature=float(rng.choice([0.7, 1.0])), topK=ks[b % len(ks)],
                          topP=float(rng.choice([0.9, 1.0])), minP=float(rng.choice([0.0, 0.05])),
                          repeatPenalty=1.1, repeatLastN=32, presencePenalty=0.3,
                          frequencyPenalty=0.5, seed=1))
        ids = rng.choice(V, 6, replace=False)
        bias = {int(i): float(rng.uniform(-5, 5)) for i in ids}
        bias[int(ids[0])] = -math.inf
        bias[int(ids[1])] = 6.0  # a raising bias
        biases.append(bias)
    u = rng.random(B)
    params = [to_pkg_params(pkg, plist[b], biases[b]) for b in range(B)]
    ids_, dbg = run_gpu(pkg, torch, x, params, hist, u, debug_cap=64)
    compare_rows(x, plist, [list(hist[b]) for b in range(B)], biases, u, ids_, dbg, "two_per_cu")


@pytest.mark.parametrize("B,V,k", [(256, 128256, 50), (64, 50000, 300)])
def test_long_windows_full_batch(pkg, torch, B, V, k):
    """Whole-history penalties (repeatLastN = 0) over 6000 accepted ids per row,
    4500 of them distinct, plus 50 bias ids: more patched ids than the
    streaming kernel's LDS table holds, on every row of a full batch.  The
    rows go to the whole-row kernel, launched across the CUs; ids,
    candidates, probabilities, n and total against the oracle, and the call
    stays within a few times the streaming kernel's time (no serial cliff)."""
    rng = np.random.default_rng(4096 + k)
    H, distinct = 6000, 4500
    say(f"[long_windows] B={B} V={V} k={k} H={H} distinct={distinct}")
    x = (rng.standard_normal((B, V)) * 2.5).astype(np.float32)
    hist = np.empty((B, H), dtype=np.int64)
    for b in range(B):
        ids = rng.choice(V, distinct, replace=False)
        hist[b] = np.concatenate([ids, ids[:H - distinct]])[rng.permutation(H)]
    plist, biases = [], []
    for b in range(B):
        plist.append(dict(temperature=0.0 if b % 8 == 7 else 1.0, topK=k, topP=0.95, minP=0.0,
                          repeatPenalty=1.0 if k == 50 else 1.1, repeatLastN=0,
                          presencePenalty=0.3, frequencyPenalty=0.5, seed=1))
        bid = rng.choice(V, 50, replace=False)
        bias = {int(i): float(rng.uniform(-5, 5)) for i in bid}
        for i in bid[:5]:
            bias[int(i)] = -math.inf
        biases.append(bias)
    u = rng.random(B)
    params = [to_pkg_params(pkg, plist[b], biases[b]) for b in range(B)]
    s = pkg.BatchSampler(params, V)
    try:
        s.accept(hist)
        d = torch.from_numpy(x).cuda()
        du = torch.from_numpy(u).cuda()
        ids_, dbg = s.sample(d, du, debug_cap=64)
        torch.cuda.synchronize()
        ids_ = ids_.cpu().numpy()
        dbg = {kk: v.cpu().numpy() for kk, v in dbg.items()}
        out = torch.empty(B, dtype=torch.int32, device="cuda")
        for _ in range(3):
            s.sample(d, du, out)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(10):
            s.sample(d, du, out)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 100.0
        say(f"[long_windows] B={B} V={V} k={k}: {us:.1f} us per call; paths "
            f"{np.bincount(dbg['path'], minlength=6).tolist()}")
    finally:
        s.close()
    compare_rows(x, plist, [list(hist[b]) for b in range(B)], biases, u, ids_, dbg, "long_windows")
    topk_rows = np.array([p["temperature"] > 0 for p in plist])
    assert np.all(dbg["path"][topk_rows] == 5), np.bincount(dbg["path"][topk_rows], minlength=6).tolist()
    assert us < 5000.0, us


def test_k64_long_candidate_lists(pkg, torch):
    """Top-k rows (k <= 64) whose candidate list at the end of the stream is
    longer than the rank table (the penalties recipe at V = 151936 with the
    benchmark's seed) take the workgroup select over the list, not the
    whole-row path; rows with a flat top (logits on a coarse grid, whose ties
    can also fill a wave's buffer and hand the row on) stay exact; every row
    against the oracle."""
    from nimllm_amd import workloads

    rng = np.random.default_rng(2024)
    B, V = 64, 128256
    x = (np.round(rng.standard_normal((B, V)) * 2.0) / 2.0).astype(np.float32)
    plist = [dict(temperature=1.0, topK=[50, 64, 20, 33][b % 4], topP=0.95, minP=0.0, repeatPenalty=1.0,
                  repeatLastN=0, presencePenalty=0.0, frequencyPenalty=0.0, seed=1) for b in range(B)]
    u = rng.random(B)
    say(f"[k64_long_lists] grid rows B={B} V={V}")
    ids, dbg = run_gpu(pkg, torch, x, [to_pkg_params(pkg, p, {}) for p in plist], None, u, debug_cap=64)
    say(f"[k64_long_lists] grid rows: paths {np.bincount(dbg['path'], minlength=6).tolist()}")
    compare_rows(x, plist, [[] for _ in range(B)], [{} for _ in range(B)], u, ids, dbg, "grid")
    w = workloads.make("penalties_152k", seed=1234)
    say(f"[k64_long_lists] penalties_152k seed 1234 B={w.B} V={w.V}")
    ids, dbg = run_gpu(pkg, torch, w.logits, workloads.sampler_params(w, pkg), w.hist, w.u, debug_cap=64)
    assert np.all(dbg["path"] == 2), np.bincount(dbg["path"], minlength=6).tolist()
    bid, bval, bcnt = w.bias_arrays()
    ref = O.sample_batch([O.make_params(**r.as_kwargs()) for r in w.rows], w.logits, w.hist,
                         np.full(w.B, w.hist.shape[1]), bid, bval, bcnt, w.u, O.EXPF_CR, nthreads=8)
    assert np.array_equal(ids, ref), np.nonzero(ids != ref)[0][:10]


def test_golden_fixtures(pkg, torch):
    import json
    import os

    path = os.path.join(os.path.dirname(__file__), "golden", "sampler_cases.json")
    cases = json.load(open(path))["cases"]
    for c in cases:
        say(f"[golden] {c['name']} V={c['V']}")
        x = np.array(c["logits_bits"], dtype=np.uint32).view(np.float32).reshape(1, -1)
        bias = {k: (-math.inf if v == "-inf" else math.inf if v == "inf" else v) for k, v in c["bias"]}
        p = to_pkg_params(pkg, c["params"], bias)
        hist = np.array([c["history"]], dtype=np.int64).reshape(1, -1)
        ids, dbg = run_gpu(pkg, torch, x, [p], hist, np.array([c["u"]]), debug_cap=c["V"] + 4)
        e = c["expect"]
        assert int(ids[0]) == e["id"], c["name"]
        if not e["greedy"]:
            n = int(dbg["n"][0])
            assert n == e["n"], c["name"]
            assert [int(v) for v in dbg["cand_ids"][0][:n]] == e["cand"], c["name"]
            assert [int(v) for v in dbg["cand_probs"][0][:n].view(np.uint32)] == e["probs_bits"]


WORKLOAD_NAMES = ["single_32k", "zipf_minp_128k", "headline", "penalties_152k", "flat_topk1000",
                  "mixed_ties_152k"]
# The parity window: a row may differ from the reference (the oracle
# with the C library's expf) only when one of its draws or cutoffs lies within
# 1e-6 of a boundary: the draw (margin_draw, in units of the CDF), the top-p
# running sum (margin_topp, absolute) or the min-p threshold (margin_minp,
# relative to the threshold).
EXC_WINDOW = 1e-6


def exception_classes(res):
    """The exception classes (draw, top-p, min-p boundary) a row falls in, from
    an oracle Result."""
    out = []
    if res.greedy:
        return out
    if res.margin_draw < EXC_WINDOW:
        out.append("E1_draw")
    if res.margin_topp < EXC_WINDOW:
        out.append("E2_topp")
    if res.margin_minp < EXC_WINDOW:
        out.append("E3_minp")
    return out


def write_report(name, record):
    """Appends one JSON line per workload to $NLS_PARITY_REPORT when set."""
    import json
    import os

    path = os.environ.get("NLS_PARITY_REPORT")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps(dict(workload=name, **record)) + "\n")


@pytest.mark.parametrize("name", WORKLOAD_NAMES)
def test_workload_parity(pkg, torch, name):
    """Every row of the workload at full size against the oracle, in both exp
    modes.  Against the correctly rounded exp (the device's) ids, n, the
    total and the first min(n, 64) kept candidates (ids and probabilities)
    are bit-exact on every sampling row.  Against the C library's expf (what the
    reference's exp(float32) calls) a row may differ only inside the 1e-6
    window of a draw or cutoff boundary, which the libm oracle's own margins must show."""
    from nimllm_amd import workloads

    w = workloads.make(name, seed=7)
    say(f"[workload_parity] {name} B={w.B} V={w.V}")
    params = workloads.sampler_params(w, pkg)
    ids, dbg = run_gpu(pkg, torch, w.logits, params, w.hist, w.u, debug_cap=64)
    assert ids.min() >= 0 and ids.max() < w.V
    bid, bval, bcnt = w.bias_arrays()
    plist = [O.make_params(**r.as_kwargs()) for r in w.rows]
    H = w.hist.shape[1]
    hist = w.hist if H else None
    hl = np.full(w.B, H)
    cap = dbg["cand_ids"].shape[1]
    oc, rc, oci, ocp = O.sample_batch(plist, w.logits, hist, hl, bid, bval, bcnt, w.u, O.EXPF_CR,
                                      nthreads=8, want_res=True, cand_cap=cap)
    ol, rl = O.sample_batch(plist, w.logits, hist, hl, bid, bval, bcnt, w.u, O.EXPF_LIBM,
                            nthreads=8, want_res=True)
    say(f"[workload_parity] {name}: oracle done for {w.B} rows in both exp modes")
    # (1) correctly rounded exp: every row bit-exact (id, n, total, and the
    # first min(n, 64) kept candidates' ids and probabilities)
    bad = np.nonzero(ids != oc)[0]
    assert bad.size == 0, (name, bad[:10].tolist())
    # the same call without candidate lists (the launches a caller's call
    # makes: with full-sort rows the grouped rows in a launch of their own,
    # then the rows it leaves)
    ids_plain, _ = run_gpu(pkg, torch, w.logits, params, w.hist, w.u)
    bad = np.nonzero(ids_plain != oc)[0]
    assert bad.size == 0, (name, "without candidate lists", bad[:10].tolist())
    cand_rows = 0
    for b in range(w.B):
        r = rc[b]
        if r.greedy:
            continue
        assert int(dbg["n"][b]) == r.n, (name, b, int(dbg["n"][b]), r.n)
        assert dbg["total"][b].view(np.uint32) == np.float32(r.total).view(np.uint32), (name, b)
        m = min(int(r.n), cap)
        assert np.array_equal(dbg["cand_ids"][b, :m].astype(np.int64), oci[b, :m]), (name, b)
        assert np.array_equal(dbg["cand_probs"][b, :m].view(np.uint32), ocp[b, :m].view(np.uint32)), (
            name, b)
        cand_rows += 1
    # (2) the C library's expf: differing rows lie in the 1e-6 window
    counts = {"E1_draw": 0, "E2_topp": 0, "E3_minp": 0}
    for b in range(w.B):
        for c in exception_classes(rl[b]):
            counts[c] += 1
    differ = np.nonzero(ids != ol)[0]
    for b in differ:
        cls = exception_classes(rl[b])
        assert cls, (name, int(b), "differs from the libm-exp oracle outside the 1e-6 window",
                     rl[b].margin_draw, rl[b].margin_topp, rl[b].margin_minp)
    oracle_flips = int(np.sum(oc != ol))
    paths = np.bincount(dbg["path"], minlength=5).tolist()
    record = {"rows": int(w.B), "rows_bit_exact_cr_exp": int(w.B - bad.size),
              "rows_candidates_compared": cand_rows,
              "rows_differing_from_libm_exp": int(differ.size),
              "rows_where_oracle_cr_and_libm_differ_E4": oracle_flips,
              "rows_in_window": counts, "paths_greedy_topk_full_generic": paths[1:]}
    write_report(name, record)
    say(f"[workload_parity] {name}: {record}")
    # full-sort rows (k = 0) take the grouped sort path: their distinct values,
    # patched ids and cutoffs all fit its tables on these workloads
    full = np.array([r.temperature > 0 and not (0 < r.topK < w.V) for r in w.rows])
    if full.any():
        assert np.all(dbg["path"][full] == 3), (name, np.bincount(dbg["path"][full], minlength=5).tolist())


def test_device_rng_stream_and_greedy_rows_draw_nothing(pkg, torch):
    """u = NULL draws rand(1.0) from each row's own initRand(seed) stream, only
    on rows with temperature > 0 (sampler.nim:77-78,117)."""
    rng = np.random.default_rng(5)
    V, B, steps = 3000, 6, 4
    say(f"[device_rng] V={V} B={B} steps={steps}")
    seeds = [0, 1, 7, 1234, 99, 5]
    temps = [0.9, 0.0, 1.1, 0.7, 0.0, 1.0]
    plist = [dict(temperature=temps[b], topK=[0, 0, 30, 0, 0, 200][b], topP=0.9, minP=0.0,
                  repeatPenalty=1.0, repeatLastN=0, presencePenalty=0.0, frequencyPenalty=0.0,
                  seed=seeds[b]) for b in range(B)]
    s = pkg.BatchSampler([to_pkg_params(pkg, p, {}) for p in plist], V)
    streams = [list(O.uniforms(seeds[b], steps)) for b in range(B)]
    used = [0] * B
    try:
        for t in range(steps):
            x = rng.standard_normal((B, V)).astype(np.float32)
            out = s.sample(torch.from_numpy(x).cuda()).cpu().numpy()
            for b in range(B):
                u = streams[b][used[b]] if temps[b] > 0 else 0.0
                res, _, _, _ = oracle_row(x[b], plist[b], [], {}, u, O.EXPF_CR)
                assert out[b] == res.id, (t, b)
                if temps[b] > 0:
                    used[b] += 1
    finally:
        s.close()


def test_accept_loop_with_windows_and_growth(pkg, torch):
    """A generate-style loop: sample -> accept(id) on the device, with
    repeat_last_n windows and histories that outgrow the initial ring."""
    rng = np.random.default_rng(11)
    V, B, steps = 2000, 4, 40
    say(f"[accept_loop] V={V} B={B} steps={steps}")
    plist = [dict(temperature=0.8, topK=40, topP=0.95, minP=0.05, repeatPenalty=1.3,
                  repeatLastN=[0, 8, 0, 20][b], presencePenalty=0.2, frequencyPenalty=0.4,
                  seed=b) for b in range(B)]
    plist[2]["temperature"] = 0.0
    s = pkg.BatchSampler([to_pkg_params(pkg, p, {}) for p in plist], V)
    hist = [[] for _ in range(B)]
    pre = rng.integers(0, V, size=(B, 3)).astype(np.int64)
    s.accept(pre)
    for b in range(B):
        hist[b].extend(int(v) for v in pre[b])
    try:
        for t in range(steps):
            x = rng.standard_normal((B, V)).astype(np.float32) * 2
            u = rng.random(B)
            d_out = s.sample(torch.from_numpy(x).cuda(), torch.from_numpy(u).cuda())
            out = d_out.cpu().numpy()
            for b in range(B):
                res, _, _, _ = oracle_row(x[b], plist[b], hist[b], {}, float(u[b]), O.EXPF_CR)
                assert out[b] == res.id, (t, b)
                hist[b].append(int(out[b]))
            if t % 2 == 0:
                s.accept_device(d_out)
            else:
                s.accept(out.astype(np.int64))
    finally:
        s.close()


def test_batched_generate_loop_skips_end_of_generation(pkg, torch):
    """A batched generation loop over B chats (src/nimllm/chat.nim:204-208):
    every step each row samples with its own RNG stream; a row that draws an
    end-of-generation id ends its turn and accepts nothing (ACCEPT_SKIP /
    ACCEPT_SKIP32), and its next turn continues with the same history and RNG
    (Chat.sampler persists across turns, chat.nim:266,401).  Checked step by
    step against one oracle per row; histories outgrow the ring while the
    device-side skips leave the host's lengths inexact."""
    rng = np.random.default_rng(21)
    V, B, steps = 3000, 6, 48
    eog = (0, 1, 2)
    say(f"[batched_generate] V={V} B={B} steps={steps} eog={eog}")
    plist = [dict(temperature=0.8, topK=40, topP=0.95, minP=0.05, repeatPenalty=1.2,
                  repeatLastN=[0, 8, 0, 24, 0, 0][b], presencePenalty=0.3, frequencyPenalty=0.5,
                  seed=100 + b) for b in range(B)]
    plist[2]["temperature"] = 0.0          # greedy: draws nothing
    plist[4].update(topK=0, topP=0.9)      # full-sort path
    plist[5].update(topK=500)              # block top-k path
    s = pkg.BatchSampler([to_pkg_params(pkg, p, {}) for p in plist], V)
    streams = [list(O.uniforms(plist[b]["seed"], steps)) for b in range(B)]
    used = [0] * B
    hist = [[] for _ in range(B)]
    skipped = 0
    try:
        for t in range(steps):
            x = rng.standard_normal((B, V)).astype(np.float32) * 2
            # some rows are pushed towards an end-of-generation id this step
            for b in range(B):
                if rng.random() < 0.3:
                    x[b, eog[int(rng.integers(0, len(eog)))]] += 12.0
            d_out = s.sample(torch.from_numpy(x).cuda())
            out = d_out.cpu().numpy()
            for b in range(B):
                greedy = plist[b]["temperature"] <= 0
                u = 0.0 if greedy else streams[b][used[b]]
                res, _, _, _ = oracle_row(x[b], plist[b], hist[b], {}, u, O.EXPF_CR)
                assert out[b] == res.id, (t, b, int(out[b]), res.id)
                if not greedy:
                    used[b] += 1
            ended = np.isin(out, eog)
            skipped += int(ended.sum())
            if t % 2 == 0:
                d_acc = d_out.clone()
                d_acc[torch.from_numpy(ended).cuda()] = pkg.ACCEPT_SKIP32
                s.accept_device(d_acc)
            else:
                a = out.astype(np.int64)
                a[ended] = pkg.ACCEPT_SKIP
                s.accept(a)
            for b in range(B):
                if not ended[b]:
                    hist[b].append(int(out[b]))
        # RNG states advanced exactly once per non-greedy call
        for b in range(B):
            r = O.Rand()
            O.lib().nlo_init_rand(O.ctypes.byref(r), plist[b]["seed"])
            for _ in range(used[b]):
                O.lib().nlo_rand_float(O.ctypes.byref(r), 1.0)
            assert s.rng_state(b) == (r.a0, r.a1), b
    finally:
        s.close()
    say(f"[batched_generate] {skipped} row-steps ended a turn and accepted nothing")
    assert skipped > 0


def test_generate_step_batched_contexts(pkg, torch):
    """nls_generate_step: several contexts' decode loops in one handle, one
    row each (chat.nim:204-208 per row): rows sample with their own RNG
    streams (u = NULL), a row drawing an end-of-generation id finishes without
    accepting it, finished rows sample nothing (-1) and keep their RNG;
    checked step by step against per-row oracle loops."""
    rng = np.random.default_rng(404)
    V, B, steps = 3000, 6, 30
    eog = [7, 11, V - 1]
    say(f"[generate_step] V={V} B={B} steps={steps}")
    plist = [dict(temperature=[0.9, 0.0, 1.1, 0.7, 1.0, 0.8][b], topK=[40, 0, 0, 300, 5, 0][b],
                  topP=[0.95, 1.0, 0.9, 1.0, 1.0, 0.8][b], minP=[0.0, 0.0, 0.05, 0.0, 0.0, 0.1][b],
                  repeatPenalty=1.3, repeatLastN=[0, 8, 16, 0, 4, 0][b], presencePenalty=0.2,
                  frequencyPenalty=0.4, seed=[3, 0, 17, 99, 5, 2024][b]) for b in range(B)]
    s = pkg.BatchSampler([to_pkg_params(pkg, p, {}) for p in plist], V)
    streams = [list(O.uniforms(plist[b]["seed"], steps)) for b in range(B)]
    used = [0] * B
    hist = [[] for _ in range(B)]
    done = [False] * B
    d_done = torch.zeros(B, dtype=torch.int32, device="cuda")
    d_eog = torch.tensor(eog, dtype=torch.int32, device="cuda")
    try:
        for t in range(steps):
            x = (rng.standard_normal((B, V)) * 2.0).astype(np.float32)
            # make end-of-generation ids likely on some rows at some steps
            if t % 7 == 3:
                x[t % B, eog[t % 3]] += 12.0
            out = s.generate_step(torch.from_numpy(x).cuda(), d_eog, d_done).cpu().numpy()
            got_done = d_done.cpu().numpy()
            for b in range(B):
                if done[b]:
                    assert out[b] == -1, (t, b, int(out[b]))
                    continue
                u = 0.0
                if plist[b]["temperature"] > 0:
                    u = streams[b][used[b]]
                    used[b] += 1
                res, _, _, _ = oracle_row(x[b], plist[b], hist[b], {}, u, O.EXPF_CR)
                assert out[b] == res.id, (t, b, int(out[b]), res.id)
                if res.id in eog:
                    done[b] = True
                else:
                    hist[b].append(res.id)
            assert [bool(v) for v in got_done] == done, (t, got_done, done)
        assert any(done) and not all(done), done  # both kinds of rows were exercised
    finally:
        s.close()


def test_split_calls_around_an_inline_call(pkg, torch):
    """Top-k rows (sampler.nim:85-121) whose penalty windows overflow the
    streaming kernel's table: such a call hands every row to the whole-row
    launches (the first lists the rows it leaves for the second); after
    clear_history the next call is served by the streaming kernel alone, and
    after a long window again the call after it splits once more, on the same
    counter set as the first.  Four calls, each against the oracle."""
    rng = np.random.default_rng(77)
    B, V, H, distinct = 12, 50000, 6000, 4500
    say(f"[split_inline_split] B={B} V={V} H={H}")
    plist = [dict(temperature=1.0, topK=50, topP=0.95, minP=0.0, repeatPenalty=1.1, repeatLastN=0,
                  presencePenalty=0.3, frequencyPenalty=0.5, seed=1) for _ in range(B)]
    params = [to_pkg_params(pkg, p, {}) for p in plist]
    s = pkg.BatchSampler(params, V)

    def long_hist():
        h = np.empty((B, H), dtype=np.int64)
        for b in range(B):
            ids = rng.choice(V, distinct, replace=False)
            h[b] = np.concatenate([ids, ids[:H - distinct]])[rng.permutation(H)]
        return h

    try:
        for call, hist in enumerate([long_hist(), None, long_hist(), "same"]):
            if hist is None:
                s.clear_history()
                hl = [[] for _ in range(B)]
            elif isinstance(hist, np.ndarray):
                s.clear_history()
                s.accept(hist)
                hl = [list(r) for r in hist]
            x = (rng.standard_normal((B, V)) * 2.5).astype(np.float32)
            u = rng.random(B)
            ids = s.sample(torch.from_numpy(x).cuda(), torch.from_numpy(u).cuda()).cpu().numpy()
            torch.cuda.synchronize()
            say(f"[split_inline_split] call {call}")
            compare_rows(x, plist, hl, [{}] * B, u, ids, None, f"call {call}")
    finally:
        s.close()


def test_generate_step_full_sort_rows_split(pkg, torch):
    """nls_generate_step over a batch of full-sort rows only (the rows split
    over slices, sampler.nim:96-121): rows draw from their own RNG streams,
    which must advance once per step whether the slices finish the row or hand
    it on (a flat row every step: more values near its maximum than the slices
    keep); a row drawing an end-of-generation id finishes and samples nothing
    after; step by step against per-row oracle loops."""
    rng = np.random.default_rng(505)
    V, B, steps = 20000, 8, 25
    eog = [5, 9, V - 2]
    say(f"[generate_step_split] V={V} B={B} steps={steps}")
    plist = [dict(temperature=[0.7, 1.0, 0.9, 1.2, 0.6, 1.0, 0.8, 1.1][b], topK=0,
                  topP=[0.9, 1.0, 0.95, 1.0, 0.8, 1.0, 0.5, 1.0][b], minP=[0.05, 0.0, 0.0, 0.0, 0.1, 0.2, 0.0, 0.0][b],
                  repeatPenalty=1.2, repeatLastN=[0, 8, 16, 0, 4, 0, 32, 2][b], presencePenalty=0.3,
                  frequencyPenalty=0.2, seed=[7, 8, 9, 10, 11, 12, 13, 14][b]) for b in range(B)]
    s = pkg.BatchSampler([to_pkg_params(pkg, p, {}) for p in plist], V)
    streams = [list(O.uniforms(plist[b]["seed"], steps)) for b in range(B)]
    used = [0] * B
    hist = [[] for _ in range(B)]
    done = [False] * B
    d_done = torch.zeros(B, dtype=torch.int32, device="cuda")
    d_eog = torch.tensor(eog, dtype=torch.int32, device="cuda")
    try:
        assert s.plan()[0].floor_slices == 2
        for t in range(steps):
            x = rng.standard_normal((B, V)).astype(np.float32)
            for b in range(B):
                if b == 3:
                    x[b] *= np.float32(0.2)  # flat: handed on
                else:
                    x[b] += (-4.4 * np.log(1 + rng.permutation(V))).astype(np.float32)
            if t % 6 == 4:
                x[t % B, eog[t % 3]] = x[t % B].max() + 8.0
            out = s.generate_step(torch.from_numpy(x).cuda(), d_eog, d_done).cpu().numpy()
            got_done = d_done.cpu().numpy()
            for b in range(B):
                if done[b]:
                    assert out[b] == -1, (t, b, int(out[b]))
                    continue
                u = streams[b][used[b]]
                used[b] += 1
                res, _, _, _ = oracle_row(x[b], plist[b], hist[b], {}, u, O.EXPF_CR)
                assert out[b] == res.id, (t, b, int(out[b]), res.id)
                if res.id in eog:
                    done[b] = True
                else:
                    hist[b].append(res.id)
            assert [bool(v) for v in got_done] == done, (t, got_done, done)
        assert any(done) and not all(done), done
    finally:
        s.close()


def test_nim_binding_call_sequence(pkg, torch):
    """tests/nim_binding_check.c makes exactly the calls of the Nim binding of the
    sampler (create, set the RNG state from the Nim Rand, replay the
    history, then sample_host / accept per step, skipping accept on an
    end-of-generation id) and checks every id against the oracle."""
    import os
    import subprocess

    exe = os.path.join(os.path.dirname(__file__), "nim_binding_check.bin")
    assert os.path.exists(exe), "build it first: python -c 'import __graft_entry__ as g; g.build()'"
    say("[nim_binding] running tests/nim_binding_check.bin")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    say(r.stdout[-2000:])
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert "nim binding sequence ok" in r.stdout


def test_sample_host_and_single_row_sampler(pkg, torch):
    rng = np.random.default_rng(3)
    V = 5000
    say(f"[sample_host] V={V}")
    p = pkg.SamplerParams(temperature=0.7, topK=40, topP=0.95, minP=0.05, repeatPenalty=1.1,
                          repeatLastN=64, seed=42)
    s = pkg.newSampler(p, vocab=V)
    u = O.uniforms(42, 5)
    hist = []
    for t in range(5):
        x = rng.standard_normal(V).astype(np.float32) * 3
        got = s.sample(x)
        res, _, _, _ = oracle_row(x, dict(temperature=0.7, topK=40, topP=0.95, minP=0.05,
                                          repeatPenalty=1.1, repeatLastN=64, presencePenalty=0.0,
                                          frequencyPenalty=0.0, seed=42), hist, {}, float(u[t]),
                                  O.EXPF_CR)
        assert got == res.id
        s.accept(got)
        hist.append(got)


@pytest.mark.parametrize("B,V", [(3, 50000), (40, 128256)])
def test_sample_host_batches_both_sides_of_the_direct_limit(pkg, torch, B, V):
    """nls_sample_host on batches whose logits the kernel reads from the pinned
    staging directly (3 x 50000: 0.6 MB) and ones copied to device memory
    first (40 x 128256: 20.5 MB, above 8 MiB), three calls in a row on one
    handle, every id against the oracle with the rows' own RNG streams."""
    rng = np.random.default_rng(B)
    say(f"[sample_host_batches] B={B} V={V}")
    plist = [dict(temperature=0.8, topK=[40, 0, 300, 1][b % 4], topP=0.95, minP=0.0, repeatPenalty=1.0,
                  repeatLastN=0, presencePenalty=0.0, frequencyPenalty=0.0, seed=100 + b) for b in range(B)]
    s = pkg.BatchSampler([to_pkg_params(pkg, p, {}) for p in plist], V)
    try:
        us = [O.uniforms(100 + b, 3) for b in range(B)]
        for call in range(3):
            x = (rng.standard_normal((B, V)) * 2.5).astype(np.float32)
            got = s.sample_host(x)
            want = O.sample_batch([O.make_params(**p) for p in plist], x, None, None, None, None, None,
                                  np.array([us[b][call] for b in range(B)]), O.EXPF_CR, nthreads=8)
            assert np.array_equal(got, want), (B, V, call, np.flatnonzero(got != want)[:8])
    finally:
        s.close()


def test_expf_exhaustive_checksum(pkg, torch):
    """Every binary32 input in (-104, 89) through the device exp; the order-free
    checksum must equal the one of the correctly rounded results computed on
    the host (nls_expf_scan verify)."""
    say("[expf_exhaustive] 2.24e9 inputs")
    M = (1 << 64) - 1

    def s64(c):
        return c - (1 << 64) if c >= (1 << 63) else c

    g, c1, c2 = s64(0x9E3779B97F4A7C15), s64(0xBF58476D1CE4E5B9), s64(0x94D049BB133111EB)

    def lsr(z, k):
        return (z >> k) & ((1 << (64 - k)) - 1)

    neg_end, pos_end = 0xC2D00000, 0x42B20000
    ranges = [(0x80000000, neg_end), (0, pos_end)]
    total = torch.zeros((), dtype=torch.int64, device="cuda")
    step = 1 << 27
    for lo, hi in ranges:
        for a in range(lo, hi, step):
            b = min(hi, a + step)
            bits = torch.arange(a, b, dtype=torch.int64, device="cuda")
            x = bits.to(torch.int32).view(torch.float32) if lo == 0 else \
                (bits - (1 << 32)).to(torch.int32).view(torch.float32)
            y = pkg.expf_device(x.contiguous())
            yb = y.view(torch.int32).to(torch.int64) & 0xFFFFFFFF
            z = (bits << 32) | yb
            z = z + g
            z = (z ^ lsr(z, 30)) * c1
            z = (z ^ lsr(z, 27)) * c2
            z = z ^ lsr(z, 31)
            total += z.sum()
    got = int(total.item()) & M
    assert got == 0xB06E5AA31AE210E1, hex(got)


def _oracle_top_tokens(x, n):
    x = np.ascontiguousarray(x, dtype=np.float32)
    m = min(n, x.size)
    ids = np.zeros(max(m, 1), dtype=np.int64)
    pr = np.zeros(max(m, 1), dtype=np.float32)
    got = O.lib().nlo_top_tokens(x.ctypes.data_as(O.ctypes.POINTER(O.ctypes.c_float)), x.size, n,
                                 O.EXPF_CR, ids.ctypes.data_as(O.ctypes.POINTER(O.ctypes.c_int64)),
                                 pr.ctypes.data_as(O.ctypes.POINTER(O.ctypes.c_float)))
    return ids[:got], pr[:got]


def test_top_tokens_parity(pkg, torch):
    """topTokens (sampler.nim:123-130) on the device: ids and probabilities
    bit-identical to the oracle, including probabilities that tie although
    their logits differ (ordered by id), -inf entries, n beyond V and n at the
    2048 cap."""
    rng = np.random.default_rng(11)
    cases = [("normal 128256", rng.normal(0, 2.5, (4, 128256)).astype(np.float32), (5, 50, 2048)),
             ("quarter steps", (np.round(rng.normal(0, 2, (3, 32000)) * 4) / 4).astype(np.float32),
              (1, 100, 700))]
    col = rng.normal(-6, 1, (2, 4096)).astype(np.float32)
    col[:, [3, 10, 400, 999]] = np.array([-2.5e-8, -1e-8, 0.0, -2e-8], np.float32)
    cases.append(("probabilities tied by rounding", col, (4, 9)))
    neg = rng.normal(0, 1, (2, 5000)).astype(np.float32)
    neg[:, ::2] = -np.inf
    cases.append(("every other -inf", neg, (10,)))
    cases.append(("all equal", np.full((1, 1000), 0.75, np.float32), (7,)))
    cases.append(("V below n", rng.normal(0, 1, (3, 10)).astype(np.float32), (20, 10, 1)))
    cases.append(("V = 1", np.array([[1.5]], np.float32), (5,)))
    for name, x, ns in cases:
        d = torch.from_numpy(np.ascontiguousarray(x)).cuda()
        for n in ns:
            say(f"topTokens {name}: rows={x.shape[0]} V={x.shape[1]} n={n}")
            ids, pr = pkg.top_tokens_device(d, n)
            torch.cuda.synchronize()
            ids, pr = ids.cpu().numpy(), pr.cpu().numpy()
            assert ids.shape == (x.shape[0], min(n, x.shape[1]))
            for r in range(x.shape[0]):
                wi, wp = _oracle_top_tokens(x[r], n)
                assert np.array_equal(ids[r], wi), (name, n, r, ids[r][:8], wi[:8])
                assert np.array_equal(pr[r].view(np.uint32), wp.view(np.uint32)), (name, n, r)
    # the reference's signature: one row in, (id, probability) pairs out
    x = cases[1][1][0]
    wi, wp = _oracle_top_tokens(x, 5)
    assert pkg.topTokens(x, 5) == [(int(i), float(p)) for i, p in zip(wi, wp)]
    with pytest.raises(pkg.SamplerError):
        pkg.top_tokens_device(torch.zeros((1, 5000), device="cuda"), 2049)


def _softmax_rows_input(rows, V, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((rows, V)) * rng.choice([0.5, 2.5, 8.0], size=(rows, 1))).astype(np.float32)
    if rows > 0:
        x[0] = (np.round(x[0] * 4) / 4).astype(np.float32)  # ties
    if rows > 1:
        x[1] = np.float32(1.75)  # equal logits
    if rows > 2 and V > 3:
        x[2, :: max(1, V // 7)] = -np.inf
        x[2, V // 2] = np.nan  # skipped by the maximum, NaN probabilities
    if rows > 3:
        x[3] *= np.float32(30.0)  # most exponentials underflow
    return x


@pytest.mark.parametrize("rows,V", [(4, 1), (8, 7), (16, 5001), (8, 32000), (64, 128256), (16, 151936)])
def test_softmax_rows_parity(pkg, torch, rows, V):
    """softmaxInPlace (sampler.nim:51-57) on the device: every probability of
    every row bit for bit against the oracle (correctly rounded exp), out of
    place and in place, on rows with ties, equal logits, -inf and NaN
    entries and a wide range."""
    x = _softmax_rows_input(rows, V, 900 + V)
    say(f"[softmax_rows] rows={rows} V={V}")
    d = torch.from_numpy(x).cuda()
    got = pkg.softmax_device(d)
    torch.cuda.synchronize()
    got = got.cpu().numpy()
    d2 = d.clone()
    pkg.softmax_device(d2, out=d2)
    torch.cuda.synchronize()
    inplace = d2.cpu().numpy()
    for r in range(rows):
        want = O.softmax(x[r])
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(got[r]), nan), (V, r)
        assert np.array_equal(got[r][~nan].view(np.uint32), want[~nan].view(np.uint32)), (V, r)
        assert np.array_equal(np.isnan(inplace[r]), nan), (V, r)
        assert np.array_equal(inplace[r][~nan].view(np.uint32), want[~nan].view(np.uint32)), (V, r)


@pytest.mark.parametrize("rows,V", [(16, 5001), (128, 128256)])
def test_log_prob_parity(pkg, torch, rows, V):
    """logProb's per-token term (nimllm-doc-en.md:1700-1707): p[target] bit
    for bit against the oracle, ln(float64(p)) within 2 ulps of the C
    library's log, and the continuation sum."""
    x = _softmax_rows_input(rows, V, 77 + V)
    rng = np.random.default_rng(V)
    t = rng.integers(0, V, size=rows).astype(np.int32)
    t[4] = int(np.argmax(x[4]))
    t[5] = int(np.argmin(x[5]))
    say(f"[log_prob] rows={rows} V={V}")
    prob, logp = pkg.log_prob_device(torch.from_numpy(x).cuda(), torch.from_numpy(t).cuda())
    torch.cuda.synchronize()
    prob, logp = prob.cpu().numpy(), logp.cpu().numpy()
    total = 0.0
    for r in range(rows):
        wp, wl = O.log_prob(x[r], int(t[r]))
        if wp != wp:
            assert prob[r] != prob[r] and logp[r] != logp[r], r
            continue
        assert prob[r].view(np.uint32) == wp.view(np.uint32), (r, prob[r], wp)
        if wl == -math.inf:
            assert logp[r] == -math.inf, r
        else:
            assert abs(logp[r] - wl) <= 2 * np.spacing(abs(wl)), (r, logp[r], wl)
            total += wl
    ok = [r for r in range(rows) if math.isfinite(O.log_prob(x[r], int(t[r]))[1])]
    got_sum = pkg.log_prob(torch.from_numpy(x[ok]).cuda(), torch.from_numpy(t[ok]).cuda())
    assert abs(got_sum - total) <= 1e-12 * max(1.0, abs(total)), (got_sum, total)


def test_row_nll_parity(pkg, torch):
    """perplexity's per-position term (src/nimllm/model.nim:578-583) on the
    device against the oracle's index-order float64 sum.  The device sums in a
    fixed tree order, so the bar is float64 rounding: relative 1e-12."""
    import math

    rng = np.random.default_rng(99)
    say("[row_nll] rows of 128256 and 32000")
    for B, V, scale in ((64, 128256, 2.5), (8, 32000, 3.0), (5, 7, 1.0)):
        x = (rng.standard_normal((B, V)) * scale).astype(np.float32)
        x[0] = np.round(x[0] * 4.0) / 4.0                 # ties
        if B > 2:
            x[1, rng.choice(V, min(V, 5), replace=False)] = -np.inf  # banned ids
            x[2, :] = 1.0                                  # flat row: ln(V)
        t = rng.integers(0, V, size=B).astype(np.int32)
        got = pkg.row_nll_device(torch.from_numpy(x).cuda(), torch.from_numpy(t)).cpu().numpy()
        for b in range(B):
            ref = O.row_nll(x[b], int(t[b]))
            if not math.isfinite(ref):  # a banned target: +inf on both sides
                assert got[b] == ref, (B, V, b, got[b], ref)
                continue
            assert abs(got[b] - ref) <= 1e-12 * max(1.0, abs(ref)), (B, V, b, got[b], ref)
        if B > 2:
            assert got[2] == math.log(V) or abs(got[2] - math.log(V)) <= 1e-15 * math.log(V)
    # a NaN logit makes the term NaN (the sum takes exp(NaN)); a bad target too
    x = rng.standard_normal((2, 1000)).astype(np.float32)
    x[0, 10] = np.nan
    t = np.array([3, 5000], np.int32)
    got = pkg.row_nll_device(torch.from_numpy(x).cuda(), torch.from_numpy(t)).cpu().numpy()
    assert math.isnan(got[0]) and math.isnan(got[1])


def test_argmax_parity(pkg, torch):
    """argmax (src/nimllm/sampler.nim:45-49) on the device against the
    oracle's nlo_argmax (pinned to numpy.argmax's first maximum): ties, -0 and
    +0, -inf, NaN at index 0 and elsewhere, rows of NaN only, one-element and
    empty rows, rows whose length is not a multiple of 4 (4-byte loads) and
    rows of the vocabularies the sampler serves (16-byte loads)."""
    import ctypes

    rng = np.random.default_rng(45)
    L = O.lib()
    P = ctypes.POINTER(ctypes.c_float)

    def ref(row):
        r = np.ascontiguousarray(row, dtype=np.float32)
        return int(L.nlo_argmax(r.ctypes.data_as(P), len(r))) if len(r) else 0

    for B, V in ((13, 1), (13, 7), (13, 1001), (16, 32000), (64, 128256), (8, 151936), (9, 40003)):
        say(f"[argmax] B={B} V={V}")
        x = (rng.standard_normal((B, V)) * 2).astype(np.float32)
        if V >= 7:
            x[0] = np.round(x[0])                          # ties everywhere
            x[1, :] = -np.inf                              # all -inf: 0
            x[2, 0] = np.nan                               # NaN at 0: 0
            x[3, rng.choice(V, 3, replace=False)] = np.nan  # NaN elsewhere: skipped
            x[4, :] = np.nan                               # NaN only: 0
            x[5, :] = 0.0
            x[5, V // 2] = -0.0                            # +0 and -0 tie: the first
            x[6, :] = -np.inf
            x[6, V - 1] = -1e30                            # the last element
            if B > 8:
                x[7, rng.choice(V, min(V, 20), replace=False)] = np.float32(50.0)  # equal maxima
                x[8, :] = np.float32(3.0)
                x[8, 0] = -np.inf                          # from -inf at 0 up
        got = pkg.argmax_device(torch.from_numpy(x).cuda()).cpu().numpy()
        want = np.array([ref(x[b]) for b in range(B)])
        assert np.array_equal(got, want), (B, V, np.flatnonzero(got != want)[:8])
    # an empty row answers 0, as the reference's loop never runs
    got = pkg.argmax_device(torch.zeros((3, 0), dtype=torch.float32, device="cuda")).cpu().numpy()
    assert got.tolist() == [0, 0, 0]
    # the host-sequence form
    assert pkg.argmax([1.0, 3.0, 3.0, -2.0]) == 1


@pytest.mark.parametrize("rows,V,off", [(6, 32000, 1), (6, 32000, 2), (5, 5003, 3), (3, 128256, 1)])
def test_row_entry_points_on_unaligned_rows(pkg, torch, rows, V, off):
    """topTokens, softmaxInPlace, logProb's term, perplexity's term and argmax
    (sampler.nim:45-57,123-130; model.nim:578-583) on rows whose logits start
    off a 16-byte boundary (the kernels' 4-byte load paths), every result
    against the oracle as in the aligned tests."""
    x = _softmax_rows_input(rows, V, 300 + V + off)
    rng = np.random.default_rng(off)
    t = rng.integers(0, V, size=rows).astype(np.int32)
    flat = torch.zeros(rows * V + off, dtype=torch.float32, device="cuda")
    flat[off:] = torch.from_numpy(x.reshape(-1)).cuda()
    d = flat[off:].view(rows, V)
    assert d.data_ptr() % 16 != 0
    say(f"[unaligned_rows] rows={rows} V={V} offset={off}")
    # topTokens (a row holding NaN has NaN probabilities, whose order the
    # reference's comparator leaves open: ids 0 .. m-1, as documented)
    for n in (1, 64, 700):
        ids, pr = pkg.top_tokens_device(d, n)
        ids, pr = ids.cpu().numpy(), pr.cpu().numpy()
        for r in range(rows):
            if np.isnan(x[r]).any():
                assert np.array_equal(ids[r], np.arange(min(n, V))), (n, r)
                continue
            wi, wp = _oracle_top_tokens(x[r], n)
            assert np.array_equal(ids[r], wi), (n, r)
            assert np.array_equal(pr[r].view(np.uint32), wp.view(np.uint32)), (n, r)
    # softmaxInPlace, out of place
    got = pkg.softmax_device(d).cpu().numpy()
    for r in range(rows):
        want = O.softmax(x[r])
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(got[r]), nan), r
        assert np.array_equal(got[r][~nan].view(np.uint32), want[~nan].view(np.uint32)), r
    # logProb's term
    prob, _ = pkg.log_prob_device(d, torch.from_numpy(t).cuda())
    prob = prob.cpu().numpy()
    for r in range(rows):
        wp, _ = O.log_prob(x[r], int(t[r]))
        assert (prob[r] != prob[r]) if wp != wp else prob[r].view(np.uint32) == wp.view(np.uint32), r
    # perplexity's term
    nll = pkg.row_nll_device(d, torch.from_numpy(t)).cpu().numpy()
    for r in range(rows):
        ref = O.row_nll(x[r], int(t[r]))
        if math.isfinite(ref):
            assert abs(nll[r] - ref) <= 1e-12 * max(1.0, abs(ref)), r
        else:
            assert nll[r] == ref or (math.isnan(ref) and math.isnan(nll[r])), r
    # argmax
    am = pkg.argmax_device(d).cpu().numpy()
    L = O.lib()
    for r in range(rows):
        row = np.ascontiguousarray(x[r])
        assert am[r] == L.nlo_argmax(row.ctypes.data_as(O.ctypes.POINTER(O.ctypes.c_float)), V), r


@pytest.mark.parametrize("name", ["k64_rows", "split_rows_tied", "block_path_tied", "whole_row_mix",
                                  "long_bias_lists", "drawn_2", "drawn_6_tied"])
def test_random_batches_own_rng_streams(pkg, torch, name):
    """The sweep's batches with u = NULL, three calls on one sampler: each
    sampling row draws rand(1.0) from its own initRand(seed) stream once per
    call and greedy rows draw nothing (sampler.nim:77-78,117), whichever
    kernel serves the row -- including rows one kernel hands on to another,
    which must not draw twice.  The history grows by each call's ids."""
    B, V, ks, off = SWEEP[name][:4]
    max_bias = SWEEP[name][4] if len(SWEEP[name]) > 4 else 8
    rng = np.random.default_rng(abs(sum(map(ord, name))) + 1)
    say(f"[rng_sweep] {name}: B={B} V={V}")
    plist, biases = [], []
    for b in range(B):
        p = rand_params(rng, V)
        if p["temperature"] > 0:
            p["topK"] = int(rng.choice(ks))
        p["seed"] = int(rng.integers(0, 1 << 40))
        plist.append(p)
        nb = int(rng.integers(0, min(V, max_bias) + 1))
        ids = rng.choice(V, size=nb, replace=False) if nb else []
        biases.append({int(i): float(rng.choice([-math.inf, -3.0, 0.5, 4.0])) for i in ids})
    hist = [list(rng.integers(-3, V + 3, size=32)) for _ in range(B)]
    streams = [list(O.uniforms(plist[b]["seed"], 3)) for b in range(B)]
    drawn = [0] * B
    s = pkg.BatchSampler([to_pkg_params(pkg, plist[b], biases[b]) for b in range(B)], V)
    try:
        s.accept(np.array(hist, dtype=np.int64))
        for call in range(3):
            x = (rng.standard_normal((B, V)) * 2.5).astype(np.float32)
            if "tied" in name:
                x = (np.round(x * 4.0) / 4.0).astype(np.float32)
            ids = s.sample(torch.from_numpy(x).cuda()).cpu().numpy()
            for b in range(B):
                greedy = plist[b]["temperature"] <= 0
                u = 0.5 if greedy else float(streams[b][drawn[b]])
                res, _, _, _ = oracle_row(x[b], plist[b], hist[b], biases[b], u, O.EXPF_CR)
                assert ids[b] == res.id, (name, call, b, int(ids[b]), res.id)
                drawn[b] += 0 if greedy else 1
                hist[b].append(int(ids[b]))
            s.accept(ids.astype(np.int64).reshape(B, 1))
    finally:
        s.close()


@pytest.mark.parametrize("B,V,ks", [(300, 50000, (0, 20, 64)), (40, 100000, (0, 1, 50)),
                                    (600, 30000, (65, 300)), (24, 70000, (0, 1000, 3000))])
def test_generate_step_every_path(pkg, torch, B, V, ks):
    """nls_generate_step over the planner's paths (one workgroup per row,
    split rows, the k > 64 block path, whole-row rows with the claiming
    grid): six steps of B contexts with random parameters on their own RNG
    streams, end-of-generation ids made likely on some rows, finished rows
    sampling nothing (-1) in every kernel, and every id against per-row
    oracle loops (chat.nim:204-208)."""
    rng = np.random.default_rng(B + V)
    steps = 6
    eog = [3, 17, V - 2]
    say(f"[generate_step_paths] B={B} V={V} k={ks}")
    plist = []
    for b in range(B):
        p = rand_params(rng, V)
        if p["temperature"] > 0:
            p["topK"] = int(rng.choice(ks))
        p["seed"] = int(rng.integers(0, 1 << 31))
        plist.append(p)
    streams = [list(O.uniforms(plist[b]["seed"], steps)) for b in range(B)]
    used = [0] * B
    hist = [[] for _ in range(B)]
    done = [False] * B
    s = pkg.BatchSampler([to_pkg_params(pkg, p, {}) for p in plist], V)
    d_done = torch.zeros(B, dtype=torch.int32, device="cuda")
    d_eog = torch.tensor(eog, dtype=torch.int32, device="cuda")
    try:
        for t in range(steps):
            x = (rng.standard_normal((B, V)) * 2.0).astype(np.float32)
            hot = rng.choice(B, size=max(1, B // 5), replace=False)
            x[hot, eog[t % 3]] += 15.0  # these rows likely end here
            out = s.generate_step(torch.from_numpy(x).cuda(), d_eog, d_done).cpu().numpy()
            got_done = d_done.cpu().numpy()
            for b in range(B):
                if done[b]:
                    assert out[b] == -1, (t, b, int(out[b]))
                    continue
                u = 0.0
                if plist[b]["temperature"] > 0:
                    u = streams[b][used[b]]
                    used[b] += 1
                res, _, _, _ = oracle_row(x[b], plist[b], hist[b], {}, u, O.EXPF_CR)
                assert out[b] == res.id, (t, b, int(out[b]), res.id)
                if res.id in eog:
                    done[b] = True
                else:
                    hist[b].append(res.id)
            assert [bool(v) for v in got_done] == done, t
        assert any(done) and not all(done)
    finally:
        s.close()
