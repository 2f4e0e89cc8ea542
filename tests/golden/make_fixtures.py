"""Writes tests/golden/sampler_cases.json: small sampler cases with expected outputs.

The reference ships no sampler fixtures (its tests pin greedy decoding only,
tests/t_complet.nim:37-39), so these are generated here from the C restatement
of src/nimllm/sampler.nim:59-121 and accepted only where the independent Python
restatement (heapq / stable sorted / numpy float32 / libm expf) agrees bit for
bit.  Expected values are recorded for the correctly rounded exp (the sampler's
exp) and, separately, the id under the C library's expf.

    python tests/golden/make_fixtures.py
"""
import json
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "tests"))

import oracle as O  # noqa: E402
import pyref_sampler as R  # noqa: E402


def f32bits(a):
    return [int(v) for v in np.asarray(a, dtype=np.float32).view(np.uint32)]


def case(name, x, params, hist=(), bias=None, u=0.5):
    x = np.asarray(x, dtype=np.float32)
    bias = bias or {}
    out = {"name": name, "V": int(x.size), "logits_bits": f32bits(x), "params": params,
           "history": [int(h) for h in hist],
           "bias": [[int(k), (v if math.isfinite(v) else ("-inf" if v < 0 else "inf"))]
                    for k, v in bias.items()],
           "u": float(u)}
    for cr in (True, False):
        res, cand, probs, fl = O.sample(O.make_params(**params), x, list(hist), bias, u,
                                        O.EXPF_CR if cr else O.EXPF_LIBM)
        pr = R.sample(R.Params(logitBias=bias, **params), x, list(hist), u, cr=cr)
        assert res.id == pr.id, name
        if not pr.greedy:
            assert list(cand) == list(pr.cand), name
            assert np.array_equal(probs.view(np.uint32),
                                  np.array(pr.probs, dtype=np.float32).view(np.uint32)), name
            assert res.n == pr.n
        if cr:
            out["expect"] = {"id": int(res.id), "greedy": bool(res.greedy), "n": int(res.n),
                             "ncand": int(res.ncand),
                             "cand": [int(c) for c in cand[:max(res.n, 0)]],
                             "probs_bits": f32bits(probs[:max(res.n, 0)]),
                             "total_bits": f32bits([res.total])[0]}
        else:
            out["id_libm"] = int(res.id)
    return out


def P(**kw):
    base = dict(temperature=1.0, topK=0, topP=1.0, minP=0.0, repeatPenalty=1.0, repeatLastN=0,
                presencePenalty=0.0, frequencyPenalty=0.0, seed=0)
    base.update(kw)
    return base


def main():
    rng = np.random.default_rng(20261201)
    cases = []
    # greedy with ties (first index wins)
    cases.append(case("greedy_ties", [1, 3, 3, -2, 3, 0], P(temperature=0.0)))
    cases.append(case("greedy_neg_zero", [-1.0, -0.0, 0.0, -0.5], P(temperature=0.0)))
    # heap path: ties at the k boundary (documented example + wider)
    cases.append(case("heap_tie_example", [1, 2, 2, 2, 0.5], P(topK=2), u=0.9))
    x = (rng.integers(-3, 4, size=300) * 0.5).astype(np.float32)
    for k in (1, 7, 40, 299):
        for u in (0.0, 0.37, 0.999999):
            cases.append(case(f"heap_grid_k{k}_u{u}", x, P(topK=k, temperature=0.9), u=u))
    # sort path with ties and signed zeros
    xs = (rng.integers(-4, 5, size=257) * 0.25).astype(np.float32)
    xs[xs == 0] = -0.0
    for tp, mp in ((1.0, 0.0), (0.8, 0.0), (1.0, 0.1), (0.9, 0.05)):
        cases.append(case(f"sort_ties_p{tp}_minp{mp}", xs, P(topK=0, topP=tp, minP=mp), u=0.61))
    # -inf bias, bias on the max, out-of-range bias ids
    xb = rng.standard_normal(500).astype(np.float32) * 2
    top = int(np.argmax(xb))
    cases.append(case("bias_forbid_max", xb, P(topK=10),
                      bias={top: -math.inf, 3: 2.5, -4: 9.0, 500: 9.0}, u=0.2))
    cases.append(case("bias_greedy", xb, P(temperature=0.0), bias={top: -math.inf, 17: 1.0}))
    # repetition / frequency / presence penalties with repeats and a window
    hist = [int(h) for h in rng.integers(-2, 502, size=120)] + [top] * 5
    cases.append(case("penalties_all", xb, P(topK=50, topP=0.95, repeatPenalty=1.3,
                                             presencePenalty=0.3, frequencyPenalty=0.5),
                      hist=hist, u=0.44))
    cases.append(case("penalties_window", xb, P(topK=0, topP=0.9, minP=0.05, repeatPenalty=1.1,
                                                repeatLastN=16), hist=hist, u=0.73))
    cases.append(case("penalty_rp_zero", xb, P(topK=5, repeatPenalty=0.0), hist=hist, u=0.5))
    cases.append(case("penalties_greedy", xb, P(temperature=0.0, repeatPenalty=1.5), hist=hist))
    # top-p / min-p cutoffs on a peaked row, u at the ends
    xp = (rng.standard_normal(1000) * 4).astype(np.float32)
    for u in (0.0, 0.5, 0.9999999):
        cases.append(case(f"peaked_topp_minp_u{u}", xp, P(temperature=0.7, topP=0.5, minP=0.02),
                          u=u))
    cases.append(case("k_ge_V", xp[:64], P(topK=64, topP=0.95), u=0.3))
    cases.append(case("single_token", [0.25], P(topK=0), u=0.9))
    path = os.path.join(HERE, "sampler_cases.json")
    with open(path, "w") as f:
        json.dump({"source": "oracle/nls_oracle.c cross-checked with tests/pyref_sampler.py",
                   "cases": cases}, f, separators=(",", ":"))
    print(f"wrote {len(cases)} cases to {path}")


if __name__ == "__main__":
    main()
