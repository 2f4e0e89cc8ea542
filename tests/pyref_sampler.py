"""Independent Python restatement of nimllm's sampler, used only to check the C oracle.

Built from library routines instead of the oracle's hand-written parts:
``collections.Counter`` for the CountTable (src/nimllm/sampler.nim:66-68),
``heapq`` for the HeapQueue (sampler.nim:88-95), ``sorted`` (stable) for
algorithm.sort (sampler.nim:97), numpy float32 scalars for every fp32 operation
and the C library ``expf`` through ctypes for ``exp(float32)`` (sampler.nim:56).
Slow (pure Python loops): use on small rows only.
"""
from __future__ import annotations

import ctypes
import ctypes.util
import heapq
import math
from collections import Counter
from dataclasses import dataclass, field

import numpy as np

_libm = ctypes.CDLL(ctypes.util.find_library("m"))
_libm.expf.restype = ctypes.c_float
_libm.expf.argtypes = [ctypes.c_float]
_libm.expl.restype = ctypes.c_longdouble
_libm.expl.argtypes = [ctypes.c_longdouble]

F32 = np.float32


def expf_libm(x: np.float32) -> np.float32:
    return F32(_libm.expf(float(x)))


def expf_cr(x: np.float32) -> np.float32:
    return F32(np.longdouble(_libm.expl(np.longdouble(float(x)))))


@dataclass
class Params:
    """SamplerParams (sampler.nim:11-21); every field set explicitly."""

    temperature: float = 0.0
    topK: int = 0
    topP: float = 0.0
    minP: float = 0.0
    repeatPenalty: float = 0.0
    repeatLastN: int = 0
    presencePenalty: float = 0.0
    frequencyPenalty: float = 0.0
    seed: int = 0
    logitBias: dict = field(default_factory=dict)


@dataclass
class Result:
    id: int
    greedy: bool
    cand: list
    probs: list  # float32 softmax probabilities in candidate order
    n: int
    final_logits: np.ndarray


def sample(p: Params, logits_in, history, u: float, cr: bool = False) -> Result:
    """One call of Sampler.sample (sampler.nim:59-121)."""
    ex = expf_cr if cr else expf_libm
    logits = [F32(v) for v in np.asarray(logits_in, dtype=np.float32)]
    V = len(logits)
    if len(history) > 0 and (p.repeatPenalty != 1.0 or p.presencePenalty != 0
                             or p.frequencyPenalty != 0):
        start = max(0, len(history) - p.repeatLastN) if p.repeatLastN > 0 else 0
        counts = Counter(history[start:])
        rp32 = F32(p.repeatPenalty)
        for tok, cnt in counts.items():
            if tok < 0 or tok >= V:
                continue
            if p.repeatPenalty != 1.0:
                if logits[tok] > 0:
                    logits[tok] = F32(logits[tok] / rp32)
                else:
                    logits[tok] = F32(logits[tok] * rp32)
            pen = float(cnt) * p.frequencyPenalty + p.presencePenalty
            logits[tok] = F32(logits[tok] - F32(pen))
    for tok, b in p.logitBias.items():
        if 0 <= tok < V:
            logits[tok] = F32(logits[tok] + F32(b))
    if p.temperature <= 0:
        best = 0
        for i in range(1, V):
            if logits[i] > logits[best]:
                best = i
        return Result(best, True, [], [], 0, np.array(logits, dtype=np.float32))
    invT = F32(1.0 / p.temperature)
    logits = [F32(v * invT) for v in logits]
    k = min(p.topK, V) if p.topK > 0 else V
    if k < V:
        # heapq on (value, index): Python compares floats with -0.0 == 0.0,
        # then the index, exactly as Nim's tuple `<` through `cmp`.
        h: list = []
        for i in range(V):
            if len(h) < k:
                heapq.heappush(h, (float(logits[i]), i))
            elif logits[i] > h[0][0]:
                heapq.heapreplace(h, (float(logits[i]), i))
        order = []
        while h:
            order.append(heapq.heappop(h)[1])
        idx = order[::-1]
    else:
        idx = sorted(range(V), key=lambda i: -float(logits[i]))
    probs = [logits[i] for i in idx]
    mx = F32(-np.inf)
    for v in probs:
        mx = v if mx <= v else mx
    s = F32(0.0)
    for j in range(len(probs)):
        probs[j] = ex(F32(probs[j] - mx))
        s = F32(s + probs[j])
    probs = [F32(v / s) for v in probs]
    n = len(probs)
    if 0 < p.topP < 1:
        cum = F32(0.0)
        for i in range(n):
            cum = F32(cum + probs[i])
            if float(cum) >= p.topP:
                n = i + 1
                break
    if p.minP > 0:
        thr = F32(probs[0] * F32(p.minP))
        m = 1
        while m < n and probs[m] >= thr:
            m += 1
        n = m
    total = F32(0.0)
    for i in range(n):
        total = F32(total + probs[i])
    r = F32(F32(u) * total)
    chosen = idx[n - 1]
    for i in range(n):
        r = F32(r - probs[i])
        if r <= 0:
            chosen = idx[i]
            break
    return Result(chosen, False, idx, probs, n, np.array(logits, dtype=np.float32))


def heap_rule(values, k):
    """Closed-form top-k membership and order of the reference's heap path.

    T = k-th largest value; G = {l > T}; m = k - |G|; p* = first index at which
    the running count of {l >= T} reaches k; members = G plus the m largest
    indices among {i <= p*: l_i = T}; order = descending (value, index).
    """
    vals = [float(v) for v in values]
    V = len(vals)
    srt = sorted(vals, reverse=True)
    T = srt[k - 1]
    G = [i for i in range(V) if vals[i] > T]
    m = k - len(G)
    cnt = 0
    pstar = V - 1
    for i in range(V):
        if vals[i] >= T:
            cnt += 1
            if cnt == k:
                pstar = i
                break
    ties = [i for i in range(pstar + 1) if vals[i] == T]
    members = G + ties[len(ties) - m:] if m > 0 else G
    return sorted(members, key=lambda i: (vals[i], i), reverse=True)


def nim_rand_next(state):
    """xoroshiro128+ step on a [a0, a1] list (Python ints); returns the output."""
    M = (1 << 64) - 1
    s0, s1 = state
    res = (s0 + s1) & M
    s1 ^= s0
    state[0] = (((s0 << 55) | (s0 >> 9)) & M) ^ s1 ^ ((s1 << 14) & M)
    state[1] = ((s1 << 36) | (s1 >> 28)) & M
    return res


def float_from_next(x: int) -> float:
    """rand(1.0) closed form: the top 52 bits of x as a fraction of 2^52."""
    return (x >> 12) / float(1 << 52)


def cr_exp(x: float) -> float:
    return math.exp(x)
