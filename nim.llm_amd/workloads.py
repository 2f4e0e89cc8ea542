"""Synthetic sampler workloads (seeded numpy), shared by bench.py and the tests.

Each workload is a batch of rows: fp32 logits [B, V], one SamplerParams per
row (every field set explicitly -- Nim zero-initialises omitted fields), the
rows' accepted-token histories and one uniform per row standing for
rand(1.0) (src/nimllm/sampler.nim:117), taken in row order from a single Nim
std/random stream (initRand(seed)).

Workloads (B x V):
  single_32k      1 x 32000    N(0, 3^2); T 0.8, top-k 40, top-p 0.95
  zipf_minp_128k  64 x 128256  N(0,1) + Zipf head -4.4 ln(rank); T 0.7, top-p 0.9,
                               min-p 0.05, repetition 1.1 over 256 uniform ids
  penalties_152k  256 x 151936 N(0, 2.5^2); frequency 0.5, presence 0.3 over 1024
                               Zipf(1.2) ids; 50 bias ids/row in [-5, 5], 5 at -inf;
                               top-k 50, top-p 0.95, T 1.0
  flat_topk1000   1024 x 128256 N(0,1); T 1.2, top-k 1000, top-p 0.99
  mixed_ties_152k 2048 x 151936 N(0, 2^2) rounded to 0.25; rows 25% greedy /
                               min-p 0.1 / top-k 20 / top-p 0.8; repetition 1.05
                               over 512 uniform ids
  headline        256 x 128256  the penalties_152k recipe at V = 128256
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

WORKLOADS = ("single_32k", "zipf_minp_128k", "penalties_152k", "flat_topk1000",
             "mixed_ties_152k", "headline")

SHAPES = {
    "single_32k": (1, 32000),
    "zipf_minp_128k": (64, 128256),
    "penalties_152k": (256, 151936),
    "flat_topk1000": (1024, 128256),
    "mixed_ties_152k": (2048, 151936),
    "headline": (256, 128256),
}


@dataclass
class RowSpec:
    temperature: float = 1.0
    topK: int = 0
    topP: float = 1.0
    minP: float = 0.0
    repeatPenalty: float = 1.0
    repeatLastN: int = 0
    presencePenalty: float = 0.0
    frequencyPenalty: float = 0.0
    seed: int = 1
    logitBias: dict = None

    def as_kwargs(self):
        d = dict(temperature=self.temperature, topK=self.topK, topP=self.topP, minP=self.minP,
                 repeatPenalty=self.repeatPenalty, repeatLastN=self.repeatLastN,
                 presencePenalty=self.presencePenalty, frequencyPenalty=self.frequencyPenalty,
                 seed=self.seed)
        return d


@dataclass
class Workload:
    name: str
    logits: np.ndarray   # float32 [B, V]
    rows: list           # RowSpec per row
    hist: np.ndarray     # int64 [B, H] (H may be 0)
    u: np.ndarray        # float64 [B]
    seed: int

    @property
    def B(self):
        return self.logits.shape[0]

    @property
    def V(self):
        return self.logits.shape[1]

    def bias_arrays(self):
        """(ids [B, NB] int64, vals [B, NB] float64, counts [B] int64)."""
        nb = max((len(r.logitBias or {}) for r in self.rows), default=0)
        ids = np.zeros((self.B, max(nb, 1)), dtype=np.int64)
        vals = np.zeros((self.B, max(nb, 1)), dtype=np.float64)
        cnt = np.zeros(self.B, dtype=np.int64)
        for b, r in enumerate(self.rows):
            d = r.logitBias or {}
            cnt[b] = len(d)
            for j, (k, v) in enumerate(d.items()):
                ids[b, j], vals[b, j] = k, v
        return ids, vals, cnt

    def row_bytes(self) -> list:
        """Bytes a perfect implementation must move for each row: logits read
        once, int32 history window, (int32 id + fp32 value) per bias entry, the
        float64 uniform and the int32 output id."""
        out = []
        for b, r in enumerate(self.rows):
            h = self.hist.shape[1] if (r.repeatPenalty != 1.0 or r.presencePenalty != 0 or
                                       r.frequencyPenalty != 0) else 0
            if r.repeatLastN > 0:
                h = min(h, r.repeatLastN)
            out.append(4 * self.V + 4 * h + 8 * len(r.logitBias or {}) + 8 + 4)
        return out

    def algorithmic_bytes(self) -> int:
        """Bytes a perfect implementation must move, summed over the rows."""
        return sum(self.row_bytes())


def nim_uniforms(seed: int, n: int) -> np.ndarray:
    """rand(1.0) x n from initRand(seed) -- std/random, restated in numpy-free
    Python so this module needs no compiled code."""
    M = (1 << 64) - 1

    def nxt(st):
        s0, s1 = st
        res = (s0 + s1) & M
        s1 ^= s0
        st[0] = (((s0 << 55) | (s0 >> 9)) & M) ^ s1 ^ ((s1 << 14) & M)
        st[1] = ((s1 << 36) | (s1 >> 28)) & M
        return res

    s = seed if seed != 0 else 2147483647
    st = [(s >> 16) & M, s & 0xFFFF]
    j0 = j1 = 0
    for w in (0xBEAC0467EBA5FACB, 0xD86B048B86AA9922):
        for b in range(64):
            if (w >> b) & 1:
                j0 ^= st[0]
                j1 ^= st[1]
            nxt(st)
    st = [j0, j1]
    nxt(st)
    out = np.empty(n, dtype=np.float64)
    for i in range(n):
        out[i] = (nxt(st) >> 12) / float(1 << 52)
    return out


def _zipf_ids(rng, n, V, a=1.2):
    perm = rng.permutation(V)
    z = rng.zipf(a, size=n)
    return perm[(z - 1) % V].astype(np.int64)


_PENALTY_ROWS = ("fp32 logits N(0, 2.5^2); frequency 0.5 / presence 0.3 over 1024 Zipf(1.2) history ids; "
                 "50 bias ids per row (5 at -inf); top-k 50, top-p 0.95, T 1.0")
DESCRIPTIONS = {
    "single_32k": "fp32 logits N(0, 3^2); top-k 40, top-p 0.95, T 0.8; no history, no bias",
    "zipf_minp_128k": ("fp32 logits N(0, 1) - 4.4 ln(rank), a random rank per id (Zipf head); "
                       "full sort (k = 0), top-p 0.9, min-p 0.05, T 0.7; repeat penalty 1.1 over "
                       "256 uniform history ids"),
    "penalties_152k": _PENALTY_ROWS,
    "headline": _PENALTY_ROWS,
    "flat_topk1000": "fp32 logits N(0, 1); top-k 1000, top-p 0.99, T 1.2; no history, no bias",
    "mixed_ties_152k": ("fp32 logits round(4 N(0, 8^2)) / 4 (heavy ties); each row at random greedy, "
                        "full sort with min-p 0.1, top-k 20, or full sort with top-p 0.8 (T 1.0); "
                        "repeat penalty 1.05 over 512 uniform history ids"),
}


def describe(name: str, B: int, V: int) -> str:
    """The workload's full description, as the benchmark reports it."""
    return f"{name}: B={B} x V={V} {DESCRIPTIONS[name]}"


def make(name: str, seed: int = 1234, B: int | None = None, V: int | None = None) -> Workload:
    B0, V0 = SHAPES[name]
    B = B0 if B is None else B
    V = V0 if V is None else V
    rng = np.random.default_rng(seed)
    rows = []
    hist = np.zeros((B, 0), dtype=np.int64)
    if name == "single_32k":
        x = (rng.standard_normal((B, V), dtype=np.float32) * np.float32(3.0))
        rows = [RowSpec(temperature=0.8, topK=40, topP=0.95) for _ in range(B)]
    elif name == "zipf_minp_128k":
        x = rng.standard_normal((B, V), dtype=np.float32)
        for b in range(B):
            rank = 1 + rng.permutation(V)
            x[b] += (-4.4 * np.log(rank)).astype(np.float32)
        rows = [RowSpec(temperature=0.7, topK=0, topP=0.9, minP=0.05, repeatPenalty=1.1,
                        repeatLastN=0) for _ in range(B)]
        hist = rng.integers(0, V, size=(B, 256), dtype=np.int64)
    elif name in ("penalties_152k", "headline"):
        x = rng.standard_normal((B, V), dtype=np.float32) * np.float32(2.5)
        hist = np.stack([_zipf_ids(rng, 1024, V) for _ in range(B)])
        for b in range(B):
            ids = rng.choice(V, size=50, replace=False)
            vals = rng.uniform(-5.0, 5.0, size=50)
            vals[:5] = -math.inf
            rows.append(RowSpec(temperature=1.0, topK=50, topP=0.95, repeatPenalty=1.0,
                                repeatLastN=0, presencePenalty=0.3, frequencyPenalty=0.5,
                                logitBias={int(i): float(v) for i, v in zip(ids, vals)}))
    elif name == "flat_topk1000":
        x = rng.standard_normal((B, V), dtype=np.float32)
        rows = [RowSpec(temperature=1.2, topK=1000, topP=0.99) for _ in range(B)]
    elif name == "mixed_ties_152k":
        x = (np.round(rng.standard_normal((B, V), dtype=np.float32) * np.float32(8.0))
             / np.float32(4.0)).astype(np.float32)
        modes = rng.integers(0, 4, size=B)
        for b in range(B):
            m = int(modes[b])
            if m == 0:
                r = RowSpec(temperature=0.0)
            elif m == 1:
                r = RowSpec(temperature=1.0, topK=0, minP=0.1)
            elif m == 2:
                r = RowSpec(temperature=1.0, topK=20)
            else:
                r = RowSpec(temperature=1.0, topK=0, topP=0.8)
            r.repeatPenalty = 1.05
            r.repeatLastN = 0
            rows.append(r)
        hist = rng.integers(0, V, size=(B, 512), dtype=np.int64)
    else:
        raise KeyError(name)
    u = nim_uniforms(seed, B)
    return Workload(name, np.ascontiguousarray(x, dtype=np.float32), rows, hist, u, seed)


def sampler_params(w: Workload, mod):
    """SamplerParams objects of package module `mod` for every row."""
    out = []
    for r in w.rows:
        p = mod.SamplerParams(**r.as_kwargs())
        p.logitBias = dict(r.logitBias or {})
        out.append(p)
    return out


# --- the output projection (LM head) -------------------------------------

# GGML type codes and their blocks (src/nimllm/quant.nim:14-63): code ->
# (weights per block, bytes per block, byte offsets of the fp16 scale fields)
LM_TYPES = {
    0: (1, 4, ()), 1: (1, 2, ()), 30: (1, 2, ()),
    2: (32, 18, (0,)), 3: (32, 20, (0, 2)), 6: (32, 22, (0,)), 7: (32, 24, (0, 2)), 8: (32, 34, (0,)),
    10: (256, 84, (80, 82)), 11: (256, 110, (108,)), 12: (256, 144, (0, 2)), 13: (256, 176, (0, 2)),
    14: (256, 210, (208,)), 15: (256, 292, ()),
}
LM_TYPE_NAMES = {"F32": 0, "F16": 1, "Q4_0": 2, "Q4_1": 3, "Q5_0": 6, "Q5_1": 7, "Q8_0": 8, "Q2_K": 10,
                 "Q3_K": 11, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14, "Q8_K": 15, "BF16": 30}


def lm_row_bytes(t: int, cols: int) -> int:
    bs, ts, _ = LM_TYPES[t]
    assert cols % bs == 0
    return cols // bs * ts


def make_lm_weights(t: int, rows: int, cols: int, seed: int = 1234) -> np.ndarray:
    """Synthetic GGUF weight rows [rows, rowBytes] of type t: random bytes
    (every bit pattern is a valid block), with the fp16 / fp32 scale fields
    set to finite values of the size a quantiser writes; F32 / F16 / BF16
    rows hold N(0, 0.5^2) weights."""
    rng = np.random.default_rng(seed)
    bs, ts, halves = LM_TYPES[t]
    rb = lm_row_bytes(t, cols)
    if bs == 1:
        v = (rng.standard_normal(size=(rows, cols), dtype=np.float32) * np.float32(0.5))
        if t == 0:
            return v.view(np.uint8).reshape(rows, rb)
        if t == 1:
            return v.astype(np.float16).view(np.uint8).reshape(rows, rb)
        return (v.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).reshape(rows, rb)
    raw = rng.integers(0, 256, size=(rows, rb), dtype=np.uint8)
    blocks = raw.reshape(rows, rb // ts, ts)
    if t == 15:
        d = rng.uniform(1e-3, 2e-2, size=blocks.shape[:2]).astype(np.float32)
        blocks[:, :, 0:4] = d.view(np.uint8).reshape(rows, rb // ts, 4)
    for off in halves:
        h = (rng.uniform(-1, 1, size=blocks.shape[:2]) *
             np.exp2(rng.integers(-12, -4, size=blocks.shape[:2]))).astype(np.float16)
        blocks[:, :, off:off + 2] = h.view(np.uint8).reshape(rows, rb // ts, 2)
    return raw


def make_lm_hidden(nb: int, cols: int, seed: int = 1234) -> np.ndarray:
    """Normalised hidden states [nb, cols] (rmsnorm output scale)."""
    rng = np.random.default_rng(seed + 1)
    return (rng.standard_normal(size=(nb, cols), dtype=np.float32) * np.float32(2.0))
