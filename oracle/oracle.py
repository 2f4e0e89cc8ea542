"""ctypes binding of the CPU restatement (liboracle) -- TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this
module.  It loads ``oracle/libnls_oracle.so`` (built by ``oracle/Makefile``) and
exposes the restated sampler (src/nimllm/sampler.nim:59-121), argmax (:45-49),
softmaxInPlace (:51-57), topTokens (:123-130), Nim std/random, and the output
projection `matmul` (src/nimllm/model.nim:144-200) over the weight formats of
src/nimllm/quant.nim.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# NLS_ORACLE_LIB names another build of the same sources (the sanitizer build)
LIB_PATH = os.environ.get("NLS_ORACLE_LIB") or os.path.join(HERE, "libnls_oracle.so")

EXPF_LIBM = 0
EXPF_CR = 1


class Params(ctypes.Structure):
    _fields_ = [
        ("temperature", ctypes.c_double),
        ("topK", ctypes.c_int64),
        ("topP", ctypes.c_double),
        ("minP", ctypes.c_double),
        ("repeatPenalty", ctypes.c_double),
        ("repeatLastN", ctypes.c_int64),
        ("presencePenalty", ctypes.c_double),
        ("frequencyPenalty", ctypes.c_double),
        ("seed", ctypes.c_int64),
    ]


class Rand(ctypes.Structure):
    _fields_ = [("a0", ctypes.c_uint64), ("a1", ctypes.c_uint64)]


class Result(ctypes.Structure):
    _fields_ = [
        ("id", ctypes.c_int64),
        ("greedy", ctypes.c_int32),
        ("heap", ctypes.c_int32),
        ("ncand", ctypes.c_int64),
        ("n", ctypes.c_int64),
        ("pos", ctypes.c_int64),
        ("sum", ctypes.c_float),
        ("total", ctypes.c_float),
        ("r0", ctypes.c_float),
        ("thr", ctypes.c_float),
        ("margin_draw", ctypes.c_double),
        ("margin_topp", ctypes.c_double),
        ("margin_minp", ctypes.c_double),
    ]


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.POINTER
        L.nlo_init_rand.argtypes = [P(Rand), ctypes.c_int64]
        L.nlo_next.argtypes = [P(Rand)]
        L.nlo_next.restype = ctypes.c_uint64
        L.nlo_skip_random_numbers.argtypes = [P(Rand)]
        L.nlo_rand_float.argtypes = [P(Rand), ctypes.c_double]
        L.nlo_rand_float.restype = ctypes.c_double
        L.nlo_uniforms.argtypes = [ctypes.c_int64, ctypes.c_int64, P(ctypes.c_double)]
        L.nlo_expf_cr.argtypes = [ctypes.c_float]
        L.nlo_expf_cr.restype = ctypes.c_float
        L.nlo_expf.argtypes = [ctypes.c_float, ctypes.c_int]
        L.nlo_expf.restype = ctypes.c_float
        L.nlo_sample.argtypes = [
            P(Params), P(ctypes.c_float), ctypes.c_int64,
            P(ctypes.c_int64), ctypes.c_int64,
            P(ctypes.c_int64), P(ctypes.c_double), ctypes.c_int64,
            ctypes.c_double, ctypes.c_int, P(Result),
            P(ctypes.c_int64), P(ctypes.c_float), P(ctypes.c_float),
        ]
        L.nlo_sample.restype = ctypes.c_int64
        L.nlo_sample_batch.argtypes = [
            P(Params), P(ctypes.c_float), ctypes.c_int64, ctypes.c_int64,
            P(ctypes.c_int64), ctypes.c_int64, P(ctypes.c_int64),
            P(ctypes.c_int64), P(ctypes.c_double), ctypes.c_int64, P(ctypes.c_int64),
            P(ctypes.c_double), ctypes.c_int, P(ctypes.c_int64), ctypes.c_int,
        ]
        L.nlo_sample_batch_res.argtypes = L.nlo_sample_batch.argtypes[:-1] + [P(Result), ctypes.c_int]
        L.nlo_sample_batch_cand.argtypes = L.nlo_sample_batch.argtypes[:-1] + [
            P(Result), ctypes.c_int64, P(ctypes.c_int64), P(ctypes.c_float), ctypes.c_int]
        L.nlo_argmax.argtypes = [P(ctypes.c_float), ctypes.c_int64]
        L.nlo_argmax.restype = ctypes.c_int64
        L.nlo_softmax_inplace.argtypes = [P(ctypes.c_float), ctypes.c_int64, ctypes.c_int]
        L.nlo_top_tokens.argtypes = [P(ctypes.c_float), ctypes.c_int64, ctypes.c_int64,
                                     ctypes.c_int, P(ctypes.c_int64), P(ctypes.c_float)]
        L.nlo_top_tokens.restype = ctypes.c_int64
        L.nlo_row_nll.argtypes = [P(ctypes.c_float), ctypes.c_int64, ctypes.c_int64]
        L.nlo_row_nll.restype = ctypes.c_double
        L.nlo_log_prob.argtypes = [P(ctypes.c_float), ctypes.c_int64, ctypes.c_int64, ctypes.c_int,
                                   P(ctypes.c_float)]
        L.nlo_log_prob.restype = ctypes.c_double
        vp = ctypes.c_void_p
        L.nlo_block_size.argtypes = [ctypes.c_int32]
        L.nlo_block_size.restype = ctypes.c_int32
        L.nlo_type_size.argtypes = [ctypes.c_int32]
        L.nlo_type_size.restype = ctypes.c_int32
        L.nlo_row_bytes.argtypes = [ctypes.c_int32, ctypes.c_int64]
        L.nlo_row_bytes.restype = ctypes.c_int64
        L.nlo_half_to_float.argtypes = [ctypes.c_uint16]
        L.nlo_half_to_float.restype = ctypes.c_float
        L.nlo_dequant_row.argtypes = [ctypes.c_int32, vp, P(ctypes.c_float), ctypes.c_int64]
        L.nlo_dequant_row.restype = ctypes.c_int32
        L.nlo_dot_f32.argtypes = [P(ctypes.c_float), P(ctypes.c_float), ctypes.c_int64]
        L.nlo_dot_f32.restype = ctypes.c_float
        L.nlo_act_block_len.argtypes = [ctypes.c_int32]
        L.nlo_act_block_len.restype = ctypes.c_int32
        L.nlo_quantize_act.argtypes = [P(ctypes.c_float), ctypes.c_int64, ctypes.c_int32,
                                       P(ctypes.c_float), P(ctypes.c_int8), P(ctypes.c_int32)]
        L.nlo_dot_row_act.argtypes = [ctypes.c_int32, vp, P(ctypes.c_float), P(ctypes.c_int8),
                                      P(ctypes.c_int32), ctypes.c_int64, ctypes.c_int64]
        L.nlo_dot_row_act.restype = ctypes.c_float
        L.nlo_matmul_uses_act.argtypes = [ctypes.c_int32, ctypes.c_int64, ctypes.c_int32,
                                          ctypes.c_int32]
        L.nlo_matmul_uses_act.restype = ctypes.c_int32
        L.nlo_matmul.argtypes = [ctypes.c_int32, vp, ctypes.c_int64, ctypes.c_int64,
                                 P(ctypes.c_float), ctypes.c_int32, P(ctypes.c_float),
                                 ctypes.c_int32, P(ctypes.c_float), P(ctypes.c_float),
                                 ctypes.c_int32, ctypes.c_float, ctypes.c_int64, ctypes.c_int64]
        L.nlo_matmul.restype = ctypes.c_int32
        _lib = L
    return _lib


def _ptr(a, ct):
    if a is None:
        return None
    return a.ctypes.data_as(ctypes.POINTER(ct))


def make_params(**kw) -> Params:
    p = Params()
    for name, _ in Params._fields_:
        setattr(p, name, kw.get(name, 0))
    return p


def uniforms(seed: int, n: int) -> np.ndarray:
    out = np.zeros(n, dtype=np.float64)
    if n:
        lib().nlo_uniforms(seed, n, _ptr(out, ctypes.c_double))
    return out


def sample(params: Params, logits, history=(), bias=None, u=0.5,
           expf_mode=EXPF_LIBM, want_cand=True):
    """Run one restated `sample` call.  Returns (Result, cand, probs, final_logits)."""
    L = lib()
    x = np.ascontiguousarray(logits, dtype=np.float32)
    V = x.shape[0]
    h = np.ascontiguousarray(history, dtype=np.int64)
    bias = bias or {}
    bid = np.array(list(bias.keys()), dtype=np.int64)
    bval = np.array(list(bias.values()), dtype=np.float64)
    res = Result()
    cand = np.zeros(max(V, 1), dtype=np.int64) if want_cand else None
    probs = np.zeros(max(V, 1), dtype=np.float32) if want_cand else None
    fl = np.zeros(max(V, 1), dtype=np.float32) if want_cand else None
    L.nlo_sample(ctypes.byref(params), _ptr(x, ctypes.c_float), V,
                 _ptr(h, ctypes.c_int64) if h.size else None, h.size,
                 _ptr(bid, ctypes.c_int64) if bid.size else None,
                 _ptr(bval, ctypes.c_double) if bval.size else None, bid.size,
                 float(u), expf_mode, ctypes.byref(res),
                 _ptr(cand, ctypes.c_int64), _ptr(probs, ctypes.c_float), _ptr(fl, ctypes.c_float))
    if want_cand:
        nc = res.ncand
        return res, cand[:nc].copy(), probs[:nc].copy(), fl[:V].copy()
    return res, None, None, None


def sample_batch(params_list, logits, hist=None, hlen=None, bias_ids=None, bias_vals=None,
                 nb=None, u=None, expf_mode=EXPF_LIBM, nthreads=1, want_res=False, cand_cap=0):
    """Rows [B, V] through the restated sampler on `nthreads` threads.  Returns
    the ids, or (ids, list of Result) with want_res, or with cand_cap > 0
    (ids, list of Result, cand_ids [B, cand_cap], cand_probs [B, cand_cap]):
    each row's first cand_cap candidates in the order sampler.nim:85-100
    leaves them (-1 / 0 past the row's candidate count)."""
    L = lib()
    x = np.ascontiguousarray(logits, dtype=np.float32)
    B, V = x.shape
    parr = (Params * B)(*params_list)
    H = 0 if hist is None else hist.shape[1]
    NB = 0 if bias_ids is None else bias_ids.shape[1]
    hist64 = None if hist is None else np.ascontiguousarray(hist, dtype=np.int64)
    hlen64 = None if hlen is None else np.ascontiguousarray(hlen, dtype=np.int64)
    bid = None if bias_ids is None else np.ascontiguousarray(bias_ids, dtype=np.int64)
    bv = None if bias_vals is None else np.ascontiguousarray(bias_vals, dtype=np.float64)
    nb64 = None if nb is None else np.ascontiguousarray(nb, dtype=np.int64)
    uu = np.ascontiguousarray(u, dtype=np.float64)
    out = np.zeros(B, dtype=np.int64)
    args = (parr, _ptr(x, ctypes.c_float), B, V,
            _ptr(hist64, ctypes.c_int64), H, _ptr(hlen64, ctypes.c_int64),
            _ptr(bid, ctypes.c_int64), _ptr(bv, ctypes.c_double), NB,
            _ptr(nb64, ctypes.c_int64), _ptr(uu, ctypes.c_double), expf_mode,
            _ptr(out, ctypes.c_int64))
    if not want_res:
        L.nlo_sample_batch(*args, nthreads)
        return out
    res = (Result * max(B, 1))()
    if cand_cap > 0:
        ci = np.zeros((B, cand_cap), dtype=np.int64)
        cp = np.zeros((B, cand_cap), dtype=np.float32)
        L.nlo_sample_batch_cand(*args, res, cand_cap, _ptr(ci, ctypes.c_int64),
                                _ptr(cp, ctypes.c_float), nthreads)
        return out, [res[i] for i in range(B)], ci, cp
    L.nlo_sample_batch_res(*args, res, nthreads)
    return out, [res[i] for i in range(B)]


def softmax(x, expf_mode=EXPF_CR):
    """softmaxInPlace (src/nimllm/sampler.nim:51-57) of a copy of x."""
    import numpy as np
    y = np.array(x, dtype=np.float32, copy=True)
    lib().nlo_softmax_inplace(y.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), y.size, expf_mode)
    return y


def log_prob(x, target, expf_mode=EXPF_CR):
    """logProb's per-token term (nimllm-doc-en.md:1700-1707): (p[target] as
    float32, ln(float64(p[target]))) with p = softmaxInPlace(x)."""
    import numpy as np
    x = np.ascontiguousarray(x, dtype=np.float32)
    p = ctypes.c_float()
    lp = lib().nlo_log_prob(x.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), len(x), int(target),
                            expf_mode, ctypes.byref(p))
    return np.float32(p.value), lp


def row_nll(x, target):
    """perplexity's per-position term (src/nimllm/model.nim:578-583)."""
    import numpy as np
    x = np.ascontiguousarray(x, dtype=np.float32)
    return lib().nlo_row_nll(x.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), len(x), int(target))


# --- output projection (src/nimllm/quant.nim, src/nimllm/model.nim:144-200) ---

GGML = {"F32": 0, "F16": 1, "Q4_0": 2, "Q4_1": 3, "Q5_0": 6, "Q5_1": 7, "Q8_0": 8,
        "Q2_K": 10, "Q3_K": 11, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14, "Q8_K": 15, "BF16": 30}


def block_size(t: int) -> int:
    return lib().nlo_block_size(t)


def type_size(t: int) -> int:
    return lib().nlo_type_size(t)


def row_bytes(t: int, n: int) -> int:
    return lib().nlo_row_bytes(t, n)


def half_to_float(h: int) -> np.float32:
    return np.float32(lib().nlo_half_to_float(h))


def dequant_row(t: int, raw, n: int) -> np.ndarray:
    """dequantRow (quant.nim:336-352) of one row of raw bytes."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    y = np.zeros(n, dtype=np.float32)
    if lib().nlo_dequant_row(t, raw.ctypes.data, _ptr(y, ctypes.c_float), n) != 0:
        raise ValueError(f"unsupported type {t}")
    return y


def dot_f32(a, b) -> np.float32:
    """dotF32 (quant.nim:362-374)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return np.float32(lib().nlo_dot_f32(_ptr(a, ctypes.c_float), _ptr(b, ctypes.c_float), a.size))


def act_block_len(t: int) -> int:
    return lib().nlo_act_block_len(t)


def quantize_act(x, block_len: int):
    """quantizeAct (quant.nim:646-667): (d, qs, bsums)."""
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    n = x.size
    d = np.zeros(n // block_len, dtype=np.float32)
    qs = np.zeros(n, dtype=np.int8)
    bs = np.zeros(max(n // 16, 1), dtype=np.int32)
    lib().nlo_quantize_act(_ptr(x, ctypes.c_float), n, block_len, _ptr(d, ctypes.c_float),
                           _ptr(qs, ctypes.c_int8), _ptr(bs, ctypes.c_int32))
    return d, qs, bs[: n // 16]


def dot_row_act(t: int, row, act, off: int, n: int) -> np.float32:
    """dotRowAct (quant.nim:788-798) of one raw row against quantize_act's output."""
    row = np.ascontiguousarray(row, dtype=np.uint8)
    d, qs, bs = act
    bs = np.ascontiguousarray(bs if bs.size else np.zeros(1, np.int32), dtype=np.int32)
    return np.float32(lib().nlo_dot_row_act(t, row.ctypes.data, _ptr(d, ctypes.c_float),
                                            _ptr(qs, ctypes.c_int8), _ptr(bs, ctypes.c_int32),
                                            off, n))


def matmul_uses_act(t: int, cols: int, nb: int, exact: bool = False) -> bool:
    return bool(lib().nlo_matmul_uses_act(t, cols, nb, int(exact)))


def matmul(t: int, w, rows: int, cols: int, x, exact: bool = False, lora=None,
           first: int = 0, last: int | None = None) -> np.ndarray:
    """matmul (model.nim:179-200): y[nb, rows] = x[nb, cols] . W^T for raw
    weight bytes w (rows x rowBytes).  lora = (a [rank, cols], b [rows, rank],
    scale).  With first/last only those rows are computed (the rest stay 0)."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, cols)
    nb = x.shape[0]
    last = rows if last is None else last
    y = np.zeros((nb, rows), dtype=np.float32)
    la = lb = None
    rank, scale = 0, 0.0
    if lora is not None:
        la = np.ascontiguousarray(lora[0], dtype=np.float32)
        lb = np.ascontiguousarray(lora[1], dtype=np.float32)
        rank, scale = la.shape[0], float(lora[2])
    rc = lib().nlo_matmul(t, w.ctypes.data, rows, cols, _ptr(x, ctypes.c_float), nb,
                          _ptr(y, ctypes.c_float), int(exact), _ptr(la, ctypes.c_float),
                          _ptr(lb, ctypes.c_float), rank, scale, first, last)
    if rc != 0:
        raise ValueError("unsupported type or shape")
    return y
