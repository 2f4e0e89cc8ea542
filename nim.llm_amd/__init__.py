"""MI355X token sampler -- Python host mirror of nimllm's `Sampler` over the C ABI.

The compute lives in ``libnimllm_sampler.so`` (HIP kernels for gfx950, built from
``csrc/`` by ``csrc/Makefile``); this module only marshals arguments through
ctypes.  It mirrors src/nimllm/sampler.nim:

* ``SamplerParams`` (:11-21), ``defaultSampling`` (:28-31), ``greedySampling`` (:33-35)
* ``newSampler`` / ``Sampler.accept`` / ``Sampler.sample`` (:37-43, :59-121) for one
  row, and ``BatchSampler`` for B independent rows on the device.

There is no CPU fallback: without the built library or a GPU every entry
point raises.
"""
from __future__ import annotations

import ctypes
import math
import os
from dataclasses import dataclass, field
from typing import Optional, Sequence

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libnimllm_sampler.so")

NLS_OK = 0
PATH_GREEDY, PATH_TOPK, PATH_FULL, PATH_GENERIC = 1, 2, 3, 4
# accept entries that append nothing (a row that ended this step):
# NLS_ACCEPT_SKIP for host int64 ids, NLS_ACCEPT_SKIP32 for device int32 ids
ACCEPT_SKIP = -(1 << 63)
ACCEPT_SKIP32 = -(1 << 31)

EXPORTED = (
    "nls_default_sampling", "nls_greedy_sampling", "nls_create", "nls_destroy",
    "nls_set_stream", "nls_batch", "nls_vocab", "nls_accept", "nls_accept_row",
    "nls_accept_device", "nls_generate_step", "nls_clear_history", "nls_sample", "nls_sample_host",
    "nls_sample_host_noalloc",
    "nls_synchronize", "nls_rng_uniforms", "nls_get_rng_state", "nls_set_rng_state",
    "nls_top_tokens", "nls_row_nll", "nls_softmax_rows", "nls_log_prob", "nls_expf_device",
    "nls_profile_next",
    "nls_profile_next_generic", "nls_get_plan", "nls_status_string", "nls_last_error",
    "nls_lm_head_workspace", "nls_lm_head", "nls_lm_head_row_bytes", "nls_argmax",
)


class NlsLora(ctypes.Structure):
    """nls_lora: a LoRA adapter on the output matrix (LoraPair, model.nim:34-39)."""

    _fields_ = [("d_a", ctypes.c_void_p), ("d_b", ctypes.c_void_p), ("rank", ctypes.c_int32),
                ("scale", ctypes.c_float)]


class NlsParams(ctypes.Structure):
    _fields_ = [
        ("temperature", ctypes.c_double),
        ("top_k", ctypes.c_int64),
        ("top_p", ctypes.c_double),
        ("min_p", ctypes.c_double),
        ("repeat_penalty", ctypes.c_double),
        ("repeat_last_n", ctypes.c_int64),
        ("presence_penalty", ctypes.c_double),
        ("frequency_penalty", ctypes.c_double),
        ("seed", ctypes.c_int64),
        ("logit_bias_ids", ctypes.POINTER(ctypes.c_int64)),
        ("logit_bias_values", ctypes.POINTER(ctypes.c_double)),
        ("logit_bias_count", ctypes.c_int64),
    ]


class NlsDebug(ctypes.Structure):
    _fields_ = [
        ("n", ctypes.c_void_p),
        ("ncand", ctypes.c_void_p),
        ("cand_ids", ctypes.c_void_p),
        ("cand_probs", ctypes.c_void_p),
        ("total", ctypes.c_void_p),
        ("path", ctypes.c_void_p),
        ("cap", ctypes.c_int32),
    ]


class NlsPlan(ctypes.Structure):
    _fields_ = [
        ("stream_threads", ctypes.c_int32),
        ("slices", ctypes.c_int32),
        ("generic_launch", ctypes.c_int32),
        ("streamed_rows", ctypes.c_int32),
        ("first_unit_bytes", ctypes.c_int64),
        ("k64", ctypes.c_int32),
        ("walk_split", ctypes.c_int32),
        ("floor_slices", ctypes.c_int32),
    ]


class SamplerError(RuntimeError):
    pass


_lib = None


def lib():
    """Load the HIP library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise SamplerError(f"{LIB_PATH} is missing: build it with `make -C {HERE}/csrc`")
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.POINTER
        vp = ctypes.c_void_p
        L.nls_default_sampling.restype = NlsParams
        L.nls_greedy_sampling.restype = NlsParams
        L.nls_create.argtypes = [P(NlsParams), ctypes.c_int32, ctypes.c_int64, vp, P(vp)]
        L.nls_destroy.argtypes = [vp]
        L.nls_set_stream.argtypes = [vp, vp]
        L.nls_batch.argtypes = [vp]
        L.nls_batch.restype = ctypes.c_int32
        L.nls_vocab.argtypes = [vp]
        L.nls_vocab.restype = ctypes.c_int64
        L.nls_accept.argtypes = [vp, P(ctypes.c_int64), ctypes.c_int32]
        L.nls_accept_row.argtypes = [vp, ctypes.c_int32, P(ctypes.c_int64), ctypes.c_int32]
        L.nls_accept_device.argtypes = [vp, vp]
        L.nls_generate_step.argtypes = [vp, vp, vp, vp, vp, ctypes.c_int32, vp]
        L.nls_clear_history.argtypes = [vp]
        L.nls_sample.argtypes = [vp, vp, vp, vp, P(NlsDebug)]
        L.nls_sample_host.argtypes = [vp, P(ctypes.c_float), P(ctypes.c_int64)]
        L.nls_sample_host_noalloc.argtypes = [vp, P(ctypes.c_float), P(ctypes.c_int64)]
        L.nls_synchronize.argtypes = [vp]
        L.nls_rng_uniforms.argtypes = [ctypes.c_int64, ctypes.c_int64, P(ctypes.c_double)]
        L.nls_get_rng_state.argtypes = [vp, ctypes.c_int32, P(ctypes.c_uint64), P(ctypes.c_uint64)]
        L.nls_set_rng_state.argtypes = [vp, ctypes.c_int32, ctypes.c_uint64, ctypes.c_uint64]
        L.nls_top_tokens.argtypes = [vp, ctypes.c_int32, ctypes.c_int64, ctypes.c_int32, vp, vp, vp]
        L.nls_row_nll.argtypes = [vp, ctypes.c_int32, ctypes.c_int64, vp, vp, vp]
        L.nls_softmax_rows.argtypes = [vp, ctypes.c_int32, ctypes.c_int64, vp, vp]
        L.nls_log_prob.argtypes = [vp, ctypes.c_int32, ctypes.c_int64, vp, vp, vp, vp]
        L.nls_expf_device.argtypes = [vp, vp, ctypes.c_int64, vp]
        L.nls_profile_next.argtypes = [vp, vp, vp]
        L.nls_profile_next_generic.argtypes = [vp, vp, vp]
        L.nls_get_plan.argtypes = [vp, P(NlsPlan), P(ctypes.c_int32)]
        L.nls_status_string.argtypes = [ctypes.c_int]
        L.nls_status_string.restype = ctypes.c_char_p
        L.nls_last_error.restype = ctypes.c_char_p
        L.nls_lm_head_workspace.argtypes = [ctypes.c_int32, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32,
                                            ctypes.c_int32]
        L.nls_lm_head_workspace.restype = ctypes.c_size_t
        L.nls_lm_head_row_bytes.argtypes = [ctypes.c_int32, ctypes.c_int64]
        L.nls_lm_head_row_bytes.restype = ctypes.c_int64
        L.nls_argmax.argtypes = [vp, ctypes.c_int32, ctypes.c_int64, vp, vp]
        L.nls_lm_head.argtypes = [vp, ctypes.c_int32, ctypes.c_int64, ctypes.c_int64, vp, ctypes.c_int32, vp,
                                  ctypes.c_int32, P(NlsLora), vp, ctypes.c_size_t, vp]
        L.nls_lm_head.restype = ctypes.c_int32
        _lib = L
    return _lib


def check(status: int, what: str = "") -> None:
    if status != NLS_OK:
        L = lib()
        raise SamplerError(f"{what}: {L.nls_status_string(status).decode()} "
                           f"({L.nls_last_error().decode()})")


@dataclass
class SamplerParams:
    """SamplerParams (sampler.nim:11-21).  Omitted fields are zero, as in Nim."""

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


def defaultSampling() -> SamplerParams:
    """sampler.nim:28-31"""
    return SamplerParams(temperature=0.7, topK=40, topP=0.95, minP=0.05,
                         repeatPenalty=1.1, repeatLastN=64, seed=-1)


def greedySampling() -> SamplerParams:
    """sampler.nim:33-35"""
    return SamplerParams(temperature=0.0, topK=0, topP=1.0, repeatPenalty=1.0, seed=0)


def _to_c(p: SamplerParams, keep: list) -> NlsParams:
    c = NlsParams()
    c.temperature = p.temperature
    c.top_k = p.topK
    c.top_p = p.topP
    c.min_p = p.minP
    c.repeat_penalty = p.repeatPenalty
    c.repeat_last_n = p.repeatLastN
    c.presence_penalty = p.presencePenalty
    c.frequency_penalty = p.frequencyPenalty
    c.seed = p.seed
    n = len(p.logitBias)
    if n:
        ids = (ctypes.c_int64 * n)(*[int(k) for k in p.logitBias.keys()])
        vals = (ctypes.c_double * n)(*[float(v) for v in p.logitBias.values()])
        keep.extend([ids, vals])
        c.logit_bias_ids = ids
        c.logit_bias_values = vals
    c.logit_bias_count = n
    return c


def rng_uniforms(seed: int, n: int):
    """The first n values of rand(1.0) after initRand(seed) (Nim std/random)."""
    arr = (ctypes.c_double * max(n, 1))()
    check(lib().nls_rng_uniforms(seed, n, arr), "nls_rng_uniforms")
    return [arr[i] for i in range(n)]


def _ptr(t) -> Optional[int]:
    return None if t is None else t.data_ptr()


class BatchSampler:
    """B independent samplers (one per row) on the current HIP device.

    ``sample`` takes a device tensor of shape [B, V] (float32) and returns the
    sampled ids as a device int32 tensor; it is asynchronous on ``stream``.
    """

    def __init__(self, params: Sequence[SamplerParams], vocab: int, stream=None):
        import torch

        self._torch = torch
        L = lib()
        keep: list = []
        B = len(params)
        arr = (NlsParams * B)(*[_to_c(p, keep) for p in params])
        self._stream = stream
        self.B, self.V = B, int(vocab)
        h = ctypes.c_void_p()
        check(L.nls_create(arr, B, int(vocab), self._stream_ptr(), ctypes.byref(h)), "nls_create")
        self._h = h

    def _stream_ptr(self):
        s = self._stream
        if s is None:
            return None
        return ctypes.c_void_p(s.cuda_stream if hasattr(s, "cuda_stream") else int(s))

    def close(self):
        if getattr(self, "_h", None):
            lib().nls_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def accept(self, ids, row: Optional[int] = None):
        """accept (sampler.nim:41-43): one id per row ([B]) or [B, n] ids; or
        ids for a single `row`.  ACCEPT_SKIP entries append nothing."""
        import numpy as np

        a = np.ascontiguousarray(np.asarray(ids, dtype=np.int64))
        L = lib()
        if row is not None:
            a = a.reshape(-1)
            check(L.nls_accept_row(self._h, int(row), a.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)),
                                   a.size), "nls_accept_row")
            return
        a = a.reshape(self.B, -1)
        check(L.nls_accept(self._h, a.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)), a.shape[1]),
              "nls_accept")

    def accept_device(self, d_ids):
        """One id per row from device int32 [B]; ACCEPT_SKIP32 appends nothing."""
        assert d_ids.dtype == self._torch.int32 and d_ids.is_cuda and d_ids.numel() == self.B
        check(lib().nls_accept_device(self._h, ctypes.c_void_p(d_ids.data_ptr())), "nls_accept_device")

    def clear_history(self):
        check(lib().nls_clear_history(self._h), "nls_clear_history")

    def sample(self, logits, u=None, out=None, debug_cap: int = 0):
        """sample (sampler.nim:59-121) for every row.  `u` (float64 [B], device)
        stands for each row's rand(1.0); None draws from the rows' own RNGs.
        With debug_cap > 0 returns (ids, debug dict of device tensors)."""
        torch = self._torch
        assert logits.is_cuda and logits.dtype == torch.float32 and logits.is_contiguous()
        assert tuple(logits.shape) == (self.B, self.V), (logits.shape, self.B, self.V)
        if u is not None:
            assert u.is_cuda and u.dtype == torch.float64 and u.numel() == self.B and u.is_contiguous()
        if out is None:
            out = torch.empty(self.B, dtype=torch.int32, device=logits.device)
        dbgp = None
        dbg = None
        if debug_cap > 0:
            dev = logits.device
            dbg = {
                "n": torch.full((self.B,), -1, dtype=torch.int32, device=dev),
                "ncand": torch.full((self.B,), -1, dtype=torch.int32, device=dev),
                "cand_ids": torch.full((self.B, debug_cap), -1, dtype=torch.int32, device=dev),
                "cand_probs": torch.zeros((self.B, debug_cap), dtype=torch.float32, device=dev),
                "total": torch.zeros((self.B,), dtype=torch.float32, device=dev),
                "path": torch.zeros((self.B,), dtype=torch.int32, device=dev),
            }
            dbgp = NlsDebug(dbg["n"].data_ptr(), dbg["ncand"].data_ptr(), dbg["cand_ids"].data_ptr(),
                            dbg["cand_probs"].data_ptr(), dbg["total"].data_ptr(),
                            dbg["path"].data_ptr(), debug_cap)
        check(lib().nls_sample(self._h, ctypes.c_void_p(logits.data_ptr()),
                               ctypes.c_void_p(_ptr(u)) if u is not None else None,
                               ctypes.c_void_p(out.data_ptr()),
                               ctypes.byref(dbgp) if dbgp is not None else None), "nls_sample")
        return (out, dbg) if debug_cap > 0 else out

    def generate_step(self, logits, eog, done, u=None, out=None):
        """One step of batched generation (chat.nim:204-208 for every row): rows
        with done == 0 sample; a row drawing an id in `eog` (int32 device
        tensor) gets done = 1 and accepts nothing, the others accept their id.
        Finished rows sample nothing (out = -1) and keep their RNG state.
        `done`: int32 device tensor [B], zero before the first step.  Returns out."""
        torch = self._torch
        assert logits.is_cuda and logits.dtype == torch.float32 and logits.is_contiguous()
        assert tuple(logits.shape) == (self.B, self.V)
        assert done.is_cuda and done.dtype == torch.int32 and done.numel() == self.B and done.is_contiguous()
        assert eog.is_cuda and eog.dtype == torch.int32 and eog.is_contiguous()
        if u is not None:
            assert u.is_cuda and u.dtype == torch.float64 and u.numel() == self.B and u.is_contiguous()
        if out is None:
            out = torch.empty(self.B, dtype=torch.int32, device=logits.device)
        check(lib().nls_generate_step(self._h, ctypes.c_void_p(logits.data_ptr()),
                                      ctypes.c_void_p(_ptr(u)) if u is not None else None,
                                      ctypes.c_void_p(out.data_ptr()),
                                      ctypes.c_void_p(eog.data_ptr()) if eog.numel() else None,
                                      int(eog.numel()), ctypes.c_void_p(done.data_ptr())),
              "nls_generate_step")
        return out

    def sample_host(self, logits):
        """Blocking: host [B, V] float32 logits -> host int64 [B] ids."""
        import numpy as np

        x = np.ascontiguousarray(np.asarray(logits, dtype=np.float32).reshape(self.B, self.V))
        o = np.zeros(self.B, dtype=np.int64)
        check(lib().nls_sample_host(self._h, x.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                    o.ctypes.data_as(ctypes.POINTER(ctypes.c_int64))), "nls_sample_host")
        return o

    def sample_host_noalloc(self, logits):
        """sample_host through the library's static staging (nothing allocated)."""
        import numpy as np

        x = np.ascontiguousarray(np.asarray(logits, dtype=np.float32).reshape(self.B, self.V))
        o = np.zeros(self.B, dtype=np.int64)
        check(lib().nls_sample_host_noalloc(self._h, x.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                            o.ctypes.data_as(ctypes.POINTER(ctypes.c_int64))),
              "nls_sample_host_noalloc")
        return o

    def profile_next(self, start_event, stop_event):
        """Time the next sample()'s streaming kernel with two torch.cuda.Events
        (recorded on this sampler's stream)."""
        check(lib().nls_profile_next(self._h, ctypes.c_void_p(start_event.cuda_event),
                                     ctypes.c_void_p(stop_event.cuda_event)), "nls_profile_next")

    def profile_next_generic(self, start_event, stop_event):
        """Time the next sample()'s whole-row kernel (when it launches one)."""
        check(lib().nls_profile_next_generic(self._h, ctypes.c_void_p(start_event.cuda_event),
                                             ctypes.c_void_p(stop_event.cuda_event)), "nls_profile_next_generic")

    def plan(self):
        """(NlsPlan, per-row list: 1 where the streaming kernel runs the row)."""
        p = NlsPlan()
        rows = (ctypes.c_int32 * self.B)()
        check(lib().nls_get_plan(self._h, ctypes.byref(p), rows), "nls_get_plan")
        return p, list(rows)

    def synchronize(self):
        check(lib().nls_synchronize(self._h), "nls_synchronize")

    def rng_state(self, row: int):
        a0, a1 = ctypes.c_uint64(), ctypes.c_uint64()
        check(lib().nls_get_rng_state(self._h, row, ctypes.byref(a0), ctypes.byref(a1)), "rng")
        return a0.value, a1.value

    def set_rng_state(self, row: int, a0: int, a1: int):
        check(lib().nls_set_rng_state(self._h, row, a0, a1), "rng")


class Sampler:
    """One nimllm Sampler (sampler.nim:23-26) backed by a one-row BatchSampler.

    ``sample(logits)`` accepts a host sequence/ndarray (through
    nls_sample_host: the kernel reads it from the handle's pinned staging) or a
    1-D device tensor, and returns the id as a Python int.
    """

    def __init__(self, p: SamplerParams, vocab: int):
        self.params = p
        self._b = BatchSampler([p], vocab)

    def accept(self, tok: int):
        self._b.accept([int(tok)])

    def sample(self, logitsIn) -> int:
        torch = self._b._torch
        if isinstance(logitsIn, torch.Tensor) and logitsIn.is_cuda:
            out = self._b.sample(logitsIn.reshape(1, -1).contiguous().float())
            return int(out.cpu()[0])
        return int(self._b.sample_host(logitsIn)[0])


def newSampler(p: Optional[SamplerParams] = None, vocab: int = 0) -> Sampler:
    """newSampler (sampler.nim:37-39).  The vocabulary size is fixed per sampler
    here because the device buffers are sized from it."""
    if vocab <= 0:
        raise SamplerError("newSampler needs the vocabulary size")
    return Sampler(p if p is not None else defaultSampling(), vocab)


TOP_TOKENS_MAX = 2048  # largest number of entries per row nls_top_tokens returns


def top_tokens_device(logits, n: int = 5):
    """topTokens (sampler.nim:123-130) for a [rows, V] float32 device tensor:
    returns int32 ids and float32 probabilities, both [rows, min(n, V)], in the
    reference's order (probability descending, ascending id on ties)."""
    import torch

    x = logits if logits.dim() == 2 else logits.reshape(1, -1)
    assert x.is_cuda and x.dtype == torch.float32 and x.is_contiguous()
    rows, V = x.shape
    m = max(0, min(n, V))
    ids = torch.empty((rows, max(n, 1)), dtype=torch.int32, device=x.device)
    probs = torch.empty((rows, max(n, 1)), dtype=torch.float32, device=x.device)
    stream = torch.cuda.current_stream(x.device).cuda_stream
    check(lib().nls_top_tokens(ctypes.c_void_p(x.data_ptr()), rows, V, n,
                               ctypes.c_void_p(ids.data_ptr()), ctypes.c_void_p(probs.data_ptr()),
                               ctypes.c_void_p(stream)), "nls_top_tokens")
    return ids[:, :m], probs[:, :m]


def topTokens(logits, n: int = 5):
    """topTokens (sampler.nim:123-130): the n most probable ids of one row of
    logits (any float32 sequence or tensor) with their probabilities, as a list
    of (id, probability) pairs, computed on the device."""
    import numpy as np
    import torch

    x = logits if torch.is_tensor(logits) else torch.from_numpy(np.ascontiguousarray(logits, dtype=np.float32))
    x = x.reshape(1, -1).to(device="cuda", dtype=torch.float32).contiguous()
    ids, probs = top_tokens_device(x, n)
    return [(int(i), float(p)) for i, p in zip(ids[0].tolist(), probs[0].tolist())]


def argmax_device(logits):
    """argmax (sampler.nim:45-49) of every row of a [rows, V] (or [V])
    float32 device tensor: int32 [rows], the first index of each row's
    greatest value (a NaN never taken; a NaN at index 0 answers 0)."""
    import torch

    x = logits if logits.dim() == 2 else logits.reshape(1, -1)
    assert x.is_cuda and x.dtype == torch.float32 and x.is_contiguous()
    rows, V = x.shape
    out = torch.empty(rows, dtype=torch.int32, device=x.device)
    stream = torch.cuda.current_stream(x.device).cuda_stream
    check(lib().nls_argmax(ctypes.c_void_p(x.data_ptr()) if V else None, rows, V,
                           ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(stream)), "nls_argmax")
    return out


def argmax(logits) -> int:
    """argmax (sampler.nim:45-49) of one row of logits (any float32 sequence
    or tensor), computed on the device."""
    import numpy as np
    import torch

    x = logits if torch.is_tensor(logits) else torch.from_numpy(np.ascontiguousarray(logits, dtype=np.float32))
    x = x.reshape(1, -1).to(device="cuda", dtype=torch.float32).contiguous()
    return int(argmax_device(x)[0].item())


def row_nll_device(logits, targets):
    """perplexity's per-position term (src/nimllm/model.nim:578-583) for a
    [rows, V] float32 device tensor and int32 target ids [rows]: float64
    -(l[t] - max) + ln(sum of exp(l - max)) per row."""
    import torch

    x = logits if logits.dim() == 2 else logits.reshape(1, -1)
    assert x.is_cuda and x.dtype == torch.float32 and x.is_contiguous()
    t = targets.to(device=x.device, dtype=torch.int32).contiguous()
    rows, V = x.shape
    assert t.numel() == rows
    out = torch.empty(rows, dtype=torch.float64, device=x.device)
    stream = torch.cuda.current_stream(x.device).cuda_stream
    check(lib().nls_row_nll(ctypes.c_void_p(x.data_ptr()), rows, V, ctypes.c_void_p(t.data_ptr()),
                            ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(stream)), "nls_row_nll")
    return out


def softmax_device(logits, out=None):
    """softmaxInPlace (src/nimllm/sampler.nim:51-57) of every row of a
    [rows, V] (or [V]) float32 device tensor; `out` may be `logits` itself
    (the reference's in-place form).  Returns out."""
    import torch

    x = logits if logits.dim() == 2 else logits.reshape(1, -1)
    assert x.is_cuda and x.dtype == torch.float32 and x.is_contiguous()
    rows, V = x.shape
    if out is None:
        out = torch.empty_like(logits)
    assert out.is_cuda and out.dtype == torch.float32 and out.is_contiguous() and out.numel() == x.numel()
    stream = torch.cuda.current_stream(x.device).cuda_stream
    check(lib().nls_softmax_rows(ctypes.c_void_p(x.data_ptr()), rows, V, ctypes.c_void_p(out.data_ptr()),
                                 ctypes.c_void_p(stream)), "nls_softmax_rows")
    return out


def log_prob_device(logits, targets):
    """logProb's per-token term (nimllm-doc-en.md:1700-1707) for a [rows, V]
    float32 device tensor and int32 target ids [rows]: (p[target] float32,
    ln(float64(p[target])) float64) per row, p = softmaxInPlace of the row."""
    import torch

    x = logits if logits.dim() == 2 else logits.reshape(1, -1)
    assert x.is_cuda and x.dtype == torch.float32 and x.is_contiguous()
    t = targets.to(device=x.device, dtype=torch.int32).contiguous()
    rows, V = x.shape
    assert t.numel() == rows
    prob = torch.empty(rows, dtype=torch.float32, device=x.device)
    logp = torch.empty(rows, dtype=torch.float64, device=x.device)
    stream = torch.cuda.current_stream(x.device).cuda_stream
    check(lib().nls_log_prob(ctypes.c_void_p(x.data_ptr()), rows, V, ctypes.c_void_p(t.data_ptr()),
                             ctypes.c_void_p(prob.data_ptr()), ctypes.c_void_p(logp.data_ptr()),
                             ctypes.c_void_p(stream)), "nls_log_prob")
    return prob, logp


def log_prob(context_logits, continuation):
    """logProb (nimllm-doc-en.md:1700-1707) given the logits the model
    produced before each continuation token ([len, V] device tensor) and the
    continuation's ids: the float64 sum of ln(p[id]) in token order."""
    _, lp = log_prob_device(context_logits, continuation)
    total = 0.0
    for v in lp.cpu().tolist():
        total += v
    return total


def perplexity(logits, targets):
    """exp of the mean per-position term over the rows (model.nim:570-589,
    for logits already evaluated), computed on the device."""
    import math

    nll = row_nll_device(logits, targets)
    return math.exp(float(nll.sum().item()) / max(1, nll.numel()))


def expf_device(x, out=None):
    """Correctly rounded exp of a float32 device tensor."""
    import torch

    assert x.is_cuda and x.dtype == torch.float32 and x.is_contiguous()
    if out is None:
        out = torch.empty_like(x)
    check(lib().nls_expf_device(ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(out.data_ptr()),
                                x.numel(), None), "nls_expf_device")
    return out


def inf_bias() -> float:
    return -math.inf


# GGML type codes (src/nimllm/quant.nim:14-19) nls_lm_head reads
GGML_TYPES = {"F32": 0, "F16": 1, "Q4_0": 2, "Q4_1": 3, "Q5_0": 6, "Q5_1": 7, "Q8_0": 8, "Q2_K": 10,
              "Q3_K": 11, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14, "Q8_K": 15, "BF16": 30}


def lm_head_workspace(ggml_type: int, cols: int, nb: int, lora_rank: int = 0, exact: bool = False) -> int:
    return int(lib().nls_lm_head_workspace(ggml_type, cols, nb, lora_rank, int(exact)))


def lm_head(weight, ggml_type: int, rows: int, cols: int, x, exact: bool = False, lora=None, out=None,
            work=None):
    """matmul(m.output, x, y, nb) (src/nimllm/model.nim:179-200) on the device:
    weight is a uint8 device tensor of rows * rowBytes(type, cols) GGUF bytes,
    x a float32 device tensor [nb, cols] (or [cols]); returns y [nb, rows]
    float32 ([rows] for a 1-D x).  exact is the reference's exactMatmul;
    lora = (a [rank, cols], b [rows, rank], scale) device tensors.  `work`
    may pass a preallocated uint8 device workspace."""
    import torch

    x2 = x if x.dim() == 2 else x.reshape(1, -1)
    assert x2.is_cuda and x2.dtype == torch.float32 and x2.is_contiguous() and x2.shape[1] == cols
    rb = int(lib().nls_lm_head_row_bytes(ggml_type, cols))
    if rb < 0:
        raise SamplerError(f"lm_head: type {ggml_type} with cols={cols} is not a readable GGUF row "
                           "(rowBytes raises)")
    assert weight.is_cuda and weight.is_contiguous() and weight.dtype == torch.uint8
    assert weight.device == x2.device, "lm_head: weight and x on different devices"
    assert weight.numel() >= rows * rb, (
        f"lm_head: weight holds {weight.numel()} bytes, rows x rowBytes = {rows * rb}")
    nb = x2.shape[0]
    if out is None:
        out = torch.empty((nb, rows), dtype=torch.float32, device=x2.device)
    assert out.is_cuda and out.dtype == torch.float32 and out.is_contiguous() and out.numel() == nb * rows
    lo = None
    rank = 0
    if lora is not None:
        a, b, scale = lora
        assert a.is_contiguous() and b.is_contiguous() and a.dtype == torch.float32 and b.dtype == torch.float32
        assert a.is_cuda and b.is_cuda and a.device == x2.device and b.device == x2.device
        assert a.dim() == 2 and b.dim() == 2
        rank = a.shape[0]
        assert tuple(a.shape) == (rank, cols) and tuple(b.shape) == (rows, rank), (
            f"lm_head: LoRA a {tuple(a.shape)} must be ({rank}, {cols}), b {tuple(b.shape)} ({rows}, {rank})")
        lo = NlsLora(a.data_ptr(), b.data_ptr(), rank, float(scale))
    need = lm_head_workspace(ggml_type, cols, nb, rank, exact)
    if work is None or work.numel() < need:
        work = torch.empty(max(need, 1), dtype=torch.uint8, device=x2.device)
    stream = torch.cuda.current_stream(x2.device).cuda_stream
    check(lib().nls_lm_head(ctypes.c_void_p(weight.data_ptr()), ggml_type, rows, cols,
                            ctypes.c_void_p(x2.data_ptr()), nb, ctypes.c_void_p(out.data_ptr()), int(exact),
                            ctypes.byref(lo) if lo is not None else None, ctypes.c_void_p(work.data_ptr()),
                            work.numel(), ctypes.c_void_p(stream)), "nls_lm_head")
    return out if x.dim() == 2 else out.reshape(rows)
