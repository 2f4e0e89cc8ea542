"""The C ABI's argument checks (include/nimllm_sampler.h, nimllm_lmhead.h):
every malformed call returns its status code before any device work, never
crashes, and leaves a handle usable.  The reference raises on an empty row
(IndexDefect, src/nimllm/sampler.nim:121), which the ABI reports as
NLS_ERR_EMPTY_VOCAB."""
import ctypes
import sys

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

OK, INVALID, EMPTY, UNSUPPORTED = 0, 1, 2, 6


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def test_malformed_calls_return_status_codes(pkg):
    import torch

    assert torch.cuda.is_available(), "no GPU"
    L = pkg.lib()
    P = ctypes.POINTER
    vp = ctypes.c_void_p
    keep = []
    p = pkg.SamplerParams(temperature=0.8, topK=5, topP=0.9, repeatPenalty=1.0, seed=3)
    arr = (pkg.NlsParams * 2)(pkg._to_c(p, keep), pkg._to_c(p, keep))
    h = vp()
    say("[errors] nls_create")
    assert L.nls_create(arr, 2, 100, None, None) == INVALID
    assert L.nls_create(None, 2, 100, None, ctypes.byref(h)) == INVALID and not h.value
    assert L.nls_create(arr, 0, 100, None, ctypes.byref(h)) == INVALID
    assert L.nls_create(arr, 2, 0, None, ctypes.byref(h)) == EMPTY
    assert L.nls_create(arr, 2, 1 << 31, None, ctypes.byref(h)) == UNSUPPORTED
    assert L.nls_destroy(None) == INVALID
    assert L.nls_create(arr, 2, 100, None, ctypes.byref(h)) == OK and h.value
    try:
        say("[errors] handle calls")
        ids = np.array([1, 2, 3], dtype=np.int64)
        ip = ids.ctypes.data_as(P(ctypes.c_int64))
        assert L.nls_accept(h, None, 3) == INVALID
        assert L.nls_accept(h, ip, -1) == INVALID
        assert L.nls_accept_row(h, 2, ip, 1) == INVALID
        assert L.nls_accept_row(h, -1, ip, 1) == INVALID
        out = torch.zeros(2, dtype=torch.int32, device="cuda")
        x = torch.zeros((2, 100), dtype=torch.float32, device="cuda")
        assert L.nls_sample(h, None, None, vp(out.data_ptr()), None) == INVALID
        assert L.nls_sample(h, vp(x.data_ptr()), None, None, None) == INVALID
        dbg = pkg.NlsDebug(None, None, None, None, None, None, -1)
        assert L.nls_sample(h, vp(x.data_ptr()), None, vp(out.data_ptr()), ctypes.byref(dbg)) == INVALID
        done = torch.zeros(2, dtype=torch.int32, device="cuda")
        assert L.nls_generate_step(h, vp(x.data_ptr()), None, vp(out.data_ptr()), None, 2,
                                   vp(done.data_ptr())) == INVALID
        a0, a1 = ctypes.c_uint64(), ctypes.c_uint64()
        assert L.nls_get_rng_state(h, 2, ctypes.byref(a0), ctypes.byref(a1)) == INVALID
        assert L.nls_set_rng_state(h, -1, 1, 2) == INVALID
        hx = np.zeros((2, 100), dtype=np.float32)
        o = np.zeros(2, dtype=np.int64)
        assert L.nls_sample_host(h, None, o.ctypes.data_as(P(ctypes.c_int64))) == INVALID
        assert L.nls_sample_host(h, hx.ctypes.data_as(P(ctypes.c_float)), None) == INVALID
        # the handle still samples, against the oracle, after the refused calls
        rng = np.random.default_rng(4)
        xs = (rng.standard_normal((2, 100)) * 2).astype(np.float32)
        u = rng.random(2)
        du = torch.from_numpy(u).cuda()
        assert L.nls_sample(h, vp(torch.from_numpy(xs).cuda().data_ptr()), vp(du.data_ptr()),
                            vp(out.data_ptr()), None) == OK
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        op = O.make_params(temperature=0.8, topK=5, topP=0.9, minP=0.0, repeatPenalty=1.0, repeatLastN=0,
                           presencePenalty=0.0, frequencyPenalty=0.0, seed=3)
        for b in range(2):
            assert got[b] == O.sample(op, xs[b], (), {}, float(u[b]), O.EXPF_CR, want_cand=False)[0].id
    finally:
        assert L.nls_destroy(h) == OK
    say("[errors] row entry points")
    d = torch.zeros((3, 64), dtype=torch.float32, device="cuda")
    t = torch.zeros(3, dtype=torch.int32, device="cuda")
    o32 = torch.zeros((3, 64), dtype=torch.int32, device="cuda")
    of = torch.zeros((3, 64), dtype=torch.float32, device="cuda")
    o64 = torch.zeros(3, dtype=torch.float64, device="cuda")
    dp, tp = vp(d.data_ptr()), vp(t.data_ptr())
    assert L.nls_top_tokens(dp, -1, 64, 5, vp(o32.data_ptr()), vp(of.data_ptr()), None) == INVALID
    assert L.nls_top_tokens(dp, 3, 1 << 29, 5, vp(o32.data_ptr()), vp(of.data_ptr()), None) == INVALID
    assert L.nls_top_tokens(dp, 3, 4096, 2049, vp(o32.data_ptr()), vp(of.data_ptr()), None) == INVALID
    assert L.nls_top_tokens(dp, 3, 64, 5, None, vp(of.data_ptr()), None) == INVALID
    assert L.nls_top_tokens(dp, 0, 64, 5, None, None, None) == OK
    assert L.nls_row_nll(dp, 3, 0, tp, vp(o64.data_ptr()), None) == EMPTY
    assert L.nls_row_nll(dp, 3, 64, None, vp(o64.data_ptr()), None) == INVALID
    assert L.nls_softmax_rows(dp, 3, 0, vp(of.data_ptr()), None) == EMPTY
    assert L.nls_softmax_rows(dp, 0, 64, None, None) == OK
    assert L.nls_log_prob(dp, 3, 64, tp, None, vp(o64.data_ptr()), None) == INVALID
    assert L.nls_argmax(dp, 3, 1 << 29, vp(o32.data_ptr()), None) == INVALID
    assert L.nls_argmax(dp, 3, 64, None, None) == INVALID
    assert L.nls_argmax(None, 0, 64, None, None) == OK
    assert L.nls_expf_device(None, None, 5, None) == INVALID
    say("[errors] lm head")
    w = torch.zeros(1 << 16, dtype=torch.uint8, device="cuda")
    xw = torch.zeros((1, 256), dtype=torch.float32, device="cuda")
    yw = torch.zeros((1, 64), dtype=torch.float32, device="cuda")
    q6k = 14
    work_n = int(L.nls_lm_head_workspace(q6k, 256, 1, 0, 0))
    work = torch.zeros(max(work_n, 1), dtype=torch.uint8, device="cuda")
    args = lambda t_, cols, nb, wb: (vp(w.data_ptr()), t_, 64, cols, vp(xw.data_ptr()), nb, vp(yw.data_ptr()), 0,
                                     None, vp(work.data_ptr()), wb, None)
    assert L.nls_lm_head(*args(99, 256, 1, work.numel())) == INVALID  # a type the reference cannot read
    assert L.nls_lm_head(*args(q6k, 255, 1, work.numel())) == INVALID  # rowBytes raises: cols not whole blocks
    if work_n > 0:
        assert L.nls_lm_head(*args(q6k, 256, 1, work_n - 1)) == INVALID  # short workspace
    assert L.nls_lm_head(*args(q6k, 256, 0, work.numel())) == OK  # nb == 0 does nothing
    torch.cuda.synchronize()
    for code in (OK, INVALID, EMPTY, 3, 4, 5, UNSUPPORTED):
        assert L.nls_status_string(code)
