"""nls_sample_host_noalloc (no counterpart in the reference): the
allocation-free variant of nls_sample_host, checked through the C ABI against
nls_sample_host on the same inputs, two calls in a row, the second smaller,
and with the device's free memory unchanged across its calls (the first call
after nls_create included)."""
import ctypes
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _handles(pkg, B, V, seed, hist):
    """Two handles with the same rows (same seeds) and the same history."""
    L = pkg.lib()
    keep = []
    rows = []
    for b in range(B):
        p = pkg.SamplerParams(temperature=0.8, topK=[40, 0, 300, 0][b % 4], topP=0.95,
                              minP=[0.0, 0.05, 0.0, 0.0][b % 4], repeatPenalty=1.1, repeatLastN=0,
                              presencePenalty=0.2, frequencyPenalty=0.3, seed=seed + b)
        if b % 4 == 3:
            p.temperature = 0.0
        p.logitBias = {5: -float("inf"), 17: 1.5}
        rows.append(pkg._to_c(p, keep))
    arr = (pkg.NlsParams * B)(*rows)
    hs = []
    for _ in range(2):
        h = ctypes.c_void_p()
        pkg.check(L.nls_create(arr, B, V, None, ctypes.byref(h)), "nls_create")
        a = np.ascontiguousarray(hist, dtype=np.int64)
        pkg.check(L.nls_accept(h, a.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)), a.shape[1]),
                  "nls_accept")
        hs.append(h)
    return hs


def test_sample_host_noalloc_matches_sample_host(pkg):
    import torch

    assert torch.cuda.is_available(), "no GPU"
    L = pkg.lib()
    rng = np.random.default_rng(31)
    for call, (B, V) in enumerate([(8, 128256), (3, 50000)]):
        say(f"[no_alloc] call {call}: B={B} V={V}")
        hist = rng.integers(0, V, size=(B, 200))
        h_ref, h_na = _handles(pkg, B, V, 77 + call, hist)
        try:
            free0 = None
            for step in range(3):
                x = np.ascontiguousarray(rng.standard_normal((B, V)).astype(np.float32) * 2.5)
                xp = x.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
                want = np.zeros(B, dtype=np.int64)
                got = np.full(B, -7, dtype=np.int64)
                # (the reference call's first run allocates its own buffers and
                # loads the kernels, before the free memory is read)
                pkg.check(L.nls_sample_host(h_ref, xp, want.ctypes.data_as(ctypes.POINTER(ctypes.c_int64))),
                          "nls_sample_host")
                torch.cuda.synchronize()
                if free0 is None:
                    free0 = torch.cuda.mem_get_info()[0]
                pkg.check(L.nls_sample_host_noalloc(h_na, xp, got.ctypes.data_as(ctypes.POINTER(ctypes.c_int64))),
                          "nls_sample_host_noalloc")
                assert np.array_equal(got, want), (call, step, got, want)
            torch.cuda.synchronize()
            free1 = torch.cuda.mem_get_info()[0]
            assert free1 == free0, (call, free0, free1)
        finally:
            L.nls_destroy(h_ref)
            L.nls_destroy(h_na)
    # beyond the 16 MiB staging the call is refused before any device work
    V = 128256
    B = (16 << 20) // (4 * V) + 1
    say(f"[no_alloc] oversized: B={B} V={V}")
    h = ctypes.c_void_p()
    arr = (pkg.NlsParams * B)(*[L.nls_greedy_sampling() for _ in range(B)])
    pkg.check(L.nls_create(arr, B, V, None, ctypes.byref(h)), "nls_create")
    try:
        x = np.zeros((B, V), dtype=np.float32)
        o = np.zeros(B, dtype=np.int64)
        st = L.nls_sample_host_noalloc(h, x.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                       o.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)))
        assert st == 6, st  # NLS_ERR_UNSUPPORTED
        assert b"16 MiB" in L.nls_last_error()
    finally:
        L.nls_destroy(h)
