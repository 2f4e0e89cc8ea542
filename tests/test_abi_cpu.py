"""C-ABI checks that need no GPU: the library loads, exports every symbol
include/*.h declares, and its host-only entry points behave."""
import ctypes
import glob
import os
import re

import numpy as np
import pytest

import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = sorted(glob.glob(os.path.join(ROOT, "include", "*.h")))


def declared_symbols():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names |= set(re.findall(r"\b(nls_[a-z_]+)\s*\(", text))
    return sorted(names)


def test_header_and_binding_agree(pkg):
    assert sorted(pkg.EXPORTED) == declared_symbols()


def test_library_exports_every_declared_symbol(pkg):
    L = pkg.lib()
    for name in declared_symbols():
        assert hasattr(L, name), name


def test_rng_uniforms_match_oracle(pkg):
    for seed in (0, 1, 42, 1234, 2**40 + 7):
        assert pkg.rng_uniforms(seed, 64) == list(O.uniforms(seed, 64))
    from nimllm_amd import workloads

    assert np.array_equal(workloads.nim_uniforms(99, 32), O.uniforms(99, 32))


def test_presets_mirror_reference(pkg):
    L = pkg.lib()
    d = L.nls_default_sampling()
    assert (d.temperature, d.top_k, d.top_p, d.min_p, d.repeat_penalty, d.repeat_last_n,
            d.seed) == (0.7, 40, 0.95, 0.05, 1.1, 64, -1)
    g = L.nls_greedy_sampling()
    assert (g.temperature, g.top_k, g.top_p, g.repeat_penalty, g.seed) == (0.0, 0, 1.0, 1.0, 0)
    dp = pkg.defaultSampling()
    assert (dp.temperature, dp.topK, dp.topP, dp.minP, dp.repeatPenalty, dp.repeatLastN,
            dp.seed) == (0.7, 40, 0.95, 0.05, 1.1, 64, -1)


def test_error_paths_without_device(pkg):
    """Invalid arguments are rejected before any device work; create without
    a GPU reports NLS_ERR_NO_DEVICE instead of crashing."""
    L = pkg.lib()
    h = ctypes.c_void_p()
    p = (pkg.NlsParams * 1)(L.nls_greedy_sampling())
    assert L.nls_create(p, 0, 10, None, ctypes.byref(h)) == 1      # batch < 1
    assert L.nls_create(p, 1, 0, None, ctypes.byref(h)) == 2       # empty vocab
    assert L.nls_create(None, 1, 10, None, ctypes.byref(h)) == 1
    assert L.nls_sample(None, None, None, None, None) == 1
    assert L.nls_accept(None, None, 0) == 1
    assert L.nls_rng_uniforms(1, -1, None) == 1
    # topTokens: nothing to return is a no-op; more than 2048 results per row,
    # negative sizes and missing buffers are rejected before any device work
    assert L.nls_top_tokens(None, 1, 10, 0, None, None, None) == 0
    assert L.nls_top_tokens(None, 0, 10, 5, None, None, None) == 0
    assert L.nls_top_tokens(None, -1, 10, 5, None, None, None) == 1
    assert L.nls_top_tokens(None, 1, 100000, 3000, None, None, None) == 1
    assert L.nls_top_tokens(None, 1, 100, 5, None, None, None) == 1
    assert L.nls_row_nll(None, 0, 100, None, None, None) == 0      # no rows
    assert L.nls_row_nll(None, -1, 100, None, None, None) == 1
    assert L.nls_row_nll(None, 1, 0, None, None, None) == 2        # empty vocab
    assert L.nls_row_nll(None, 1, 100, None, None, None) == 1      # null buffers
    assert L.nls_status_string(5) == b"no usable device"
    import torch

    if not torch.cuda.is_available():
        assert L.nls_create(p, 1, 10, None, ctypes.byref(h)) == 5


def test_fixture_file_is_consistent_with_oracle():
    """The committed fixtures still match the oracle (guards both)."""
    import json
    import math

    d = json.load(open(os.path.join(ROOT, "tests", "golden", "sampler_cases.json")))
    assert len(d["cases"]) >= 20
    for c in d["cases"]:
        x = np.array(c["logits_bits"], dtype=np.uint32).view(np.float32)
        bias = {k: (-math.inf if v == "-inf" else math.inf if v == "inf" else v)
                for k, v in c["bias"]}
        res, cand, probs, _ = O.sample(O.make_params(**c["params"]), x, c["history"], bias, c["u"],
                                       O.EXPF_CR)
        e = c["expect"]
        assert res.id == e["id"] and res.n == e["n"]
        assert [int(v) for v in cand[:res.n]] == e["cand"]
        assert [int(v) for v in probs[:res.n].view(np.uint32)] == e["probs_bits"]
        r2, _, _, _ = O.sample(O.make_params(**c["params"]), x, c["history"], bias, c["u"],
                               O.EXPF_LIBM)
        assert r2.id == c["id_libm"]


def test_lm_head_host_checks(pkg):
    """nls_lm_head's argument checks run on the host before any launch."""
    L = pkg.lib()
    # workspace: int8 activations (nb * cols bytes) + block scales, each
    # 256-byte aligned; none on the float path
    assert L.nls_lm_head_workspace(14, 2048, 1, 0, 0) == 2048 + 256
    assert L.nls_lm_head_workspace(14, 2048, 1, 0, 1) == 0
    assert L.nls_lm_head_workspace(8, 2048, 5, 0, 0) == 0          # Q8_0, nb > 4: float path
    assert L.nls_lm_head_workspace(8, 2048, 4, 0, 0) == 8192 + 1024
    assert L.nls_lm_head_workspace(1, 1000, 2, 3, 0) == 256         # LoRA tmp only
    assert L.nls_lm_head_workspace(9, 2048, 1, 0, 0) == 0           # Q8_1: not readable
    INVALID = 1
    assert L.nls_lm_head(None, 9, 10, 256, None, 1, None, 0, None, None, 0, None) == INVALID
    assert L.nls_lm_head(None, 14, 10, 100, None, 1, None, 0, None, None, 0, None) == INVALID
    assert L.nls_lm_head(None, 14, 0, 256, None, 1, None, 0, None, None, 0, None) == 0
    assert L.nls_lm_head(None, 14, 10, 256, None, 0, None, 0, None, None, 0, None) == 0
    assert L.nls_lm_head(None, 14, 10, 256, None, 1, None, 0, None, None, 0, None) == INVALID
