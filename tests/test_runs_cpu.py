"""CPU checks of the grouped sort path (nim.llm_amd/csrc/nls_runs.h and
nls_grouped.h, which the gfx950 kernel compiles as device code).

* tests/runs_check.cpp: the closed forms of a run of equal terms against the
  plain sequential fp32 loops, on random and constructed runs (ties to even,
  binade crossings, runs of millions of terms, targets on exact partial sums).
* tests/exp64_check.cpp: the float64 exp of the row log-sum-exp
  (nls_exp64.h) against the C library's exp on float32 arguments.
* tests/seqsum_check.cpp: the workgroup evaluation of the sequential fp32 sum
  (nls_seqsum.h: parity maps scanned per binade, replays, binade changes)
  against one-at-a-time adds, on softmax terms, exact ties at every scale,
  subnormals, sums parked at 2^24 and NaN / infinite terms.
* tests/grouped_check.cpp: the whole group walk -- softmax sum, top-p, min-p,
  total, draw, and the drawn member -- against the oracle's sort path
  (src/nimllm/sampler.nim:96-121) on rows with ties, wide and narrow ranges,
  incomplete group tables and the extreme uniforms.
"""
import ctypes
import os
import subprocess

import numpy as np
import pytest

import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
FLAGS = ["-O2", "-ffp-contract=off", "-fno-fast-math", "-std=c++17", "-Wall"]
# AddressSanitizer + UndefinedBehaviorSanitizer: every check below also runs
# built with these (test_sanitized_checks), so an out-of-bounds table index
# or an undefined shift in the device logic fails the CPU suite
SANFLAGS = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g"]
if os.environ.get("NLS_SANITIZE") == "1":
    FLAGS = FLAGS + SANFLAGS


@pytest.fixture(scope="module")
def built(tmp_path_factory):
    d = tmp_path_factory.mktemp("runs")
    exe = str(d / "runs_check")
    so = str(d / "grouped_check.so")
    subprocess.run(["g++", *FLAGS, "-o", exe, os.path.join(HERE, "runs_check.cpp")], check=True)
    subprocess.run(["g++", *FLAGS, "-shared", "-fPIC", "-o", so,
                    os.path.join(HERE, "grouped_check.cpp")], check=True)
    return exe, so


def test_parallel_sequential_sum(tmp_path):
    exe = str(tmp_path / "seqsum_check")
    subprocess.run(["g++", *FLAGS, "-o", exe, os.path.join(HERE, "seqsum_check.cpp")], check=True)
    r = subprocess.run([exe], capture_output=True, text=True)
    assert r.returncode == 0 and "all sums bit-identical" in r.stdout, r.stdout[-4000:]


def test_exp64_matches_libm(tmp_path):
    exe = str(tmp_path / "exp64_check")
    subprocess.run(["g++", *FLAGS, "-o", exe, os.path.join(HERE, "exp64_check.cpp"), "-lm"], check=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert "0 failures" in r.stdout


def test_run_closed_forms_match_sequential_loops(built):
    exe, _ = built
    r = subprocess.run([exe, "12000"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]
    assert "0 failures" in r.stdout


def _rows(rng):
    """(name, logits, T, topP, minP) cases of the sort path."""
    out = []
    for V in (7, 300, 5000):
        out.append(("normal", rng.standard_normal(V).astype(np.float32), 1.0, 0.9, 0.05))
    for V in (1000, 20000):
        x = (np.round(rng.standard_normal(V) * 8.0) / 4.0).astype(np.float32)
        out.append(("ties_topp", x, 1.0, 0.8, 0.0))
        out.append(("ties_minp", x, 1.0, 1.0, 0.1))
        out.append(("ties_both", x, 0.9, 0.95, 0.02))
    V = 20000
    x = rng.standard_normal(V).astype(np.float32)
    x += (-4.4 * np.log(1 + rng.permutation(V))).astype(np.float32)
    out.append(("zipf_head", x, 0.7, 0.9, 0.05))
    out.append(("zipf_topp_only", x, 0.7, 0.99, 0.0))
    out.append(("wide", (rng.standard_normal(V) * 12).astype(np.float32), 1.0, 0.95, 0.0))
    out.append(("wide_minp", (rng.standard_normal(V) * 12).astype(np.float32), 1.0, 1.0, 1e-4))
    few = np.full(V, -3.0, dtype=np.float32)
    few[rng.choice(V, 40, replace=False)] = 2.0
    out.append(("two_values", few, 1.0, 0.97, 0.0))
    out.append(("two_values_all", few, 1.0, 1.0, 0.0))
    flat = np.zeros(4096, dtype=np.float32)
    out.append(("flat", flat, 1.0, 0.5, 0.0))
    out.append(("flat_all", flat, 1.0, 1.0, 0.0))
    return out


def test_group_walk_matches_oracle_sort_path(built):
    _, so = built
    L = ctypes.CDLL(so)
    P = ctypes.POINTER
    L.grouped_sample.argtypes = [P(ctypes.c_float), ctypes.c_int64, ctypes.c_float, ctypes.c_int,
                                 ctypes.c_double, ctypes.c_int, ctypes.c_float, ctypes.c_double,
                                 P(ctypes.c_int64), P(ctypes.c_int64), P(ctypes.c_float),
                                 P(ctypes.c_int32)]
    rng = np.random.default_rng(5)
    us = [0.0, 1.0 - 2.0 ** -53, 0.5] + list(rng.random(5))
    done = need_all = 0
    for name, x, T, topP, minP in _rows(rng):
        for u in us:
            p = O.make_params(temperature=T, topK=0, topP=topP, minP=minP, repeatPenalty=1.0,
                              repeatLastN=0, presencePenalty=0.0, frequencyPenalty=0.0, seed=1)
            res, _, _, _ = O.sample(p, x, (), {}, u, O.EXPF_CR, want_cand=False)
            gid, gn, gt, gg = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_float(), ctypes.c_int32()
            xc = np.ascontiguousarray(x)
            st = L.grouped_sample(xc.ctypes.data_as(P(ctypes.c_float)), len(x),
                                  np.float32(1.0 / T), int(0 < topP < 1), topP, int(minP > 0),
                                  np.float32(minP), u, ctypes.byref(gid), ctypes.byref(gn),
                                  ctypes.byref(gt), ctypes.byref(gg))
            if st == 11:  # the walk needs candidates outside the groups: whole-row path
                need_all += 1
                continue
            assert st == 0, (name, u, st)
            assert gid.value == res.id, (name, u, gid.value, res.id)
            assert gn.value == res.n, (name, u, gn.value, res.n)
            assert np.float32(gt.value).view(np.uint32) == np.float32(res.total).view(np.uint32), (
                name, u)
            done += 1
    # rows whose cutoffs end inside the groups never need the whole row
    assert done >= 100, (done, need_all)


def _san_runtime():
    libs = []
    for name in ("libasan.so", "libubsan.so"):
        p = subprocess.run(["gcc", "-print-file-name=" + name], capture_output=True, text=True).stdout.strip()
        if not os.path.isabs(p) or not os.path.exists(p):
            pytest.skip(f"no {name} for gcc")
        libs.append(p)
    return " ".join(libs)


@pytest.mark.skipif(os.environ.get("NLS_SANITIZE") == "1", reason="runs the sanitized build itself")
def test_sanitized_checks(tmp_path):
    """runs_check, seqsum_check and exp64_check built with ASan + UBSan and
    run; then, in a child interpreter with the sanitizer runtime preloaded and
    the oracle's sanitizer build (oracle/Makefile `asan`), this file's checks
    (the group walk of grouped_check.cpp among them), the oracle's pins, the
    LM head oracle's pins and the correctly rounded exp's mpmath check
    (expf_cr_check.cpp), each C/C++ part built with the same flags."""
    import sys

    for name, args, want in (("runs_check", ["3000"], "0 failures"),
                             ("seqsum_check", [], "all sums bit-identical"),
                             ("exp64_check", [], "0 failures")):
        exe = str(tmp_path / (name + "_san"))
        subprocess.run(["g++", *FLAGS, *SANFLAGS, "-o", exe, os.path.join(HERE, name + ".cpp"), "-lm"],
                       check=True)
        r = subprocess.run([exe, *args], capture_output=True, text=True, timeout=300)
        assert r.returncode == 0 and want in r.stdout, (name, r.stdout[-2000:], r.stderr[-4000:])
    so = str(tmp_path / "libnls_oracle_asan.so")
    subprocess.run(["make", "-s", "-C", os.path.join(os.path.dirname(HERE), "oracle"), "asan",
                    "ASAN_OUT=" + so], check=True)
    env = dict(os.environ, LD_PRELOAD=_san_runtime(), ASAN_OPTIONS="detect_leaks=0",
               NLS_SANITIZE="1", NLS_ORACLE_LIB=so)
    files = ["test_runs_cpu.py", "test_oracle.py", "test_lmhead_oracle.py", "test_expf_mpmath.py"]
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider", "-m", "not gpu",
                        *[os.path.join(HERE, f) for f in files]],
                       capture_output=True, text=True, timeout=900, env=env, cwd=os.path.dirname(HERE))
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-4000:]
    assert " passed" in r.stdout and " failed" not in r.stdout, r.stdout[-2000:]
