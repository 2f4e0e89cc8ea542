"""Benchmark of the MI355X sampler: rows/s and HBM roofline fraction.

One step = one nls_sample call over one batch (penalties -> bias -> temperature
-> top-k -> softmax -> top-p -> min-p -> draw for every row), inputs already
resident in HBM.  The timed region rotates over enough copies of the logits to
exceed the 256 MB Infinity Cache, so every step reads its logits from HBM.

    python bench.py [--steps K] [--warmup W] [--workload headline] [--no-cpu-baseline]

Prints one JSON line.  `roofline` is for the dominant kernel of a call: the
streaming kernel (the single read of the logits, running the whole pipeline
of greedy and top-k rows: k64_kernel for k <= 64 with 1024-thread workgroups,
stream_kernel otherwise) or, when full-sort rows take longer,
the whole-row kernel (generic_kernel).  Each kernel is charged with the
algorithmic bytes of the rows it serves (`kernels` lists both) and timed with
HIP events on the sampler's stream: around K back-to-back calls when a call is
one launch, else around each kernel.  `traffic` comes from the committed
rocprofv3 counter summary (profiles/traffic_<workload>.md) only when that
summary was measured on these sources (a hash of nim.llm_amd/csrc and
include/).  `cpu_baseline` times the CPU restatement of the reference sampler
(oracle/) on one host core, `cpu_baseline_all_cores` on every core this process
may use (at most 16), each on a bounded sample of the same rows.

    python bench.py --traffic-summary --workload W --fetch-dir D1 --write-dir D2 --out F
writes such a summary from two rocprofv3 --pmc runs (no GPU needed).
"""
import argparse
import importlib.util
import json
import math
import os
import platform
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(ROOT, "nim.llm_amd")
HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, GB/s


def load_pkg():
    name = "nimllm_amd"
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, os.path.join(PKG_DIR, "__init__.py"),
                                                  submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


SOURCE_GLOBS = ("nim.llm_amd/csrc/*.hip", "nim.llm_amd/csrc/*.h", "nim.llm_amd/csrc/*.cpp",
                "nim.llm_amd/csrc/Makefile", "include/*.h")


def source_hash():
    """sha256 over the sources of the HIP library: a traffic profile is valid
    only for the code it was measured on."""
    import glob
    import hashlib

    h = hashlib.sha256()
    for pat in SOURCE_GLOBS:
        for f in sorted(glob.glob(os.path.join(ROOT, pat))):
            h.update(os.path.relpath(f, ROOT).encode())
            with open(f, "rb") as fh:
                h.update(fh.read())
    return h.hexdigest()[:16]


def traffic_path(workload):
    return os.path.join(ROOT, "profiles", f"traffic_{workload}.md")


def read_traffic(workload):
    """{kernel: HBM bytes per launch} from the committed rocprofv3 --pmc summary
    (FETCH_SIZE + WRITE_SIZE, copy-kernel scaled), or ({}, reason) when the
    summary is missing or was measured on other sources."""
    path = traffic_path(workload)
    if not os.path.exists(path):
        return {}, "no traffic profile for this workload"
    stamp, out = None, {}
    for line in open(path):
        if line.startswith("source_hash:"):
            stamp = line.split(":", 1)[1].strip()
        elif line.startswith("traffic_bytes_per_launch "):
            k, v = line[len("traffic_bytes_per_launch "):].rsplit(":", 1)
            out[k.strip()] = float(v)
    if stamp != source_hash():
        return {}, f"traffic profile measured on sources {stamp}, not these ({source_hash()})"
    return out, None


def _pmc_rows(d):
    """(kernel name, counter name, value) of every dispatch in a rocprofv3
    --pmc csv output directory."""
    import csv
    import glob

    files = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no *counter_collection.csv under {d}")
    for f in files:
        for r in csv.DictReader(open(f)):
            yield r.get("Kernel_Name", ""), r.get("Counter_Name", ""), float(r.get("Counter_Value", 0)), \
                r.get("Dispatch_Id", "")


def traffic_summary(args):
    """Writes the per-kernel HBM traffic summary of a workload from two
    rocprofv3 --pmc runs of this script (FETCH_SIZE, then WRITE_SIZE, both with
    --copy-ref), scaled by the 256 MiB copy of known size in the same runs."""
    from collections import defaultdict

    per = {}
    for counter, d in (("FETCH_SIZE", args.fetch_dir), ("WRITE_SIZE", args.write_dir)):
        acc = defaultdict(dict)
        for kern, cname, val, disp in _pmc_rows(d):
            if cname != counter:
                continue
            acc[kern][disp] = acc[kern].get(disp, 0.0) + val
        # the reference copies are the run's last three copy dispatches
        # (--copy-ref runs them after everything else); other copies, such as
        # the uploads of the inputs, may be larger and read host memory
        cps = sorted(((int(dd), v) for k, dv in acc.items() if "copyBuffer" in k for dd, v in dv.items()),
                     reverse=True)[:3]
        ref = sum(v for _, v in cps) / len(cps) if len(cps) == 3 else None
        per[counter] = {k: (sum(v.values()) / len(v), len(v), ref) for k, v in acc.items()}
    copy_bytes = 64 * 1024 * 1024 * 4
    copy = [k for k in per["FETCH_SIZE"] if "copyBuffer" in k]
    if not copy or per["FETCH_SIZE"][copy[0]][2] is None:
        raise SystemExit("no reference copies in the FETCH_SIZE run: run bench.py with --copy-ref")
    ck = copy[0]
    f_fac = copy_bytes / (per["FETCH_SIZE"][ck][2] * 1024)
    w_fac = copy_bytes / (per["WRITE_SIZE"][ck][2] * 1024)
    lines = [f"# HBM traffic per launch, workload {args.workload}", "",
             "Two counter passes, each its own run (from the repository root on an MI355X):", "", "```",
             f"cd /tmp && export TMPDIR=/tmp && timeout -s KILL 120 rocprofv3 --pmc FETCH_SIZE -f csv -d <fetch> "
             f"-o pmc -- python3 <repo>/bench.py --workload {args.workload} --steps 10 --warmup 2 "
             f"--no-cpu-baseline --copy-ref",
             f"cd /tmp && export TMPDIR=/tmp && timeout -s KILL 120 rocprofv3 --pmc WRITE_SIZE -f csv -d <write> "
             f"-o pmc -- python3 <repo>/bench.py --workload {args.workload} --steps 10 --warmup 2 "
             f"--no-cpu-baseline --copy-ref",
             f"python3 <repo>/bench.py --traffic-summary --workload {args.workload} --fetch-dir <fetch> "
             f"--write-dir <write> --out <this file>", "```", "",
             f"Scale factors from the run's last three `{ck}` dispatches, the reference copies "
             f"(256 MiB read, 256 MiB written each): "
             f"FETCH_SIZE x {f_fac:.4f}, WRITE_SIZE x {w_fac:.4f}.", "",
             "| Kernel | dispatches | FETCH_SIZE KiB/dispatch | WRITE_SIZE KiB/dispatch | HBM bytes/launch |",
             "|---|---|---|---|---|"]
    totals = {}
    for k, (fv, n, _) in sorted(per["FETCH_SIZE"].items()):
        if "copyBuffer" in k or "fillBuffer" in k or k.startswith("at::") or "at::native" in k:
            continue
        wv = per["WRITE_SIZE"].get(k, (0.0, 0, 0.0))[0]
        b = fv * 1024 * f_fac + wv * 1024 * w_fac
        short = k.split("(")[0].replace("void ", "").replace("nls::", "")
        base = short.split("<")[0]
        totals[base] = max(totals.get(base, 0.0), b)
        lines.append(f"| `{short}` | {n} | {fv:.2f} | {wv:.2f} | {b:.0f} |")
    lines += ["", f"source_hash: {source_hash()}", f"commit: {args.commit or 'unknown'}"]
    for base, b in sorted(totals.items()):
        lines.append(f"traffic_bytes_per_launch {base}: {b:.0f}")
    with open(args.out, "w") as f:
        f.write("\n".join(lines) + "\n")
    print("\n".join(lines))


def trace_summary(args):
    """Per-kernel launch durations from a rocprofv3 --kernel-trace run of this
    script (the kernel_trace.csv under --trace-dir): every launch but each
    kernel's first --skip (the parity check and the warmup, whose first
    launches run cold), as median, mean, 10th and 90th percentile.  Prints
    one JSON line."""
    import csv
    import glob
    from collections import defaultdict

    files = glob.glob(os.path.join(args.trace_dir, "**", "*kernel_trace.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no kernel_trace.csv under {args.trace_dir}")
    runs = defaultdict(list)
    for f in files:
        with open(f, newline="") as fh:
            for r in csv.DictReader(fh):
                name = r["Kernel_Name"]
                runs[name].append((int(r["Dispatch_Id"]), (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3))
    out = {}
    for name, v in runs.items():
        if "copyBuffer" in name or "fillBuffer" in name or name.startswith("at::") or "at::native" in name:
            continue
        v.sort()
        d = sorted(x for _, x in v[args.skip:]) or sorted(x for _, x in v)
        n = len(d)
        short = name.split("(")[0].replace("void ", "").replace("nls::", "")
        out[short] = {"launches": len(v), "kept": n, "median_us": d[n // 2], "mean_us": sum(d) / n,
                      "p10_us": d[n // 10], "p90_us": d[(9 * n) // 10]}
    print(json.dumps({"workload": args.workload, "skip": args.skip, "kernels": out}), flush=True)


def copy_ref(dev):
    """A plain 256 MiB device copy, three times: the kernel of known size that
    scales rocprofv3 FETCH_SIZE / WRITE_SIZE to bytes."""
    import torch

    n = 64 * 1024 * 1024  # 64 Mi floats = 256 MiB read and 256 MiB written per copy
    a = torch.empty(n, dtype=torch.float32, device=dev).fill_(1.0)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    del a, b
    return n * 4


def host_cores():
    """Cores this process may use, capped at the 16 a one-GPU box grants."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, 16))


def cpu_baseline(w, budget_s=12.0, nthreads=1):
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import oracle as O

    params = [O.make_params(**r.as_kwargs()) for r in w.rows]
    bid, bval, bcnt = w.bias_arrays()
    hl = np.full(w.B, w.hist.shape[1], dtype=np.int64)
    hist = w.hist if w.hist.shape[1] else None
    rows_done = 0
    t0 = time.perf_counter()
    # rows split in contiguous blocks over the threads: a chunk gives each
    # thread several rows
    chunk = max(1, min(w.B, 64)) if nthreads == 1 else max(nthreads, min(w.B, 8 * nthreads))
    start = 0
    while time.perf_counter() - t0 < budget_s:
        rows = np.arange(start, start + chunk) % w.B
        O.sample_batch([params[r] for r in rows], w.logits[rows],
                       None if hist is None else hist[rows], hl[rows], bid[rows], bval[rows],
                       bcnt[rows], w.u[rows], O.EXPF_LIBM, nthreads=nthreads)
        rows_done += chunk
        start = (start + chunk) % w.B
    dt = time.perf_counter() - t0
    glibc = platform.libc_ver()
    cpu = platform.processor() or platform.machine()
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    how = ("rows run serially on one thread" if nthreads == 1 else
           f"rows split over {nthreads} threads (POSIX threads, contiguous blocks of {chunk // nthreads}+ rows)")
    return {"value": rows_done / dt, "unit": "rows/s", "cores": nthreads, "kind": "port",
            "sample": f"{rows_done} rows of the same workload ({w.name}), {how} for {dt:.1f} s; "
                      f"C restatement of src/nimllm/sampler.nim:59-121 "
                      f"(-O2 -ffp-contract=off, libm expf); CPU: {cpu}; "
                      f"{glibc[0]} {glibc[1]}"}


def bench_top_tokens(args):
    """topTokens (sampler.nim:123-130) on the headline logits: n = 5 per row.
    One line of JSON like the sampler's, for this entry point."""
    import ctypes
    import numpy as np
    import torch

    pkg = load_pkg()
    from nimllm_amd import workloads

    w = workloads.make(args.workload, seed=args.seed)
    B, V, n = w.B, w.V, args.top_n
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    nbuf = max(2, math.ceil(640e6 / (B * V * 4)))
    base = torch.from_numpy(w.logits).to(dev)
    bufs = [base] + [base.clone() for _ in range(nbuf - 1)]
    ids, pr = pkg.top_tokens_device(bufs[0], n)
    torch.cuda.synchronize()
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    ok = True
    for r in (0, B // 2, B - 1):
        wi = np.zeros(n, dtype=np.int64)
        wp = np.zeros(n, dtype=np.float32)
        x = np.ascontiguousarray(w.logits[r])
        O.lib().nlo_top_tokens(x.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), V, n, O.EXPF_CR,
                               wi.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)),
                               wp.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
        ok &= bool(np.array_equal(ids[r].cpu().numpy(), wi)) and bool(
            np.array_equal(pr[r].cpu().numpy().view(np.uint32), wp.view(np.uint32)))
    for i in range(args.warmup):
        pkg.top_tokens_device(bufs[i % nbuf], n)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for i in range(args.steps):
        pkg.top_tokens_device(bufs[i % nbuf], n)
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    nbytes = float(B * V * 4 + B * n * 8)  # logits once, ids and probabilities out
    achieved = nbytes / (ms * 1e-3) / 1e9
    # the reference's sum is V dependent fp32 adds per row: one lane adding them
    # one at a time issues one every 4 cycles (a wave64 VALU instruction) at the
    # 2.4 GHz peak engine clock; the kernel evaluates the same sum in parallel
    chain_us = V * 4 / 2.4e3
    res = {"metric": f"topTokens rows/sec at B={B} x V={V} fp32, n={n}", "value": B / (ms * 1e-3),
           "unit": "rows/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
           "dtype": "f32", "data": "synthetic (the sampler workload's logits, rotated over "
                                   f"{nbuf} buffers)",
           "config": {"workload": f"{args.workload} logits, topTokens n={n}", "B": B, "V": V},
           "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": achieved / HBM_PEAK_GBS, "traffic": None,
                        "kernel": "top_tokens_kernel", "kernel_avg_us": ms * 1e3,
                        "algorithmic_bytes_per_launch": nbytes,
                        "single_lane_sum_chain_us": chain_us},
           "parity_spot_check": {"rows": 3, "bit_exact": ok}}
    if not args.no_cpu_baseline:
        t0 = time.perf_counter()
        done = 0
        wi = np.zeros(n, dtype=np.int64)
        wp = np.zeros(n, dtype=np.float32)
        while time.perf_counter() - t0 < args.cpu_budget:
            x = np.ascontiguousarray(w.logits[done % B])
            O.lib().nlo_top_tokens(x.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), V, n, O.EXPF_LIBM,
                                   wi.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)),
                                   wp.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
            done += 1
        dt = time.perf_counter() - t0
        res["cpu_baseline"] = {"value": done / dt, "unit": "rows/s", "cores": 1, "kind": "port",
                               "sample": f"{done} rows on one thread for {dt:.1f} s; C restatement of "
                                         "src/nimllm/sampler.nim:123-130 (softmaxInPlace, stable "
                                         "merge sort; -O2 -ffp-contract=off, libm expf)"}
    else:
        res["cpu_baseline"] = None
    print(json.dumps(res), flush=True)


def bench_row_nll(args):
    """perplexity's per-position term (model.nim:578-583) on the workload's
    logits, one random target id per row.  One line of JSON like the
    sampler's, for this entry point."""
    import numpy as np
    import torch

    pkg = load_pkg()
    from nimllm_amd import workloads

    w = workloads.make(args.workload, seed=args.seed)
    B, V = w.B, w.V
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    nbuf = max(2, math.ceil(640e6 / (B * V * 4)))
    base = torch.from_numpy(w.logits).to(dev)
    bufs = [base] + [base.clone() for _ in range(nbuf - 1)]
    rng = np.random.default_rng(args.seed)
    tgt = torch.from_numpy(rng.integers(0, V, size=B).astype(np.int32)).to(dev)
    out = pkg.row_nll_device(bufs[0], tgt).cpu().numpy()
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    ok = True
    for r in (0, B // 2, B - 1):
        ref = O.row_nll(w.logits[r], int(tgt[r]))
        ok &= bool(abs(out[r] - ref) <= 1e-12 * max(1.0, abs(ref)))
    for i in range(args.warmup):
        pkg.row_nll_device(bufs[i % nbuf], tgt)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for i in range(args.steps):
        pkg.row_nll_device(bufs[i % nbuf], tgt)
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    nbytes = float(B * V * 4 + B * 12)  # logits once, the target and the float64 result
    achieved = nbytes / (ms * 1e-3) / 1e9
    res = {"metric": f"perplexity terms (rows/sec) at B={B} x V={V} fp32", "value": B / (ms * 1e-3),
           "unit": "rows/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
           "dtype": "f32 logits, f64 sum", "data": "synthetic (the sampler workload's logits, rotated over "
                                                   f"{nbuf} buffers; random targets)",
           "config": {"workload": f"{args.workload} logits, row_nll", "B": B, "V": V},
           "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": achieved / HBM_PEAK_GBS, "traffic": None, "kernel": "row_nll_kernel",
                        "kernel_avg_us": ms * 1e3, "algorithmic_bytes_per_launch": nbytes},
           "parity_spot_check": {"rows": 3, "within_1e-12": ok}}
    if not args.no_cpu_baseline:
        t0 = time.perf_counter()
        done = 0
        while time.perf_counter() - t0 < args.cpu_budget:
            O.row_nll(w.logits[done % B], int(tgt[done % B]))
            done += 1
        dt = time.perf_counter() - t0
        res["cpu_baseline"] = {"value": done / dt, "unit": "rows/s", "cores": 1, "kind": "port",
                               "sample": f"{done} rows on one thread for {dt:.1f} s; C restatement of "
                                         "src/nimllm/model.nim:578-583 (-O2 -ffp-contract=off, libm exp/log)"}
    else:
        res["cpu_baseline"] = None
    print(json.dumps(res), flush=True)


def bench_softmax(args, logp):
    """softmaxInPlace (sampler.nim:51-57) over whole rows of the workload's
    logits (nls_softmax_rows), or logProb's per-token term with one random
    target per row (nls_log_prob).  One line of JSON like the sampler's."""
    import numpy as np
    import torch

    pkg = load_pkg()
    from nimllm_amd import workloads

    w = workloads.make(args.workload, seed=args.seed)
    B, V = w.B, w.V
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    nbuf = max(2, math.ceil(640e6 / (B * V * 4)))
    base = torch.from_numpy(w.logits).to(dev)
    bufs = [base] + [base.clone() for _ in range(nbuf - 1)]
    out = torch.empty_like(base)
    rng = np.random.default_rng(args.seed)
    tgt = torch.from_numpy(rng.integers(0, V, size=B).astype(np.int32)).to(dev)

    def call(x):
        if logp:
            return pkg.log_prob_device(x, tgt)
        return pkg.softmax_device(x, out)

    res0 = call(bufs[0])
    torch.cuda.synchronize()
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    ok = True
    for r in (0, B // 2, B - 1):
        if logp:
            wp, _ = O.log_prob(w.logits[r], int(tgt[r]))
            ok &= bool(res0[0][r].cpu().numpy().view(np.uint32) == wp.view(np.uint32))
        else:
            ok &= bool(np.array_equal(out[r].cpu().numpy().view(np.uint32),
                                      O.softmax(w.logits[r]).view(np.uint32)))
    for i in range(args.warmup):
        call(bufs[i % nbuf])
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for i in range(args.steps):
        call(bufs[i % nbuf])
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    # logits read once; softmax writes every probability, logProb a target,
    # a float32 and a float64 per row
    nbytes = float(B * V * 4 + (B * V * 4 if not logp else B * 16))
    achieved = nbytes / (ms * 1e-3) / 1e9
    name = "logProb terms" if logp else "softmaxInPlace rows"
    kern = "softmax_kernel<true>" if logp else "softmax_kernel<false>"
    res = {"metric": f"{name} (rows/sec) at B={B} x V={V} fp32", "value": B / (ms * 1e-3),
           "unit": "rows/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
           "dtype": "f32", "data": "synthetic (the sampler workload's logits, rotated over "
                                   f"{nbuf} buffers" + ("; random targets)" if logp else ")"),
           "config": {"workload": f"{args.workload} logits, {'nls_log_prob' if logp else 'nls_softmax_rows'}",
                      "B": B, "V": V},
           "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": achieved / HBM_PEAK_GBS, "traffic": None, "kernel": kern,
                        "kernel_avg_us": ms * 1e3, "algorithmic_bytes_per_launch": nbytes},
           "parity_spot_check": {"rows": 3, "bit_exact": ok}}
    if not args.no_cpu_baseline:
        t0 = time.perf_counter()
        done = 0
        while time.perf_counter() - t0 < args.cpu_budget:
            r = done % B
            if logp:
                O.log_prob(w.logits[r], int(tgt[r]), O.EXPF_LIBM)
            else:
                O.softmax(w.logits[r], O.EXPF_LIBM)
            done += 1
        dt = time.perf_counter() - t0
        res["cpu_baseline"] = {"value": done / dt, "unit": "rows/s", "cores": 1, "kind": "port",
                               "sample": f"{done} rows on one thread for {dt:.1f} s; C restatement of "
                                         "src/nimllm/sampler.nim:51-57 (-O2 -ffp-contract=off, libm expf"
                                         + (", log)" if logp else ")")}
    else:
        res["cpu_baseline"] = None
    print(json.dumps(res), flush=True)


def bench_lm_head(args):
    """The output projection (nls_lm_head, matmul(m.output, x, y, nb),
    src/nimllm/model.nim:179-200) on synthetic GGUF rows: one step = one call
    writing nb x rows logits.  The weight matrix is rotated over copies that
    together exceed the Infinity Cache.  Roofline: the weight bytes plus x and
    y, over the kernel time."""
    import threading

    import numpy as np
    import torch

    pkg = load_pkg()
    from nimllm_amd import workloads

    t = workloads.LM_TYPE_NAMES[args.lm_type]
    rows, cols, nb = args.lm_rows, args.lm_cols, args.lm_nb
    w_np = workloads.make_lm_weights(t, rows, cols, seed=args.seed)
    x_np = workloads.make_lm_hidden(nb, cols, seed=args.seed)
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    wbytes = w_np.nbytes
    nbuf = max(2, math.ceil(640e6 / wbytes))
    base = torch.from_numpy(w_np).to(dev)
    bufs = [base] + [base.clone() for _ in range(nbuf - 1)]
    x = torch.from_numpy(x_np).to(dev)
    y = torch.empty((nb, rows), dtype=torch.float32, device=dev)
    work = torch.empty(max(1, pkg.lm_head_workspace(t, cols, nb, 0, args.lm_exact)), dtype=torch.uint8,
                       device=dev)

    def call(wb):
        pkg.lm_head(wb, t, rows, cols, x, exact=args.lm_exact, out=y, work=work)

    call(bufs[0])
    torch.cuda.synchronize()
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    # parity spot check: the first and the last 512 rows against the oracle
    got = y.cpu().numpy()
    ok = True
    for lo, hi in ((0, min(rows, 512)), (max(0, rows - 512), rows)):
        ref = O.matmul(t, w_np, rows, cols, x_np, exact=args.lm_exact, first=lo, last=hi)
        ok &= bool(np.array_equal(got[:, lo:hi].view(np.uint32), ref[:, lo:hi].view(np.uint32)))
    for i in range(args.warmup):
        call(bufs[i % nbuf])
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for i in range(args.steps):
        call(bufs[i % nbuf])
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    nbytes = float(wbytes + nb * cols * 4 + nb * rows * 4)
    achieved = nbytes / (ms * 1e-3) / 1e9
    path = "int8 activations" if O.matmul_uses_act(t, cols, nb, args.lm_exact) else "dequantise + dotF32"
    if path != "int8 activations":
        kern = "lm_float_kernel"
    elif nb == 1 and (cols // 32 + 63) // 64 <= 4:
        kern = "lm_int1_kernel (activations quantised in the kernel)"
    else:
        kern = "quant_act_kernel + lm_int_kernel"
    res = {"metric": f"LM head calls/sec ({rows} x {cols} {args.lm_type}, nb={nb})",
           "value": 1e3 / ms, "unit": "calls/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
           "dtype": "int8 x int8 -> int32, fp32 terms" if path == "int8 activations" else "f32",
           "data": f"synthetic GGUF rows (random blocks, finite scales), rotated over {nbuf} copies",
           "config": {"workload": f"output projection {rows} x {cols} {args.lm_type}, {path}",
                      "rows": rows, "cols": cols, "nb": nb, "exact": bool(args.lm_exact)},
           "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": achieved / HBM_PEAK_GBS, "traffic": None, "kernel": kern,
                        "kernel_avg_us": ms * 1e3, "algorithmic_bytes_per_launch": nbytes},
           "parity_spot_check": {"rows": 1024, "bit_exact": ok}}
    if (t, rows, cols, nb, bool(args.lm_exact)) == (14, 128256, 2048, 1, False):
        traffic, why = read_traffic("lm_head_q6k")
        if traffic.get("lm_int1_kernel"):
            res["roofline"]["traffic"] = traffic["lm_int1_kernel"]
        else:
            res["roofline"]["traffic_note"] = why or "no lm_int1_kernel line"
    if args.copy_ref:
        res["copy_ref_bytes"] = copy_ref(dev)
    if not args.no_cpu_baseline:
        def run(nthreads, budget):
            # rows in chunks of 256 per thread until the budget is spent
            done = [0] * nthreads
            t0 = time.perf_counter()

            def worker(k):
                r = (k * 7919 * 256) % rows
                while time.perf_counter() - t0 < budget:
                    hi = min(rows, r + 256)
                    O.matmul(t, w_np, rows, cols, x_np, exact=args.lm_exact, first=r, last=hi)
                    done[k] += hi - r
                    r = hi % rows
            ths = [threading.Thread(target=worker, args=(k,)) for k in range(nthreads)]
            for th in ths:
                th.start()
            for th in ths:
                th.join()
            dt = time.perf_counter() - t0
            return sum(done), dt

        n1, dt1 = run(1, args.cpu_budget / 2)
        res["cpu_baseline"] = {"value": n1 / rows / dt1, "unit": "calls/s", "cores": 1, "kind": "port",
                               "sample": f"{n1} of the {rows} rows in {dt1:.1f} s on one thread, scaled to a "
                                         "whole call; C restatement of model.nim:144-200 with "
                                         "quant.nim:164-798 (-O2 -ffp-contract=off)"}
        nt = host_cores()
        nn, dtn = run(nt, args.cpu_budget / 2)
        res["cpu_baseline_all_cores"] = {"value": nn / rows / dtn, "unit": "calls/s", "cores": nt,
                                         "kind": "port",
                                         "sample": f"{nn} rows in {dtn:.1f} s over {nt} threads (rows in "
                                                   "chunks of 256, as parallelFor splits them)"}
    else:
        res["cpu_baseline"] = None
    print(json.dumps(res), flush=True)


def bench_sample_host(args):
    """nls_sample_host end to end -- the Nim drop-in's path (host logits in,
    a host id out: the copy to the device, the sampler, the copy back and the
    synchronisation) -- and its no-allocation variant, on the workload's rows
    one call at a time, beside the CPU restatement of the same rows.  One
    line of JSON like the sampler's."""
    import numpy as np
    import torch

    pkg = load_pkg()
    from nimllm_amd import workloads

    w = workloads.make(args.workload, seed=args.seed)
    B, V = w.B, w.V
    torch.cuda.init()
    s = pkg.BatchSampler(workloads.sampler_params(w, pkg), V)
    if w.hist.shape[1]:
        s.accept(w.hist)
    x = np.ascontiguousarray(w.logits)
    noalloc = B * V * 4 + B * 4 + 256 <= 16 << 20
    times = {}
    for name, fn in (("nls_sample_host", s.sample_host),
                     ("nls_sample_host_noalloc", s.sample_host_noalloc if noalloc else None)):
        if fn is None:
            continue
        for _ in range(args.warmup):
            fn(x)
        t = []
        for _ in range(args.steps):
            t0 = time.perf_counter()
            fn(x)
            t.append(time.perf_counter() - t0)
        t.sort()
        times[name] = {"median_us": t[len(t) // 2] * 1e6, "p10_us": t[len(t) // 10] * 1e6,
                       "p90_us": t[(9 * len(t)) // 10] * 1e6}
    s.close()
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    bid, bval, bcnt = w.bias_arrays()
    plist = [O.make_params(**r.as_kwargs()) for r in w.rows]
    hl = np.full(B, w.hist.shape[1])
    hist = w.hist if w.hist.shape[1] else None
    t = []
    for _ in range(max(5, min(args.steps, 50))):
        t0 = time.perf_counter()
        O.sample_batch(plist, x, hist, hl, bid, bval, bcnt, w.u, O.EXPF_LIBM, nthreads=1)
        t.append(time.perf_counter() - t0)
    t.sort()
    cpu_us = t[len(t) // 2] * 1e6
    med = times["nls_sample_host"]["median_us"]
    res = {"metric": f"nls_sample_host end to end (us per call) at B={B} x V={V}", "value": med,
           "unit": "us", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": med / 1e3,
           "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
           "data": "synthetic (seeded numpy logits in host memory, one blocking call at a time)",
           "config": {"workload": workloads.describe(args.workload, B, V), "B": B, "V": V}, "calls": times,
           "cpu_baseline": {"value": cpu_us, "unit": "us per call", "cores": 1, "kind": "port",
                            "sample": f"median of the same {B}-row call on one thread; C restatement of "
                                      "src/nimllm/sampler.nim:59-121 (libm expf)"}}
    print(json.dumps(res), flush=True)


def bench_decode_chain(args):
    """One decode step's tail on the device, per token, at the output shape of
    --lm-rows x --lm-cols (--lm-type; Llama-3.2-1B's 128256 x 2048 by
    default): the normalised hidden state from host memory to the device,
    the output projection (nls_lm_head, model.nim:470), the sampler
    (nls_sample, chat.nim:205) writing the id into pinned host memory, and one
    synchronisation -- beside the CPU restatement's matmul + sample of the same
    step.  Also timed: the same chain with the acceptance on the device
    (nls_generate_step, chat.nim:205-208) and the id copied back."""
    import ctypes

    import numpy as np
    import torch

    pkg = load_pkg()
    from nimllm_amd import workloads

    L = pkg.lib()
    t = workloads.LM_TYPE_NAMES[args.lm_type]
    rows, cols = args.lm_rows, args.lm_cols
    w_np = workloads.make_lm_weights(t, rows, cols, seed=args.seed)
    xs = workloads.make_lm_hidden(args.steps + args.warmup + 1, cols, seed=args.seed)
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    nbuf = max(2, math.ceil(640e6 / w_np.nbytes))
    base = torch.from_numpy(w_np).to(dev)
    bufs = [base] + [base.clone() for _ in range(nbuf - 1)]
    x_pin = torch.empty(cols, dtype=torch.float32).pin_memory()
    x_dev = torch.empty((1, cols), dtype=torch.float32, device=dev)
    y = torch.empty((1, rows), dtype=torch.float32, device=dev)
    work = torch.empty(max(1, pkg.lm_head_workspace(t, cols, 1, 0, False)), dtype=torch.uint8, device=dev)
    id_pin = torch.zeros(1, dtype=torch.int32).pin_memory()
    params = pkg.defaultSampling()
    params.seed = args.seed
    hist = np.arange(64, dtype=np.int64).reshape(1, 64) * 997 % rows
    s = pkg.BatchSampler([params], rows, stream=stream)
    s.accept(hist)
    d_id = torch.empty(1, dtype=torch.int32, device=dev)
    eog = torch.tensor([rows + 1], dtype=torch.int32, device=dev)  # no end-of-generation id is drawn
    done = torch.zeros(1, dtype=torch.int32, device=dev)

    def step(i, accept):
        x_pin.numpy()[:] = xs[i]
        x_dev.copy_(x_pin.reshape(1, cols), non_blocking=True)
        pkg.lm_head(bufs[i % nbuf], t, rows, cols, x_dev, out=y, work=work)
        if accept:
            s.generate_step(y, eog, done, out=d_id)
            id_pin.copy_(d_id, non_blocking=True)
            stream.synchronize()
        else:
            pkg.check(L.nls_sample(s._h, ctypes.c_void_p(y.data_ptr()), None,
                                   ctypes.c_void_p(id_pin.data_ptr()), None), "nls_sample")
            s.synchronize()
        return int(id_pin.numpy()[0])

    # parity: the first step's id against the oracle's matmul + sample with the
    # same first uniform of initRand(seed)
    first = step(0, False)
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    logits = O.matmul(t, w_np, rows, cols, xs[0:1])[0]
    op = O.make_params(temperature=params.temperature, topK=params.topK, topP=params.topP, minP=params.minP,
                       repeatPenalty=params.repeatPenalty, repeatLastN=params.repeatLastN,
                       presencePenalty=params.presencePenalty, frequencyPenalty=params.frequencyPenalty,
                       seed=params.seed)
    res, _, _, _ = O.sample(op, logits, hist[0], {}, float(O.uniforms(args.seed, 1)[0]), O.EXPF_CR,
                            want_cand=False)
    parity = first == res.id

    def timed(accept):
        for i in range(args.warmup):
            step(1 + i, accept)
        ts = []
        for i in range(args.steps):
            t0 = time.perf_counter()
            step(1 + args.warmup + i, accept)
            ts.append(time.perf_counter() - t0)
        ts.sort()
        return {"median_us": ts[len(ts) // 2] * 1e6, "p10_us": ts[len(ts) // 10] * 1e6,
                "p90_us": ts[(9 * len(ts)) // 10] * 1e6}

    sample_only = timed(False)
    with_accept = timed(True)
    s.close()
    med = sample_only["median_us"]
    res_line = {
        "metric": f"decode-step tail per token: hidden state in, {rows} x {cols} {args.lm_type} output "
                  "projection, sampler, id out (us per token)",
        "value": med, "unit": "us", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": med / 1e3, "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8 x int8 -> int32, fp32 terms; f32 sampler",
        "data": f"synthetic GGUF rows rotated over {nbuf} copies; one fresh hidden state per step",
        "config": {"workload": f"decode tail at the Llama-3.2-1B output shape {rows} x {cols} {args.lm_type}, "
                               "B=1, defaultSampling (T 0.7, top-k 40, top-p 0.95, min-p 0.05, repeat "
                               "penalty 1.1 over the last 64 ids)", "rows": rows, "cols": cols},
        "chain": {"sample_id_to_pinned_host": sample_only, "generate_step_id_copied_back": with_accept},
        "parity_first_step": {"bit_exact_id": bool(parity), "id": first, "oracle_id": int(res.id)},
    }
    if not args.no_cpu_baseline:
        def cpu_step(nthreads):
            import threading

            t0 = time.perf_counter()
            out = np.zeros((1, rows), np.float32)
            bounds = [rows * k // nthreads for k in range(nthreads + 1)]

            def worker(k):
                out[:, bounds[k]:bounds[k + 1]] = O.matmul(t, w_np, rows, cols, xs[1:2], first=bounds[k],
                                                           last=bounds[k + 1])[:, bounds[k]:bounds[k + 1]]
            ths = [threading.Thread(target=worker, args=(k,)) for k in range(nthreads)]
            for th in ths:
                th.start()
            for th in ths:
                th.join()
            t1 = time.perf_counter()
            O.sample(op, out[0], hist[0], {}, 0.5, O.EXPF_LIBM, want_cand=False)
            t2 = time.perf_counter()
            return (t2 - t0) * 1e6, (t2 - t1) * 1e6

        nt = host_cores()
        reps = [cpu_step(nt) for _ in range(3)]
        tot = sorted(r[0] for r in reps)[1]
        smp = sorted(r[1] for r in reps)[1]
        one = cpu_step(1)
        res_line["cpu_baseline"] = {"value": one[0], "unit": "us per token", "cores": 1, "kind": "port",
                                    "sample": f"one step on one thread (matmul {one[0] - one[1]:.0f} us + sample "
                                              f"{one[1]:.0f} us); C restatement of model.nim:144-200 and "
                                              "sampler.nim:59-121"}
        res_line["cpu_baseline_all_cores"] = {"value": tot, "unit": "us per token", "cores": nt, "kind": "port",
                                              "sample": f"median of 3 steps, matmul over {nt} threads (row "
                                                        f"ranges, as parallelFor splits them), sample "
                                                        f"{smp:.0f} us on one"}
    else:
        res_line["cpu_baseline"] = None
    print(json.dumps(res_line), flush=True)


def phase_stamps(args):
    """Per-phase wall-clock of the k64 kernel on the workload, from the
    `phases` build of the library, which this builds from the sources first
    (make -C nim.llm_amd/csrc phases: only what changed is rebuilt): medians
    over the rows' workgroups of the time each phase took, for the last of a
    run of back-to-back calls.  The output names the sources' hash."""
    import ctypes
    import numpy as np
    import torch

    import glob

    path = os.path.join(PKG_DIR, "libnimllm_sampler_phases.so")
    newest = max(os.path.getmtime(f) for pat in SOURCE_GLOBS for f in glob.glob(os.path.join(ROOT, pat)))
    if not os.path.exists(path) or os.path.getmtime(path) < newest:
        subprocess.run(["make", "-s", "-j16", "-C", os.path.join(PKG_DIR, "csrc"), "phases"], check=True,
                       stdout=subprocess.DEVNULL)
    pkg = load_pkg()
    pkg.LIB_PATH = path
    print(f"# sources: source_hash {source_hash()} (the phases build of these sources)")
    L = pkg.lib()
    from nimllm_amd import workloads

    w = workloads.make(args.workload, seed=args.seed)
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    s = pkg.BatchSampler(workloads.sampler_params(w, pkg), w.V, stream=stream)
    if w.hist.shape[1]:
        s.accept(w.hist)
    nbuf = max(2, math.ceil(640e6 / (w.B * w.V * 4)))
    base = torch.from_numpy(w.logits).to(dev)
    bufs = [base] + [base.clone() for _ in range(nbuf - 1)]
    du = torch.from_numpy(w.u).to(dev)
    out = torch.empty(w.B, dtype=torch.int32, device=dev)
    for i in range(args.steps):
        s.sample(bufs[i % nbuf], du, out)
    torch.cuda.synchronize()
    buf = np.zeros(4096 * 16, dtype=np.uint64)
    st = {}
    for which in (0, 1, 2):
        if L.nls_phase_stamps(which, buf.ctypes.data_as(ctypes.c_void_p)) != 0:
            raise SystemExit("nls_phase_stamps failed")
        st[which] = buf.reshape(4096, 16)[:w.B].astype(np.int64).copy()
    buf[:] = 0
    if L.nls_generic_stamps(buf.ctypes.data_as(ctypes.c_void_p)) != 0:
        raise SystemExit("nls_generic_stamps failed")
    G = buf.reshape(4096, 16)[:w.B].astype(np.int64).copy()
    plan, _ = s.plan()
    s.close()
    if plan.floor_slices > 0:
        # floor_kernel, by workgroup (row * S + slice): 0 start, 1 row constants,
        # 2 patch table, 3 slice maximum, 4 kept values, 5 published; the
        # merging workgroup 6 records read, 7 merged, 8 sorted, 9 tail, 10 the
        # values merged
        S = plan.floor_slices
        buf[:] = 0
        if L.nls_floor_stamps(buf.ctypes.data_as(ctypes.c_void_p)) != 0:
            raise SystemExit("nls_floor_stamps failed")
        F = buf.reshape(4096, 16)[:w.B * S].astype(np.int64).copy()
        ok = (F[:, 0] > 0) & (F[:, 5] > 0)
        mg = ok & (F[:, 9] > 0) & (F[:, 9] > F[:, 5])
        t0 = F[ok, 0].min()
        us = lambda d: d / 100.0  # 100 MHz counter
        rows = {"workgroup start after the first": us(F[:, 0] - t0),
                "row constants in": us(F[:, 1] - F[:, 0]),
                "patch table": us(F[:, 2] - F[:, 1]),
                "slice maximum (slice in)": us(F[:, 3] - F[:, 2]),
                "kept values": us(F[:, 4] - F[:, 3]),
                "published, arrival counted": us(F[:, 5] - F[:, 4]),
                "slice total": us(F[:, 5] - F[:, 0])}
        print(f"# floor_kernel phases, workload {args.workload} (B={w.B} V={w.V}, {S} slices per row), "
              f"last of {args.steps} calls; {int(ok.sum())} workgroups, {int(mg.sum())} merges")
        print("| Phase | median us | p10 | p90 |")
        print("|---|---|---|---|")
        for name, v in rows.items():
            v = v[ok]
            print(f"| {name} | {np.median(v):.2f} | {np.percentile(v, 10):.2f} | {np.percentile(v, 90):.2f} |")
        mrows = {"merge: slice records read": us(F[:, 6] - F[:, 5]),
                 "merge: values gathered": us(F[:, 7] - F[:, 6]),
                 "merge: sort": us(F[:, 8] - F[:, 7]),
                 "merge: softmax, top-p, min-p, draw": us(F[:, 9] - F[:, 8]),
                 "merging workgroup total": us(F[:, 9] - F[:, 0])}
        for name, v in mrows.items():
            v = v[mg]
            print(f"| {name} | {np.median(v):.2f} | {np.percentile(v, 10):.2f} | {np.percentile(v, 90):.2f} |")
        print(f"values merged per row (median / max): {np.median(F[mg, 10]):.0f} / {F[mg, 10].max()}")
        print(f"kernel span (first start to last end): {us(F[mg, 9].max() - t0):.2f} us")
        return
    if not plan.k64:
        # stream_kernel rows (each instance's unit keeps its own stamps): 0
        # start, 1 stream start, 2 stream end, 3 members start, 4 members
        # done, 5 tail start, 6 tail done; 7 ticks waiting for a unit's
        # data, 11 ticks at the tile barriers (block path); 12 candidates, 13
        # threshold refreshes, 14 their ticks, 15 tiles
        vec = "true" if w.V % 4 == 0 else "false"
        fn = getattr(L, f"nls_stream_stamps_{plan.stream_threads}_{vec}")
        buf[:] = 0
        if fn(buf.ctypes.data_as(ctypes.c_void_p)) != 0:
            raise SystemExit("nls_stream_stamps failed")
        P = buf.reshape(4096, 16)[:w.B].astype(np.int64).copy()
        ok = (P[:, 0] > 0) & (P[:, 6] > 0)
        if not ok.any():
            print(f"# no stream_kernel rows with every stamp in workload {args.workload}")
            return
        us = lambda d: d / 100.0  # 100 MHz counter
        t0 = P[ok, 0].min()
        rows = {"workgroup start after the first": us(P[:, 0] - t0),
                "prologue: row constants, patch table": us(P[:, 1] - P[:, 0]),
                "stream": us(P[:, 2] - P[:, 1]),
                "  of which threshold refreshes": us(P[:, 14]),
                "  of which waiting for a unit's data": us(P[:, 7]),
                "  of which at the tile barriers (block path)": us(P[:, 11]),
                "patched values, candidates": us(P[:, 3] - P[:, 2]),
                "heap-rule members": us(P[:, 4] - P[:, 3]),
                "sort of the members": us(P[:, 5] - P[:, 4]),
                "tail: softmax, top-p, min-p, draw": us(P[:, 6] - P[:, 5]),
                "workgroup total": us(P[:, 6] - P[:, 0])}
        print(f"# stream_kernel phases, workload {args.workload} (B={w.B} V={w.V}), last of {args.steps} calls; "
              f"{int(ok.sum())} rows with every stamp")
        print("| Phase | median us | p10 | p90 |")
        print("|---|---|---|---|")
        for name, v in rows.items():
            v = v[ok]
            print(f"| {name} | {np.median(v):.2f} | {np.percentile(v, 10):.2f} | {np.percentile(v, 90):.2f} |")
        print(f"per row (median / p90): tiles {np.median(P[ok, 15]):.0f} / {np.percentile(P[ok, 15], 90):.0f}; "
              f"threshold refreshes {np.median(P[ok, 13]):.0f} / {np.percentile(P[ok, 13], 90):.0f}; "
              f"candidates {np.median(P[ok, 12]):.0f} / {np.percentile(P[ok, 12], 90):.0f}")
        print(f"kernel span (first start to last end): {us(P[ok, 6].max() - t0):.2f} us")
        return
    gok = (G[:, 0] > 0) & (G[:, 7] > 0)
    if gok.any():
        g0 = G[gok, 0].min()
        grows = {
            "start after the first grouped row": (G[:, 0] - g0) / 100.0,
            "zero tables, patch table": (G[:, 1] - G[:, 0]) / 100.0,
            "pass 1: row maximum": (G[:, 2] - G[:, 1]) / 100.0,
            "pass 2: count distinct values": (G[:, 3] - G[:, 2]) / 100.0,
            "sort the groups": (G[:, 4] - G[:, 3]) / 100.0,
            "softmax sum over groups": (G[:, 5] - G[:, 4]) / 100.0,
            "top-p / min-p / draw over groups": (G[:, 6] - G[:, 5]) / 100.0,
            "pass 3: the drawn member": (G[:, 7] - G[:, 6]) / 100.0,
            "row total": (G[:, 7] - G[:, 0]) / 100.0,
        }
        if plan.walk_split:
            # three launches: the groups stored (slots 0-4), the walks (8, 5,
            # 6), the member search (9, 7); each launch's rows start after
            # the previous launch's last row
            grows = {
                "start after the first grouped row": (G[:, 0] - g0) / 100.0,
                "zero tables, patch table": (G[:, 1] - G[:, 0]) / 100.0,
                "pass 1: row maximum": (G[:, 2] - G[:, 1]) / 100.0,
                "pass 2: count distinct values": (G[:, 3] - G[:, 2]) / 100.0,
                "sort the groups, store them": (G[:, 4] - G[:, 3]) / 100.0,
                "walk launch: start after the first walk": (G[:, 8] - G[gok, 8].min()) / 100.0,
                "walk launch: softmax sum over groups": (G[:, 5] - G[:, 8]) / 100.0,
                "walk launch: top-p / min-p / draw over groups": (G[:, 6] - G[:, 5]) / 100.0,
                "search launch: start after the first search": (G[:, 9] - G[gok, 9].min()) / 100.0,
                "search launch: patch table, the drawn member": (G[:, 7] - G[:, 9]) / 100.0,
            }
            print(f"grouped launch span {(G[gok, 4].max() - g0) / 100.0:.2f} us; walk launch span "
                  f"{(G[gok, 6].max() - G[gok, 8].min()) / 100.0:.2f} us; search launch span "
                  f"{(G[gok, 7].max() - G[gok, 9].min()) / 100.0:.2f} us")
        print(f"# grouped path (whole-row kernel) phases, {int(gok.sum())} rows")
        print("| Phase | median us | p10 | p90 |")
        print("|---|---|---|---|")
        for name, v in grows.items():
            v = v[gok]
            print(f"| {name} | {np.median(v):.2f} | {np.percentile(v, 10):.2f} | {np.percentile(v, 90):.2f} |")
        print(f"grouped rows' span (first start to last end): {(G[gok, 7].max() - g0) / 100.0:.2f} us")
    P, W, D = st[0], st[1], st[2]
    us = lambda d: d / 100.0  # 100 MHz counter
    ok = (P[:, 11] > 0) & (P[:, 7] > 0)  # the rows this kernel ran to the end
    t0 = P[ok, 0].min() if ok.any() else 0
    wend = W.max(axis=1)
    wfirst = W.min(axis=1)
    rows = {
        "workgroup start after the first": us(P[:, 0] - t0),
        "row constants in": us(P[:, 1] - P[:, 0]),
        "zero tables, barrier": us(P[:, 2] - P[:, 1]),
        "patch bitmap + hash, barrier": us(P[:, 3] - P[:, 2]),
        "bootstrap bound (2 barriers)": us(P[:, 4] - P[:, 3]),
        "stream: to the first wave's end": us(wfirst - P[:, 4]),
        "stream: to the last wave's end": us(wend - P[:, 4]),
        "last wave: hand-in": us(P[:, 5] - wend),
        "patched values, bound, gather": us(P[:, 6] - P[:, 5]),
        "members in order": us(P[:, 7] - P[:, 6]),
        "tail: exp, sum chain, division": us(P[:, 9] - P[:, 8]),
        "tail: top-p chain, cut points": us(P[:, 10] - P[:, 9]),
        "tail: draw chain, output": us(P[:, 11] - P[:, 10]),
        "workgroup total": us(P[:, 11] - P[:, 0]),
    }
    if not ok.any():
        print(f"# no k64_kernel rows with every stamp in workload {args.workload}")
        return
    print(f"# k64_kernel phases, workload {args.workload} (B={w.B} V={w.V}), last of {args.steps} calls; "
          f"{int(ok.sum())} rows with every stamp")
    print("| Phase | median us | p10 | p90 |")
    print("|---|---|---|---|")
    for name, v in rows.items():
        v = v[ok]
        print(f"| {name} | {np.median(v):.2f} | {np.percentile(v, 10):.2f} | {np.percentile(v, 90):.2f} |")
    print(f"candidates at or above the shared bound per row (median / p90 / max): {np.median(P[ok, 12]):.0f} / "
          f"{np.percentile(P[ok, 12], 90):.0f} / {P[ok, 12].max()}; listed patched ids: "
          f"{np.median(P[ok, 13]):.0f} / {np.percentile(P[ok, 13], 90):.0f} / {P[ok, 13].max()}")
    def key2f(k):
        k = np.uint32(k)
        b = (k & 0x7fffffff) if (k & 0x80000000) else (~k & 0xffffffff)
        return float(np.array([b], np.uint32).view(np.float32)[0])
    print(f"bootstrap bound (median): {key2f(int(np.median(P[ok, 14]))):.4f}; final shared bound: "
          f"{key2f(int(np.median(P[ok, 15]))):.4f}")
    print(f"kernel span (first start to last end): {us(P[ok, 11].max() - t0):.2f} us")
    if D[ok, 0].max() > 0:
        det = {"second chunk requested (after the patch table)": us(D[:, 0] - P[:, 3]),
               "first chunk in": us(D[:, 1] - D[:, 0]),
               "bootstrap histogram": us(D[:, 2] - D[:, 1]),
               "barrier": us(D[:, 3] - D[:, 2]),
               "bound scan, barrier": us(P[:, 4] - D[:, 3])}
        for name, v in det.items():
            v = v[ok]
            print(f"| {name} | {np.median(v):.2f} | {np.percentile(v, 10):.2f} | {np.percentile(v, 90):.2f} |")
        if D[ok, 11].max() > 0:
            v = us(D[:, 11] - D[:, 10])[ok]
            print(f"| tail run again (warm instruction cache) | {np.median(v):.2f} | {np.percentile(v, 10):.2f} | "
                  f"{np.percentile(v, 90):.2f} |")
            v = us(P[:, 11] - P[:, 8])[ok]
            print(f"| tail, first run | {np.median(v):.2f} | {np.percentile(v, 10):.2f} | {np.percentile(v, 90):.2f} |")
        m = ok & (D[:, 9] > D[:, 8])
        if m.any():
            ghz = (D[m, 9] - D[m, 8]) / ((P[m, 11] - P[m, 5]) / 100.0) / 1e3
            print(f"shader clock over the last wave's work: {np.median(ghz):.2f} GHz (median)")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="headline")
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=12.0)
    ap.add_argument("--copy-ref", action="store_true",
                    help="also run a plain 256 MiB device copy three times (the reference "
                         "kernel that scales rocprofv3 FETCH_SIZE/WRITE_SIZE to bytes)")
    ap.add_argument("--top-tokens", action="store_true",
                    help="time topTokens (n = --top-n per row) on the workload's logits instead")
    ap.add_argument("--top-n", type=int, default=5)
    ap.add_argument("--softmax", action="store_true",
                    help="time nls_softmax_rows (softmaxInPlace over whole rows) instead of the sampler")
    ap.add_argument("--log-prob", action="store_true",
                    help="time nls_log_prob (logProb's per-token term) instead of the sampler")
    ap.add_argument("--sample-host", action="store_true",
                    help="time nls_sample_host end to end (host logits in, host id out) for the workload")
    ap.add_argument("--row-nll", action="store_true",
                    help="time perplexity's per-position term (one target per row) on the workload's logits")
    ap.add_argument("--traffic-summary", action="store_true",
                    help="write the per-kernel traffic summary from two rocprofv3 --pmc runs "
                         "(--fetch-dir, --write-dir) to --out; no GPU needed")
    ap.add_argument("--trace-summary", action="store_true",
                    help="per-kernel launch durations (median, mean, p10, p90, skipping each kernel's "
                         "first --skip launches) from a rocprofv3 --kernel-trace run (--trace-dir); no GPU needed")
    ap.add_argument("--trace-dir")
    ap.add_argument("--skip", type=int, default=6)
    ap.add_argument("--fetch-dir")
    ap.add_argument("--write-dir")
    ap.add_argument("--out")
    ap.add_argument("--commit", default="")
    ap.add_argument("--lm-head", action="store_true",
                    help="time the output projection nls_lm_head instead of the sampler")
    ap.add_argument("--lm-type", default="Q6_K")
    ap.add_argument("--lm-rows", type=int, default=128256)
    ap.add_argument("--lm-cols", type=int, default=2048)
    ap.add_argument("--lm-nb", type=int, default=1)
    ap.add_argument("--lm-exact", action="store_true", help="exactMatmul: the float path")
    ap.add_argument("--decode-chain", action="store_true",
                    help="time one decode step's tail per token: hidden state in, nls_lm_head, nls_sample, "
                         "id out (B = 1, the --lm-* output shape)")
    ap.add_argument("--lib", default="",
                    help="time this build of the library instead of nim.llm_amd/libnimllm_sampler.so")
    ap.add_argument("--phase-stamps", action="store_true",
                    help="per-phase times of the k64 kernel from the phases build of the library")
    args = ap.parse_args()
    if args.lib:
        load_pkg().LIB_PATH = os.path.abspath(args.lib)
    if args.traffic_summary:
        return traffic_summary(args)
    if args.trace_summary:
        return trace_summary(args)
    if args.phase_stamps:
        return phase_stamps(args)
    if args.gpus != 1:
        print("bench.py: this build measures one GPU only (rows shard across GPUs with no "
              "collective: each GPU samples its own rows); --gpus must be 1", file=sys.stderr)
        sys.exit(2)

    if args.top_tokens:
        return bench_top_tokens(args)
    if args.row_nll:
        return bench_row_nll(args)
    if args.softmax or args.log_prob:
        return bench_softmax(args, args.log_prob)
    if args.sample_host:
        return bench_sample_host(args)
    if args.lm_head:
        return bench_lm_head(args)
    if args.decode_chain:
        return bench_decode_chain(args)
    import numpy as np
    import torch

    pkg = load_pkg()
    from nimllm_amd import workloads

    w = workloads.make(args.workload, seed=args.seed)
    B, V = w.B, w.V
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    s = pkg.BatchSampler(workloads.sampler_params(w, pkg), V, stream=stream)
    if w.hist.shape[1]:
        s.accept(w.hist)
    plan, streamed = s.plan()
    row_bytes = B * V * 4
    nbuf = max(2, math.ceil(640e6 / row_bytes))
    base = torch.from_numpy(w.logits).to(dev)
    bufs = [base] + [base.clone() for _ in range(nbuf - 1)]
    du = torch.from_numpy(w.u).to(dev)
    out = torch.empty(B, dtype=torch.int32, device=dev)

    # parity spot check of the first call against the oracle (8 rows)
    s.sample(bufs[0], du, out)
    torch.cuda.synchronize()
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    got = out.cpu().numpy()
    bid, bval, bcnt = w.bias_arrays()
    chk = np.linspace(0, B - 1, min(B, 8)).astype(int)
    ref = O.sample_batch([O.make_params(**w.rows[r].as_kwargs()) for r in chk], w.logits[chk],
                         w.hist[chk] if w.hist.shape[1] else None,
                         np.full(len(chk), w.hist.shape[1]), bid[chk], bval[chk], bcnt[chk],
                         w.u[chk], O.EXPF_CR, nthreads=8)
    parity_ok = bool(np.array_equal(got[chk], ref))

    # The timed calls go straight to the C ABI (as a C or Nim caller makes
    # them), so the Python wrapper's checks cannot leave the GPU waiting
    # between back-to-back calls.
    import ctypes

    c_sample = pkg.lib().nls_sample
    c_bufs = [ctypes.c_void_p(b.data_ptr()) for b in bufs]
    c_du, c_out = ctypes.c_void_p(du.data_ptr()), ctypes.c_void_p(out.data_ptr())

    def call(i):
        return c_sample(s._h, c_bufs[i % nbuf], c_du, c_out, None)

    st = 0
    for i in range(args.warmup):
        st |= call(i)
    torch.cuda.synchronize()
    # (1) whole pipeline: K back-to-back calls, no per-kernel events
    t_all0, t_all1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_all0.record(stream)
    for i in range(args.steps):
        st |= call(i)
    t_all1.record(stream)
    torch.cuda.synchronize()
    pkg.check(st, "nls_sample")
    total_ms = t_all0.elapsed_time(t_all1)
    ms = total_ms / args.steps
    # (2) HIP events recorded around each kernel of a call on the sampler's
    # stream, one pair per kernel and call (each pair adds its own overhead)
    def events():
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(args.steps)]
        for a, b in ev:  # materialise the underlying hipEvents
            a.record(stream)
            b.record(stream)
        return ev
    ev_s = events()
    ev_g = events() if plan.generic_launch else None
    torch.cuda.synchronize()
    for i in range(args.steps):
        s.profile_next(ev_s[i][0], ev_s[i][1])
        if ev_g:
            s.profile_next_generic(ev_g[i][0], ev_g[i][1])
        st |= call(i)
    torch.cuda.synchronize()
    pkg.check(st, "nls_sample")

    def stats(ev):
        t = sorted(a.elapsed_time(b) for a, b in ev)
        return sum(t) / len(t), t[len(t) // 2]

    # Algorithmic bytes per kernel: the streaming kernel reads the rows it
    # runs to the end, plus the first unit a workgroup of every other row
    # requests before it leaves; the whole-row kernel reads those other rows.
    per_row = w.row_bytes()
    stream_bytes = float(sum(per_row[b] if streamed[b] else min(plan.first_unit_bytes, 4 * V)
                             for b in range(B)))
    generic_bytes = float(sum(per_row[b] for b in range(B) if not streamed[b]))
    pipe_bytes = float(sum(per_row))
    s_avg, s_med = stats(ev_s)
    sname = "k64_kernel" if plan.k64 else "stream_kernel"
    kernels = {}
    if plan.floor_slices > 0:
        # (a batch of full sorts only, split over slices: floor_kernel reads every
        # row; the whole-row kernel after it takes the rows floor_kernel leaves)
        kernels["floor_kernel"] = {"rows": B, "algorithmic_bytes_per_launch": pipe_bytes,
                                   "event_pair_avg_us": s_avg * 1e3, "event_pair_median_us": s_med * 1e3}
        generic_bytes = 0.0
    elif plan.streamed_rows > 0:  # (a batch of full sorts only runs the whole-row kernel alone)
        kernels[sname] = {"rows": int(sum(streamed)), "algorithmic_bytes_per_launch": stream_bytes,
                          "event_pair_avg_us": s_avg * 1e3, "event_pair_median_us": s_med * 1e3}
    if ev_g and plan.floor_slices > 0:
        g_avg, g_med = stats(ev_g)
        kernels["generic_kernel"] = {"rows": 0, "algorithmic_bytes_per_launch": 0.0,
                                     "event_pair_avg_us": g_avg * 1e3, "event_pair_median_us": g_med * 1e3}
    elif ev_g:
        g_avg, g_med = stats(ev_g)
        kernels["generic_kernel"] = {"rows": int(B - sum(streamed)), "algorithmic_bytes_per_launch": generic_bytes,
                                     "event_pair_avg_us": g_avg * 1e3, "event_pair_median_us": g_med * 1e3}
    # When a call is one launch (no full-sort rows: rows the streaming kernel
    # hands on are served by its last workgroup; or full sorts only: the
    # whole-row kernel alone) the kernel's average launch
    # duration is the time of the K back-to-back calls of (1) over K; otherwise
    # the event pairs of (2).
    single = not plan.generic_launch or (plan.streamed_rows == 0 and plan.floor_slices == 0)
    for name, k in kernels.items():
        k["avg_us"] = ms * 1e3 if single else k["event_pair_avg_us"]
        k["avg_from"] = "back-to-back calls" if single else "event pairs"
        k["achieved_GBs"] = k["algorithmic_bytes_per_launch"] / (k["avg_us"] * 1e-6) / 1e9
        k["frac"] = k["achieved_GBs"] / HBM_PEAK_GBS
    dom = max(kernels, key=lambda n: kernels[n]["avg_us"])
    traffic, stale = read_traffic(args.workload)
    for name, k in kernels.items():
        k["traffic"] = traffic.get(name)
    rows_per_s = B / (ms * 1e-3)
    dk = kernels[dom]
    res = {
        "metric": "sampled rows/sec at B=256 x V=128256 fp32; % of MI355X peak HBM GB/s",
        "value": rows_per_s,
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded numpy; logits resident in HBM, rotated over "
                f"{nbuf} buffers = {nbuf * row_bytes / 1e6:.0f} MB to defeat the Infinity Cache)",
        "config": {"workload": workloads.describe(args.workload, B, V), "B": B, "V": V, "seed": args.seed},
        "roofline": {"bound": "hbm", "achieved": dk["achieved_GBs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": dk["frac"], "traffic": dk["traffic"],
                     "kernel": dom, "kernel_avg_us": dk["avg_us"], "kernel_avg_from": dk["avg_from"],
                     "algorithmic_bytes_per_launch": dk["algorithmic_bytes_per_launch"]},
        "kernels": kernels,
        "pipeline": {"algorithmic_bytes": pipe_bytes,
                     "achieved_GBs": pipe_bytes / (ms * 1e-3) / 1e9,
                     "frac": pipe_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS},
        "parity_spot_check": {"rows": int(len(chk)), "bit_exact": parity_ok},
    }
    if stale:
        res["roofline"]["traffic_note"] = stale
    s.close()
    if args.copy_ref:
        res["copy_ref_bytes"] = copy_ref(dev)
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(w, args.cpu_budget)
        res["cpu_baseline_all_cores"] = cpu_baseline(w, args.cpu_budget, nthreads=host_cores())
    else:
        res["cpu_baseline"] = None
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
