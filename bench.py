"""Benchmark of the MI355X sampler: rows/s and HBM roofline fraction.

One step = one nls_sample call over one batch (penalties -> bias -> temperature
-> top-k -> softmax -> top-p -> min-p -> draw for every row), inputs already
resident in HBM.  The timed region rotates over enough copies of the logits to
exceed the 256 MB Infinity Cache, so every step reads its logits from HBM.

    python bench.py [--steps K] [--warmup W] [--workload headline] [--no-cpu-baseline]

Prints one JSON line.  `roofline` is for the streaming kernel (stream_kernel,
the single read of the logits, which runs the whole pipeline of greedy and
top-k rows), timed with HIP events on the sampler's stream (around K back-to-back calls
when a call is that one launch); `cpu_baseline` times the CPU restatement of the
reference sampler (oracle/) on the host on a bounded sample of the same rows.
"""
import argparse
import importlib.util
import json
import math
import os
import platform
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


def read_traffic(workload):
    """HBM bytes per launch of the streaming kernel, from the committed
    rocprofv3 --pmc summary (FETCH_SIZE + WRITE_SIZE, copy-kernel scaled)."""
    path = os.path.join(ROOT, "profiles", f"stream_kernel_{workload}_traffic.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def cpu_baseline(w, budget_s=12.0):
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import oracle as O

    params = [O.make_params(**r.as_kwargs()) for r in w.rows]
    bid, bval, bcnt = w.bias_arrays()
    hl = np.full(w.B, w.hist.shape[1], dtype=np.int64)
    hist = w.hist if w.hist.shape[1] else None
    rows_done = 0
    t0 = time.perf_counter()
    chunk = max(1, min(w.B, 64))
    start = 0
    while time.perf_counter() - t0 < budget_s:
        rows = np.arange(start, start + chunk) % w.B
        O.sample_batch([params[r] for r in rows], w.logits[rows],
                       None if hist is None else hist[rows], hl[rows], bid[rows], bval[rows],
                       bcnt[rows], w.u[rows], O.EXPF_LIBM, nthreads=1)
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
    return {"value": rows_done / dt, "unit": "rows/s", "cores": 1, "kind": "port",
            "sample": f"{rows_done} rows of the same workload ({w.name}), rows run serially on "
                      f"one thread for {dt:.1f} s; C restatement of src/nimllm/sampler.nim:59-121 "
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
    # the reference's sum is V dependent fp32 adds per row; one add issues every
    # 4 cycles (a wave64 VALU instruction) at the 2.4 GHz peak engine clock
    chain_us = V * 4 / 2.4e3
    res = {"metric": f"topTokens rows/sec at B={B} x V={V} fp32, n={n}", "value": B / (ms * 1e-3),
           "unit": "rows/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
           "dtype": "f32", "data": "synthetic (the sampler workload's logits, rotated over "
                                   f"{nbuf} buffers)",
           "config": {"workload": f"{args.workload} logits, topTokens n={n}", "B": B, "V": V},
           "roofline": {"bound": "latency", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": achieved / HBM_PEAK_GBS, "traffic": None,
                        "kernel": "top_tokens_kernel", "kernel_avg_us": ms * 1e3,
                        "algorithmic_bytes_per_launch": nbytes,
                        "sum_chain_bound_us": chain_us, "frac_of_chain_bound": chain_us / (ms * 1e3)},
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
    ap.add_argument("--row-nll", action="store_true",
                    help="time perplexity's per-position term (one target per row) on the workload's logits")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU only (rows shard across GPUs with no "
              "collective; see DESIGN.md); --gpus must be 1", file=sys.stderr)
        sys.exit(2)

    if args.top_tokens:
        return bench_top_tokens(args)
    if args.row_nll:
        return bench_row_nll(args)
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

    for i in range(args.warmup):
        s.sample(bufs[i % nbuf], du, out)
    torch.cuda.synchronize()
    # (1) whole pipeline: K back-to-back calls, no per-kernel events
    t_all0, t_all1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_all0.record(stream)
    for i in range(args.steps):
        s.sample(bufs[i % nbuf], du, out)
    t_all1.record(stream)
    torch.cuda.synchronize()
    total_ms = t_all0.elapsed_time(t_all1)
    ms = total_ms / args.steps
    # (2) HIP events recorded around the streaming kernel alone on the
    # sampler's stream, one pair per call (each pair adds its own overhead)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(args.steps)]
    for a, b in ev:  # materialise the underlying hipEvents
        a.record(stream)
        b.record(stream)
    torch.cuda.synchronize()
    for i in range(args.steps):
        s.profile_next(ev[i][0], ev[i][1])
        s.sample(bufs[i % nbuf], du, out)
    torch.cuda.synchronize()
    kern_ms = sorted(a.elapsed_time(b) for a, b in ev)
    kern_avg_ms = sum(kern_ms) / len(kern_ms)
    kern_med_ms = kern_ms[len(kern_ms) // 2]
    pipe_bytes = w.algorithmic_bytes()
    kern_bytes = float(pipe_bytes)  # the streaming kernel runs the whole pipeline of top-k/greedy rows
    # When every row is greedy or top-k with k <= 2048, a call is one launch of
    # the streaming kernel (rows it hands on are served by its last
    # workgroup), so the kernel's average launch duration is the time of the
    # K back-to-back calls of (1) over K; otherwise the event pairs of (2).
    single = all(r.temperature <= 0 or 0 < r.topK < min(V, 2049) for r in w.rows)
    launch_ms = ms if single else kern_avg_ms
    achieved = kern_bytes / (launch_ms * 1e-3) / 1e9
    rows_per_s = B / (ms * 1e-3)
    traffic = read_traffic(args.workload)
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
        "config": {"workload": f"{args.workload}: B={B} x V={V} fp32 logits N(0, 2.5^2); "
                               "frequency 0.5 / presence 0.3 over 1024 Zipf(1.2) history ids; "
                               "50 bias ids per row (5 at -inf); top-k 50, top-p 0.95, T 1.0"
                   if args.workload == "headline" else args.workload,
                   "B": B, "V": V, "seed": args.seed},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": traffic,
                     "kernel": "stream_kernel", "kernel_avg_us": launch_ms * 1e3,
                     "kernel_avg_from": "back-to-back calls" if single else "event pairs",
                     "event_pair_avg_us": kern_avg_ms * 1e3, "event_pair_median_us": kern_med_ms * 1e3,
                     "algorithmic_bytes_per_launch": kern_bytes},
        "pipeline": {"algorithmic_bytes": pipe_bytes,
                     "achieved_GBs": pipe_bytes / (ms * 1e-3) / 1e9,
                     "frac": pipe_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS},
        "parity_spot_check": {"rows": int(len(chk)), "bit_exact": parity_ok},
    }
    s.close()
    if args.copy_ref:
        n = 64 * 1024 * 1024  # 64 Mi floats = 256 MiB read and 256 MiB written per copy
        a = torch.empty(n, dtype=torch.float32, device=dev).fill_(1.0)
        b = torch.empty_like(a)
        torch.cuda.synchronize()
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        res["copy_ref_bytes"] = n * 4
        del a, b
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(w, args.cpu_budget)
    else:
        res["cpu_baseline"] = None
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
