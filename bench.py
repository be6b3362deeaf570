#!/usr/bin/env python3
"""Benchmark of the gfx950 token sampler. The default workload is the headline configuration (BASELINE.json
configs[2]): B=64 rows x V=262144 fp32 logits, T 0.8, top-k 64, top-p 0.95, repetition penalty 1.05 over 512-token
histories. --workload cfg1..cfg5 measures each configuration of BASELINE.json (cfg4 through fs_verify), topk0 the
headline rows with top_k = 0 (every token a candidate); --workload all prints one line per workload.

A step is one fs_sample_batch (fs_verify for cfg4) call over the whole batch (penalty -> top-k -> softmax/top-p ->
draw, one kernel) with inputs already resident in HBM. The logits rotate over enough copies (> 256 MB MALL) that
every step streams its rows from HBM. The K timed calls are captured once into a HIP graph and replayed back to
back, as a serving loop issues them (the same calls launched one by one from Python are reported beside). Each line
carries rows/s, the kernel's HBM roofline fraction (HIP events on the replay stream), the HBM traffic of the committed rocprofv3 PMC summary for that workload, and the CPU baseline
(ferro's own sampler.cpp compiled by oracle/Makefile where it supports the workload's parameters, else the oracle
restatement) timed on this host's cores on a bounded sample of the same rows. The CPU leg also checks the GPU's
tokens: rows whose token differs from the reference are counted, and so are the rows whose draw lies within 1e-6 of
a cumulative boundary (where a different summation order may legitimately pick the neighbouring token).
"""
import argparse
import ctypes
import json
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "sampled rows/s + logits HBM GB/s (% of peak), top-k/top-p, B=64, V=262144"
HBM_PEAK_GBS = 8000.0
MALL_BYTES = 256 << 20
KERNEL = "fs::segment_kernel"


def kernel_of(w, route, cus=256, verify=False):
    """The kernel a call of this workload launches, as the library routes it (fs_route_plan): fs_sample_batch_hp /
    fs_verify_hp (route "host") pick the small-k kernel (its greedy-only form for all-greedy batches) where the batch
    fits it, else the fused kernel; fs_sample_batch / fs_verify (route "device") always run the fused kernel."""
    fused = (KERNEL, "segments, then a merging workgroup per row, one grid")
    if route != "host":
        return fused
    from ferro_amd import _lib
    kind, nl, ns, per_cu = _lib.route_plan(cus, w.params, w.V, total_rows=w.B, verify=verify)
    if kind == 0:
        return (KERNEL, f"segments ({per_cu} per CU), then a merging workgroup per row, one grid")
    return (f"fs::small_k_kernel<{nl}>",
            f"{ns} segments of {1024 * nl} logits per row, the last segment of a row merges it, one grid"
            + (" (greedy-only form)" if kind == 2 else ""))

# workload -> (constructor name in ferro_amd.workloads, entry point, description)
WORKLOADS = {
    "cfg1": ("config1", "sample", "cfg1_single_row: B=1 x V=65536 fp32, N(0,2) + 8 spikes, T 0.7, top-k 40, "
                                  "top-p 0.95, repetition 1.1 over a 64-token history"),
    "cfg2": ("config2", "sample", "cfg2_greedy_freq_pres: B=8 x V=65536 fp32, greedy, frequency 0.5 / presence 0.3 "
                                  "over 256-token Zipf histories, 1% forced ties"),
    "cfg3": ("config3", "sample", "cfg3_gemma_serving: B=64 x V=262144 fp32, T 0.8, top-k 64, top-p 0.95, "
                                  "repetition 1.05 over 512-token histories"),
    "cfg4": ("config4", "verify", "cfg4_spec_verify: 16 streams x 17 rows = 272 x V=65536 fp32, greedy, "
                                  "per-position argmax + accepted prefix per stream (fs_verify)"),
    "cfg5": ("config5", "sample", "cfg5_heterogeneous: B=256 x V=262144 fp32, per-row T / top-k (1..2048) / top-p / "
                                  "repetition, frequency and presence penalties over 1024-token histories"),
    "topk0": ("config3_all_tokens", "sample", "cfg3_all_tokens: cfg3's rows with top_k = 0 (every token a "
                                              "candidate: the whole-row path)"),
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def read_traffic(name, kernel):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary of this kernel on this workload
    (profiles/<kernel>_<workload>_traffic.md: reads by request size + WRITE_SIZE, calibrated)."""
    short = kernel.split("::")[-1].split("<")[0]
    try:
        txt = open(os.path.join(ROOT, "profiles", f"{short}_{name}_traffic.md")).read()
    except OSError:
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", txt)
    return float(m.group(1)) if m else None


def n_cores():
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    return max(1, min(16, avail))                  # a GPU box's CPU share is 16 cores per GPU


def uses_extension(w):
    """ferro's SamplerParams has no frequency/presence penalty (sampler.h:12-21): such rows run on the port."""
    return bool((w.params["frequency_penalty"] != 0).any() or (w.params["presence_penalty"] != 0).any())


def verify_rows(w):
    """cfg4 as ferro's server samples it (server.cpp:627-637): row r of stream s with the stream's history plus the
    drafts fed before it; returns per-row CSR histories and per-row params."""
    hs, prm = [], []
    for s in range(len(w.row_off) - 1):
        r0, r1 = int(w.row_off[s]), int(w.row_off[s + 1])
        base = w.hist[w.hist_off[s]:w.hist_off[s + 1]]
        for r in range(r1 - r0):
            hs.append(np.concatenate([base, w.rows[r0 + 1:r0 + 1 + r]]).astype(np.int32))
            prm.append(w.params[s])
    off = np.zeros(len(hs) + 1, np.int64)
    off[1:] = np.cumsum([len(h) for h in hs])
    return np.concatenate(hs), off, np.array(prm, dtype=w.params.dtype)


def accepted_prefix(tok, rows, row_off, eos=-1):
    """The verification rule (server.cpp:627-637): 1 + leading rows whose token equals the next draft."""
    acc = np.zeros(len(row_off) - 1, np.int32)
    for s in range(len(row_off) - 1):
        r0, m = int(row_off[s]), int(row_off[s + 1] - row_off[s])
        a = 0
        for r in range(m):
            a = r + 1
            if eos >= 0 and tok[r0 + r] == eos:
                break
            if r + 1 < m and tok[r0 + r] == rows[r0 + r + 1]:
                continue
            break
        acc[s] = a
    return acc


def cpu_baseline(w, entry, gpu_tok, gpu_acc, budget_s):
    """Rows of the same workload through ferro's CPU sampler (or the oracle port where ferro lacks a parameter) on
    1 core, serial per row as ferro's server samples them, repeated up to ~budget_s seconds; then the whole batch
    once more, untimed, to count the GPU's token mismatches and the rows near a cumulative boundary."""
    from oracle import oracle as O
    if entry == "verify":
        hist, hoff, params = verify_rows(w)
    else:
        hist, hoff, params = w.hist, w.hist_off, w.params
    kind = "reference" if O.ref_available() and not uses_extension(w) else "port"
    B = w.B
    chunk = min(8, B)
    rows_done, t_used, b = 0, 0.0, 0
    while t_used < budget_s:
        e = min(b + chunk, B)
        sl = slice(b, e)
        x = np.ascontiguousarray(w.logits[sl]).copy()
        off = hoff[b:e + 1] - hoff[b]
        h = hist[hoff[b]:hoff[e]]
        t0 = time.perf_counter()
        if kind == "reference":
            O.ref_sample_batch(x, h, off, params[sl], w.seeds[sl], nthreads=1, inplace=True)
        else:
            O.sample_batch(x, h, off, params[sl], w.u[sl], nthreads=1)
        t_used += time.perf_counter() - t0
        rows_done += e - b
        b = e % B
    out = dict(value=rows_done / t_used, unit="rows/s", cores=1, kind=kind,
               sample=f"{rows_done} rows of the same B={B} x V={w.V} workload (rows cycled), serial on 1 core "
                      f"as ferro's server samples them ({t_used:.1f} s)" +
                      ("; ferro has no frequency/presence penalty, so the oracle port ran" if kind == "port" else ""))
    nth = n_cores()
    if kind == "reference":
        ref_tok = O.ref_sample_batch(w.logits, hist, hoff, params, w.seeds, nthreads=nth)
        out["all_cores"] = cpu_all_cores(w, hist, hoff, params, budget_s / 3, min(nth, B))
    else:
        ref_tok = None
    # parity leg (untimed): the oracle's candidate probabilities locate the rows near a cumulative boundary
    kmax = int(np.where(params["top_k"] <= 0, w.V, np.minimum(params["top_k"], w.V)).max())
    ora = O.sample_batch(w.logits, hist, hoff, params, w.u, kcap=min(kmax, w.V), nthreads=nth)
    ref_tok = ora["tok"] if ref_tok is None else ref_tok
    diff = np.nonzero(gpu_tok != ref_tok)[0]
    near = []
    for r in range(B):
        p = params[r]
        if p["temperature"] <= 0 or p["top_k"] == 1:
            continue
        nc = int(ora["ncand"][r])
        if O.near_boundary(ora["cand_probs"][r, :nc], int(ora["keep"][r]), float(w.u[r]), float(p["top_p"]),
                           float(p["min_p"])):
            near.append(r)
    out["parity"] = dict(rows=B, token_mismatches_vs_cpu=int(len(diff)), rows_near_boundary=len(near),
                         mismatches_near_boundary=int(np.isin(diff, near).sum()),
                         oracle_vs_reference_mismatches=int((ora["tok"] != ref_tok).sum()) if kind == "reference"
                         else None)
    if entry == "verify":
        out["parity"]["accepted_mismatches_vs_cpu"] = int(
            (accepted_prefix(ref_tok, w.rows, w.row_off) != gpu_acc).sum())
    return out


def cpu_all_cores(w, hist, hoff, params, budget_s, nth):
    """Upper bound for a CPU server: the whole batch's rows spread over this host's cores (rows are independent),
    through ferro's own sampler, repeated up to ~budget_s seconds."""
    from oracle import oracle as O
    rows_done, t_used = 0, 0.0
    while t_used < budget_s:
        x = np.ascontiguousarray(w.logits).copy()
        t0 = time.perf_counter()
        O.ref_sample_batch(x, hist, hoff, params, w.seeds, nthreads=nth, inplace=True)
        t_used += time.perf_counter() - t0
        rows_done += w.B
    return dict(value=rows_done / t_used, unit="rows/s", cores=nth,
                sample=f"{rows_done} rows (the B={w.B} batch repeated), rows spread over {nth} threads ({t_used:.1f} s)")


def graph_wall(torch, call, what, ctx, bufs, nrot, V, fixed, K, tok, want, L):
    """K calls captured into one HIP graph (torch.cuda.CUDAGraph over the capture stream) and replayed: returns the
    replay's wall-clock seconds and its HIP-event time per call (ms; an event pair on the replay stream around the
    whole replay, so back-to-back launches with no host work between them). The calls launch kernels only (no
    allocation, copy or memset once warm), so they capture as they run eagerly. Replays are checked against the
    eager tokens, with eager calls between them."""
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            cs = ctypes.c_void_p(side.cuda_stream)
            for i in range(K):
                rc = call(ctx.h, P(bufs[i % nrot]), V, *fixed[:-1], cs)
                if rc != 0:
                    raise RuntimeError(f"{what} returned {rc} under capture")
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    walls, evms = [], []
    stream = torch.cuda.current_stream()
    for rep in range(3):
        tok.fill_(-1)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e0.record(stream)
        g.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        walls.append(time.perf_counter() - t0)
        evms.append(e0.elapsed_time(e1) / K)
        if not np.array_equal(tok.cpu().numpy(), want):
            raise RuntimeError(f"graph replay {rep} changed the tokens")
        rc = call(ctx.h, P(bufs[0]), V, *fixed)          # eager work between the replays
        if rc != 0:
            raise RuntimeError(f"{what} returned {rc}")
        torch.cuda.synchronize()
    if F_device_error(L, ctx, fixed[-1]) != 0:
        raise RuntimeError("device error bits set after the graph replays")
    del g
    best = 1 + int(np.argmin(walls[1:]))
    return walls[best], evms[best]


def host_rows_rate(torch, w, dst, step_on, steps):
    """The PCIe-inclusive rate: each step first copies the batch's fp32 rows from pinned host memory to the device
    (as a caller holding host rows must; ferro's own call sites copy every row back from the GPU before sampling,
    model_lfm2_lm.cpp:477-480), then samples them. Also times the copies alone."""
    host = torch.from_numpy(w.logits).pin_memory()
    view = dst[:, :w.V] if dst.dim() == 2 else dst
    stream = torch.cuda.current_stream()

    def timed(fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(stream)
        for _ in range(steps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return time.perf_counter() - t0, e0.elapsed_time(e1) / steps

    def copy_only():
        view.copy_(host, non_blocking=True)

    def copy_and_sample():
        view.copy_(host, non_blocking=True)
        rc = step_on(dst)
        if rc != 0:
            raise RuntimeError(f"call returned {rc}")

    wall_c, ms_c = timed(copy_only)
    wall_s, ms_s = timed(copy_and_sample)
    nbytes = w.logits.nbytes
    return {"value": w.B * steps / wall_s, "unit": "rows/s", "ms_per_step": ms_s,
            "copy_ms": ms_c, "copy_GBps": nbytes / (ms_c * 1e-3) / 1e9, "bytes_copied": nbytes,
            "note": "each step copies the batch's rows host -> device (pinned, one async copy) and then samples "
                    "them; ms from HIP events on the stream"}


def run_workload(name, args, torch):
    from ferro_amd import workloads as W
    from ferro_amd import _lib
    from ferro_amd.sampler import Context

    ctor, entry, desc = WORKLOADS[name]
    t0 = time.time()
    w = getattr(W, ctor)()
    log(f"workload {w.name}: B={w.B} V={w.V} generated in {time.time() - t0:.1f}s")
    dev = torch.device("cuda", 0)
    nrot = max(2, -(-2 * MALL_BYTES // w.logits.nbytes))
    base = torch.from_numpy(w.logits).to(dev)
    bufs = [base] + [base.clone() for _ in range(nrot - 1)]
    params = torch.from_numpy(w.params.view(np.uint8).copy()).to(dev)
    hist = torch.from_numpy(w.hist).to(dev)
    hoff = torch.from_numpy(w.hist_off).to(dev)
    u = torch.from_numpy(w.u).to(dev)
    tok = torch.empty(w.B, dtype=torch.int32, device=dev)
    keep = torch.empty(w.B, dtype=torch.int32, device=dev)
    ctx = Context.default(dev)
    L = _lib.lib()
    stream = torch.cuda.current_stream()
    sh = ctypes.c_void_p(stream.cuda_stream)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    if entry == "verify":
        rows = torch.from_numpy(w.rows).to(dev)
        roff = torch.from_numpy(w.row_off).to(dev)
        S = len(w.row_off) - 1
        acc = torch.empty(S, dtype=torch.int32, device=dev)
        if args.route == "host":
            hp = np.ascontiguousarray(w.params)         # the host copy of the stream parameters
            fixed = (S, w.B, w.V, P(rows), P(roff), P(hist), P(hoff), P(params), hp.ctypes.data_as(ctypes.c_void_p),
                     P(u), -1, P(tok), P(acc), sh)
            call, what = L.fs_verify_hp, "fs_verify_hp"
        else:
            fixed = (S, w.B, w.V, P(rows), P(roff), P(hist), P(hoff), P(params), P(u), -1, P(tok), P(acc), sh)
            call, what = L.fs_verify, "fs_verify"
    elif args.route == "host":
        acc = None
        hp = np.ascontiguousarray(w.params)             # the host copy of the parameters (picks the kernel)
        fixed = (w.B, w.V, P(hist), P(hoff), P(params), hp.ctypes.data_as(ctypes.c_void_p), P(u), P(tok), 0, None,
                 None, P(keep), sh)
        call, what = L.fs_sample_batch_hp, "fs_sample_batch_hp"
    else:
        acc = None
        fixed = (w.B, w.V, P(hist), P(hoff), P(params), P(u), P(tok), 0, None, None, P(keep), sh)
        call, what = L.fs_sample_batch, "fs_sample_batch"
    kname, kdesc = kernel_of(w, args.route, ctx_cus(torch), verify=entry == "verify")

    def step(i):
        rc = call(ctx.h, P(bufs[i % nrot]), w.V, *fixed)
        if rc != 0:
            raise RuntimeError(f"{what} returned {rc}")

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    gpu_tok = tok.cpu().numpy().copy()
    gpu_acc = acc.cpu().numpy().copy() if acc is not None else None

    K = args.steps
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(K)]
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    for i in range(K):
        ev[i][0].record(stream)
        step(i)
        ev[i][1].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_start
    kern_ms = float(np.mean([a.elapsed_time(b) for a, b in ev]))
    if not np.array_equal(tok.cpu().numpy(), gpu_tok):
        raise RuntimeError("tokens changed between steps on identical inputs")
    if F_device_error(L, ctx, sh) != 0:
        raise RuntimeError("device error bits set after the timed steps")
    wall_graph, graph_ms = graph_wall(torch, call, what, ctx, bufs, nrot, w.V, fixed, K, tok, gpu_tok, L)

    alg_bytes = w.algorithmic_bytes()
    achieved = alg_bytes / (graph_ms * 1e-3) / 1e9
    out = {
        "metric": METRIC,
        "value": w.B * K / wall_graph,
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": wall_graph / K * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded; BASELINE.json's logit, history and parameter distributions for this config)",
        "config": {"workload": desc, "B": w.B, "V": w.V, "entry_point": what, "logit_copies_rotated": nrot},
        "value_note": ("rows/s over the wall clock of the K calls captured once into a HIP graph and replayed "
                       "(as a serving loop issues them); roofline.kernel_ms is the HIP-event time per call over "
                       "that replay, on its stream"),
        "python_launch": {"value": w.B * K / wall, "ms_per_step": wall / K * 1e3,
                          "note": "the same K calls launched one by one from Python through ctypes, an event pair "
                                  "around each"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": read_traffic(name, kname),
                     "kernel": f"{what}: {kname} ({kdesc})",
                     "kernel_ms": graph_ms, "kernel_ms_python_launch": kern_ms, "algorithmic_bytes": alg_bytes,
                     "algorithmic_bytes_note": "4*V per row (one read of the fp32 row) + 4 per history id"},
    }
    if args.host_rows:
        out["host_rows"] = host_rows_rate(torch, w, bufs[0], step_on=lambda dst: call(ctx.h, P(dst), w.V, *fixed),
                                          steps=K)
    if args.copy_calib:
        src = torch.empty(64 << 20, dtype=torch.float32, device=dev)   # 256 MiB
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("copy calibration: 5 copies of 268435456 bytes")
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(w, entry, gpu_tok, gpu_acc, args.cpu_seconds)
    del bufs
    torch.cuda.empty_cache()
    return out


# Stage breakdown by ablation: the same rows and call, with stages switched off one at a time (parameter overrides
# applied to every row). Differences between the lines price the penalty pass, the top-k select and the
# softmax / top-p / draw; the greedy line with no penalty is the streaming read plus an argmax.
BREAKDOWN = [
    ("full", {}),
    ("no penalty", {"repetition_penalty": 1.0, "frequency_penalty": 0.0, "presence_penalty": 0.0}),
    ("no top-p (softmax + draw over k)", {"top_p": 1.0}),
    ("no penalty, no top-p", {"repetition_penalty": 1.0, "frequency_penalty": 0.0, "presence_penalty": 0.0,
                              "top_p": 1.0}),
    ("greedy (argmax) with penalty", {"temperature": 0.0}),
    ("greedy (argmax), no penalty: stream + argmax", {"temperature": 0.0, "repetition_penalty": 1.0,
                                                      "frequency_penalty": 0.0, "presence_penalty": 0.0}),
]


def _with(w, prm):
    from dataclasses import replace
    return replace(w, params=prm)


def run_breakdown(name, args, torch):
    """One JSON line: the HIP-event time per call of each ablation variant of the workload."""
    from ferro_amd import workloads as W
    from ferro_amd import _lib
    from ferro_amd.sampler import Context

    ctor, entry, desc = WORKLOADS[name]
    if entry != "sample":
        raise SystemExit("--breakdown applies to fs_sample_batch workloads")
    w = getattr(W, ctor)()
    dev = torch.device("cuda", 0)
    nrot = max(2, -(-2 * MALL_BYTES // w.logits.nbytes))
    base = torch.from_numpy(w.logits).to(dev)
    bufs = [base] + [base.clone() for _ in range(nrot - 1)]
    hist = torch.from_numpy(w.hist).to(dev)
    hoff = torch.from_numpy(w.hist_off).to(dev)
    u = torch.from_numpy(w.u).to(dev)
    tok = torch.empty(w.B, dtype=torch.int32, device=dev)
    ctx = Context.default(dev)
    L = _lib.lib()
    stream = torch.cuda.current_stream()
    sh = ctypes.c_void_p(stream.cuda_stream)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    out = []
    for label, over in BREAKDOWN:
        prm = w.params.copy()
        for f, v in over.items():
            prm[f] = v
        params = torch.from_numpy(prm.view(np.uint8).copy()).to(dev)
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
        hp = np.ascontiguousarray(prm)
        for i in range(args.warmup + args.steps):
            if i >= args.warmup:
                ev[i - args.warmup][0].record(stream)
            if args.route == "host":
                rc = L.fs_sample_batch_hp(ctx.h, P(bufs[i % nrot]), w.V, w.B, w.V, P(hist), P(hoff), P(params),
                                          hp.ctypes.data_as(ctypes.c_void_p), P(u), P(tok), 0, None, None, None, sh)
            else:
                rc = L.fs_sample_batch(ctx.h, P(bufs[i % nrot]), w.V, w.B, w.V, P(hist), P(hoff), P(params), P(u),
                                       P(tok), 0, None, None, None, sh)
            if rc != 0:
                raise RuntimeError(f"fs_sample_batch returned {rc}")
            if i >= args.warmup:
                ev[i - args.warmup][1].record(stream)
        torch.cuda.synchronize()
        ms = float(np.median([a.elapsed_time(b) for a, b in ev]))
        out.append({"variant": label, "kernel": kernel_of(w if not over else _with(w, prm), args.route)[0],
                    "us_per_call": ms * 1e3,
                    "GB_per_s": w.algorithmic_bytes() / (ms * 1e-3) / 1e9})
    return {"breakdown": desc, "B": w.B, "V": w.V, "steps": args.steps, "timing": "median HIP-event time per call",
            "variants": out}


def run_dropin(args):
    """The C++ drop-in ferro_amd::Sampler (include/ferro_sampler.hpp) one row per call, as ferro's single-row call
    sites use ferro::Sampler (server.cpp:546, lm_cli.cpp:129,324): ferro_amd/dropin_bench, a separate process, on
    config 1's row. Microseconds per call by the host's clock, the token back on the host each time."""
    import subprocess
    exe = os.path.join(ROOT, "ferro_amd", "dropin_bench")
    if not os.path.exists(exe):
        raise SystemExit(f"{exe} is missing: run __graft_entry__.build()")
    r = subprocess.run([exe, str(max(200, args.steps * 10))], capture_output=True, text=True, timeout=300)
    if r.returncode != 0:
        raise RuntimeError(f"dropin_bench failed ({r.returncode}): {r.stderr[-500:]}")
    d = json.loads(r.stdout.strip().splitlines()[-1])
    return {"metric": "ferro_amd::Sampler per-call latency (C++ drop-in, one row per call)", "unit": "us/call",
            "value": d["host_row_us"], "higher_is_better": False, "n_gpus": 1, "dtype": "f32",
            "data": "synthetic (config 1's row: V=65536, N(0,2) + 8 spikes, repetition 1.1 over 64 ids, T 0.7, "
                    "top-k 40, top-p 0.95)",
            "config": {"workload": "dropin: ferro_amd::Sampler::sample (host row) / sample_device (device row)",
                       "calls": d["calls"], "V": d["V"]},
            "host_row_us": d["host_row_us"], "host_row_writeback_us": d["host_row_writeback_us"],
            "device_row_us": d["device_row_us"],
            "note": "host_row: the row copied host -> device each call (ferro's server call sites); "
                    "host_row_writeback: also leaves the host row penalised in place like ferro's sample "
                    "(lm_cli.cpp:353); device_row: the row already on the device. Each includes the draw, the "
                    "history upload, the kernel, the token and error bits back, one stream synchronization."}


def ctx_cus(torch):
    return torch.cuda.get_device_properties(0).multi_processor_count


def F_device_error(L, ctx, sh):
    bits = ctypes.c_int32(0)
    rc = L.fs_device_error(ctx.h, sh, ctypes.byref(bits))
    return bits.value if rc == 0 else -1


def run_decode(args, torch):
    """The one-launch decode step on cfg3's batch (fs_decode_step_hp: the small-k kernel; fs_decode_step: the fused
    kernel): each step samples every stream from its device draw stream and appends the token to its history, whose
    output becomes the next step's input. The same logits every step (a model's output would differ); µs per step
    from HIP events on the stream, launched one by one. Tokens of the two routes are compared step by step."""
    import ferro_amd as F
    from ferro_amd import workloads as W
    w = W.config3()
    x = torch.from_numpy(w.logits).cuda()
    out = {"metric": "one-launch decode step (sample + draw + history append), cfg3's batch", "unit": "us/step",
           "note": "HIP events around each Python call (its tensor allocations and launch included); the kernel "
                   "time alone comes from rocprofv3 (profiles/decode_step_cfg3_kernel_trace.md)",
           "higher_is_better": False, "n_gpus": 1, "dtype": "f32", "steps": args.steps, "warmup": args.warmup,
           "data": "synthetic (cfg3's rows every step)", "config": {"workload": "decode: cfg3 B=64 x V=262144"}}
    toks = {}
    for route, entry in (("host", "fs_decode_step_hp"), ("device", "fs_decode_step")):
        d = F.DeviceRng(np.arange(1, w.B + 1, dtype=np.uint64))
        hist = torch.from_numpy(w.hist).cuda()
        off = torch.from_numpy(w.hist_off).cuda()
        cap = int(w.hist.size + w.B * (args.warmup + args.steps + 1))
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
        seq = []
        for i in range(args.warmup + args.steps):
            if i >= args.warmup:
                ev[i - args.warmup][0].record()
            tok, _, hist, off = F.decode_step(x, w.params, d, hist=hist, hist_off=off, out_cap=cap, route=route)
            if i >= args.warmup:
                ev[i - args.warmup][1].record()
            seq.append(tok)
        torch.cuda.synchronize()
        if F.device_error() != 0:
            raise RuntimeError(f"{entry}: device error bits set")
        toks[route] = torch.stack(seq).cpu().numpy()
        out[f"{route}_us_per_step"] = float(np.median([a.elapsed_time(b) for a, b in ev]) * 1000.0)
        out[f"{route}_entry"] = entry
    out["tokens_equal_across_routes"] = bool(np.array_equal(toks["host"], toks["device"]))
    if not out["tokens_equal_across_routes"]:
        raise RuntimeError("the two decode routes disagree")
    out["value"] = out["host_us_per_step"]
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--workload", choices=list(WORKLOADS) + ["dropin", "decode", "all"], default="cfg3",
                    help="cfg3 (default): the headline; cfg1..cfg5: BASELINE.json's configurations; topk0: cfg3 with "
                         "top_k = 0; dropin: the C++ drop-in's per-call latency on one row; decode: the one-launch "
                         "decode step on cfg3's batch, both entry points; all: one line each")
    ap.add_argument("--breakdown", action="store_true",
                    help="instead of the bench line: per-stage ablation timings of the workload (one JSON line)")
    ap.add_argument("--host-rows", action="store_true",
                    help="also report the PCIe-inclusive rate: the rows copied from pinned host memory every step")
    ap.add_argument("--route", choices=["host", "device"], default="host",
                    help="host (default): sampling calls pass the host copy of the parameters too "
                         "(fs_sample_batch_hp, which picks the small-k kernel for batches it fits, as a serving loop "
                         "holding its requests' parameters does); device: fs_sample_batch (the fused kernel)")
    ap.add_argument("--copy-calib", action="store_true",
                    help="after the timed steps, run plain 256 MiB device copies (counter calibration for rocprofv3)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the sampler path is built and measured on a single MI355X "
              f"(--gpus {args.gpus} is not supported in this build)", file=sys.stderr)
        sys.exit(2)

    import torch
    torch.cuda.set_device(torch.device("cuda", 0))
    names = list(WORKLOADS) + ["dropin"] if args.workload == "all" else [args.workload]
    for name in names:
        if name == "dropin":
            if not args.breakdown:
                print(json.dumps(run_dropin(args)), flush=True)
            continue
        if name == "decode":
            if not args.breakdown:
                print(json.dumps(run_decode(args, torch)), flush=True)
            continue
        if args.breakdown:
            if WORKLOADS[name][1] == "sample":
                print(json.dumps(run_breakdown(name, args, torch)), flush=True)
        else:
            print(json.dumps(run_workload(name, args, torch)), flush=True)


if __name__ == "__main__":
    main()
