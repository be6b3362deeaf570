#!/usr/bin/env python3
"""Per-phase timeline of one sampling call, from the trace build of the library.

libferro_sampler_trace.so is the same source compiled with -DFS_TRACE (ferro_amd/build.py builds it beside the
product library): thread 0 of every workgroup stores the GPU's constant 100 MHz clock at its phase boundaries.
Segment workgroups (one per (row, segment) item): 0 start, 1 tile 0 arrived, 2 tile 0 done (penalty, first bound,
appends, check), 3 last tile done, 4 list published and counted. Merging workgroups (one per row): 0 start, 1 the
row's segments seen done, 2 candidates gathered (short merge), 3 candidates ranked (short merge), 4 row finished.
Slots 5-12 of a segment workgroup: on the fused path, when the slowest of its waves finished tiles 0-7; on the
large-k path, the row passes (see sampler_kernels.hip). Slots 13-15 tag role, row, segment.

With --route host the call goes through fs_sample_batch_hp / fs_verify_hp, which run the small-k kernel for batches it
fits. Its slots (thread 0 of every (row, segment) workgroup): 0 start, 11 the segment's logits in and transformed,
12 lane maxima sorted, 2 bound (after the barrier), 3 groups handed over, 4 candidates expanded, 5 list ranked and
published, 6 ticket taken; the row's last segment: 7 lists folded, 8 row finished. Slots 9-10: candidates and
groups; 13: role (3 segment, 4 segment that merged its row); 14-15: row, segment. Greedy rows leave 11-4 unset
(their "published" step is then counted from the start).

Usage (on a GPU):  python ferro_amd/trace_phases.py --workload cfg3 [--calls 5] [--route host]
Prints a markdown table: when each phase happens (µs from the first workgroup's start; min / median / max over the
workgroups, median over the traced calls) and how long it takes per workgroup.
"""
from __future__ import annotations

import argparse
import ctypes
import os
import sys

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

TRACE_LIB = os.path.join(PKG, "libferro_sampler_trace.so")
TRACE_W = 16
TICK_US = 0.01                                    # s_memrealtime: 100 MHz


def load():
    from ferro_amd._lib import SIGNATURES
    if not os.path.exists(TRACE_LIB):
        raise RuntimeError(f"{TRACE_LIB} is missing: build it with `python ferro_amd/build.py --trace`")
    L = ctypes.CDLL(TRACE_LIB)
    for name, (res, args) in SIGNATURES.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    L.fs_trace_set.restype = ctypes.c_int
    L.fs_trace_set.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
    return L


def one_call(L, ctx, w, entry, bufs, dev_in, trace, i, torch, hp=None):
    P = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None  # noqa: E731
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    x = bufs[i % len(bufs)]
    if hp is not None:
        h = hp.ctypes.data_as(ctypes.c_void_p)
        if entry == "verify":
            rc = L.fs_verify_hp(ctx, P(x), w.V, len(w.row_off) - 1, w.B, w.V, P(dev_in["rows"]), P(dev_in["roff"]),
                                P(dev_in["hist"]), P(dev_in["hoff"]), P(dev_in["params"]), h, P(dev_in["u"]), -1,
                                P(dev_in["tok"]), P(dev_in["acc"]), st)
        else:
            rc = L.fs_sample_batch_hp(ctx, P(x), w.V, w.B, w.V, P(dev_in["hist"]), P(dev_in["hoff"]),
                                      P(dev_in["params"]), h, P(dev_in["u"]), P(dev_in["tok"]), 0, None, None,
                                      P(dev_in["keep"]), st)
    elif entry == "verify":
        rc = L.fs_verify(ctx, P(x), w.V, len(w.row_off) - 1, w.B, w.V, P(dev_in["rows"]), P(dev_in["roff"]),
                         P(dev_in["hist"]), P(dev_in["hoff"]), P(dev_in["params"]), P(dev_in["u"]), -1,
                         P(dev_in["tok"]), P(dev_in["acc"]), st)
    else:
        rc = L.fs_sample_batch(ctx, P(x), w.V, w.B, w.V, P(dev_in["hist"]), P(dev_in["hoff"]), P(dev_in["params"]),
                               P(dev_in["u"]), P(dev_in["tok"]), 0, None, None, P(dev_in["keep"]), st)
    if rc != 0:
        raise RuntimeError(f"call returned {rc}")


def phases(tr):
    """tr: [grid, TRACE_W] uint64 of one call -> dict of per-workgroup arrays (µs from the first start)."""
    role = tr[:, 13]
    t0 = tr[role > 0, 0].min()
    rel = (tr[:, :5].astype(np.int64) - np.int64(t0)) * TICK_US
    seg, mer = role == 1, role == 2
    tiles = (tr[:, 5:13].astype(np.int64) - np.int64(t0)) * TICK_US
    out = {"seg": rel[seg], "seg_row": tr[seg, 14], "mer": rel[mer], "mer_row": tr[mer, 14],
           "mer_set": tr[mer, :5] != 0, "seg_tiles": tiles[seg], "seg_tiles_set": tr[seg, 5:13] != 0}
    return out


def summarize(calls, seg_tiles):
    def stat(vals):
        v = np.asarray(vals, float)
        return (np.min(v), np.median(v), np.max(v)) if v.size else (np.nan,) * 3

    rows = []

    def add(name, per_call, per_wg):
        """per_call: list over calls of arrays (times); per_wg: list over calls of arrays (durations)."""
        t = np.median(np.array([stat(c) for c in per_call]), axis=0) if per_call else (np.nan,) * 3
        d = np.median([np.median(c) for c in per_wg]) if per_wg and all(len(c) for c in per_wg) else np.nan
        rows.append((name, *t, d))

    S = [c["seg"] for c in calls]
    M = [c["mer"] for c in calls]
    add("segment start", [s[:, 0] for s in S], [])
    add("segment: tile 0 arrived", [s[:, 1] for s in S], [s[:, 1] - s[:, 0] for s in S])
    add("segment: tile 0 done (penalty, bound, appends)", [s[:, 2] for s in S], [s[:, 2] - s[:, 1] for s in S])
    for t in range(1, min(seg_tiles, 8)):
        ok = [c["seg_tiles_set"][:, t] for c in calls]
        if all(o.any() for o in ok):
            add(f"segment: tile {t} done (slowest wave)", [c["seg_tiles"][o, t] for c, o in zip(calls, ok)],
                [c["seg_tiles"][o, t] - c["seg_tiles"][o, t - 1] for c, o in zip(calls, ok)])
    add(f"segment: last tile done ({seg_tiles - 1} more tiles)", [s[:, 3] for s in S],
        [(s[:, 3] - s[:, 2]) / max(seg_tiles - 1, 1) for s in S])
    add("segment: list published, counted done", [s[:, 4] for s in S], [s[:, 4] - s[:, 3] for s in S])
    add("merge start", [m[:, 0] for m in M], [])
    waits = []
    for c in calls:
        last = {}
        for r, t in zip(c["seg_row"], c["seg"][:, 4]):
            last[int(r)] = max(last.get(int(r), -1e9), t)
        waits.append(np.array([m[1] - last.get(int(r), m[1]) for r, m in zip(c["mer_row"], c["mer"])]))
    add("merge: row's segments seen done", [m[:, 1] for m in M], waits)
    fast = [c["mer_set"][:, 2] & c["mer_set"][:, 3] for c in calls]
    add("merge: candidates gathered (short merge)", [m[f, 2] for m, f in zip(M, fast)],
        [m[f, 2] - m[f, 1] for m, f in zip(M, fast)])
    add("merge: candidates ranked (short merge)", [m[f, 3] for m, f in zip(M, fast)],
        [m[f, 3] - m[f, 2] for m, f in zip(M, fast)])
    add("merge: row finished (softmax, top-p, draw, outputs)", [m[:, 4] for m in M],
        [m[f, 4] - m[f, 3] for m, f in zip(M, fast)])
    span = np.median([max(c["seg"][:, 4].max(), c["mer"][:, 4].max()) for c in calls])
    return rows, span


SK_PHASES = [(11, "logits in (transformed)"), (12, "lane maxima sorted"), (2, "bound (barrier)"),
             (3, "groups handed over"), (4, "candidates expanded"), (5, "list ranked and published"),
             (6, "ticket taken")]


def summarize_small_k(trs):
    """trs: list over calls of [grid, TRACE_W] uint64 (small-k kernel) -> (rows (name, min, median, max, per
    workgroup), span, median candidates per top-k segment)."""
    per = {}
    cands, spans = [], []
    for tr in trs:
        tr = tr[tr[:, 13] >= 3]
        t0 = np.int64(tr[:, 0].min())
        rel = lambda j: (tr[:, j].astype(np.int64) - t0) * TICK_US  # noqa: E731
        topk = tr[:, 11] != 0                          # greedy rows leave the selection slots unset
        mer = tr[:, 13] == 4
        per.setdefault("segment start", []).append((rel(0), None))
        prev = 0
        for j, name in SK_PHASES:
            sel = topk if j not in (5, 6) else np.ones_like(topk)     # greedy rows: start -> published -> ticket
            step = rel(j) - np.where(topk | (j == 6), rel(prev), rel(0))
            per.setdefault(name, []).append((rel(j)[sel], step[sel]))
            prev = j
        per.setdefault("lists folded (the row's last segment)", []).append((rel(7)[mer], (rel(7) - rel(6))[mer]))
        per.setdefault("row finished (softmax, top-p, draw)", []).append((rel(8)[mer], (rel(8) - rel(7))[mer]))
        cands.append(np.median(tr[topk, 9]) if topk.any() else np.nan)
        spans.append(rel(8)[mer].max())
    rows = []
    for name, vals in per.items():
        t = [np.percentile(v, [0, 50, 100]) for v, _ in vals if v.size]
        t = np.median(np.array(t), axis=0) if t else (np.nan,) * 3
        d = [np.median(x) for _, x in vals if x is not None and x.size]
        rows.append((name, *t, np.median(d) if d else np.nan))
    return rows, float(np.median(spans)), float(np.median(cands))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--workload", default="cfg3")
    ap.add_argument("--calls", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--route", choices=["device", "host"], default="device",
                    help="host: the host copy of the parameters goes along (the small-k kernel where it fits)")
    args = ap.parse_args()

    import torch
    import bench
    from ferro_amd import workloads as W

    ctor, entry, desc = bench.WORKLOADS[args.workload]
    w = getattr(W, ctor)()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    L = load()
    ctx = ctypes.c_void_p()
    if L.fs_create(ctypes.byref(ctx)) != 0:
        raise RuntimeError("fs_create failed")
    nrot = max(2, -(-2 * bench.MALL_BYTES // w.logits.nbytes))
    base = torch.from_numpy(w.logits).to(dev)
    bufs = [base] + [base.clone() for _ in range(nrot - 1)]
    dev_in = dict(params=torch.from_numpy(w.params.view(np.uint8).copy()).to(dev),
                  hist=torch.from_numpy(w.hist).to(dev), hoff=torch.from_numpy(w.hist_off).to(dev),
                  u=torch.from_numpy(w.u).to(dev), tok=torch.empty(w.B, dtype=torch.int32, device=dev),
                  keep=torch.empty(w.B, dtype=torch.int32, device=dev))
    if entry == "verify":
        dev_in.update(rows=torch.from_numpy(w.rows).to(dev), roff=torch.from_numpy(w.row_off).to(dev),
                      acc=torch.empty(len(w.row_off) - 1, dtype=torch.int32, device=dev))
    cap = 1 << 20
    trace = torch.zeros(cap, dtype=torch.int64, device=dev)
    hp = np.ascontiguousarray(w.params) if args.route == "host" else None
    for i in range(args.warmup):
        one_call(L, ctx, w, entry, bufs, dev_in, trace, i, torch, hp)
    calls, raws = [], []
    for c in range(args.calls):
        trace.zero_()
        torch.cuda.synchronize()
        if L.fs_trace_set(ctx, ctypes.c_void_p(trace.data_ptr()), cap) != 0:
            raise RuntimeError("fs_trace_set failed")
        one_call(L, ctx, w, entry, bufs, dev_in, trace, args.warmup + c, torch, hp)
        torch.cuda.synchronize()
        L.fs_trace_set(ctx, None, 0)
        tr = trace.cpu().numpy().view(np.uint64).reshape(-1, TRACE_W)
        used = tr[:, 13] > 0
        n = int(np.nonzero(used)[0].max()) + 1 if used.any() else 0
        if n == 0:
            raise RuntimeError("nothing traced (grid larger than the trace buffer?)")
        if int(tr[used, 13].max()) >= 3:
            raws.append(tr[:n].copy())
        else:
            calls.append(phases(tr[:n]))
        one_call(L, ctx, w, entry, bufs, dev_in, trace, args.warmup + c + 1, torch, hp)   # untraced spacer
    f = lambda v: "" if np.isnan(v) else f"{v:.2f}"  # noqa: E731
    if raws:
        rows, span, cand = summarize_small_k(raws)
        print(f"Phase timeline of one call of the small-k kernel, {desc} ({len(raws[0][raws[0][:, 13] >= 3])} "
              f"segment workgroups); µs from the first workgroup's start, median over {len(raws)} traced calls; "
              f"the per-workgroup column is the step from the previous phase:\n")
        print("| phase | first | median | last | per workgroup (median) |")
        print("|---|---|---|---|---|")
        for name, lo, med, hi, d in rows:
            print(f"| {name} | {f(lo)} | {f(med)} | {f(hi)} | {f(d)} |")
        print(f"\nFirst workgroup start to the last row finished: {span:.2f} µs; candidates per top-k segment "
              f"(median): {cand:.0f}")
        return
    tiles_row = w.V // 4096
    segs = int(np.median([len(c["seg"]) for c in calls]) / max(w.B, 1))
    seg_tiles = -(-tiles_row // max(segs, 1))
    rows, span = summarize(calls, seg_tiles)
    print(f"Phase timeline of one call, {desc} ({len(calls[0]['seg'])} segment workgroups of {seg_tiles} tiles, "
          f"{len(calls[0]['mer'])} merging workgroups); µs from the first workgroup's start, median over "
          f"{args.calls} traced calls:\n")
    print("| phase | first | median | last | per workgroup (median) |")
    print("|---|---|---|---|---|")
    for name, lo, med, hi, d in rows:
        print(f"| {name} | {f(lo)} | {f(med)} | {f(hi)} | {f(d)} |")
    print(f"\nFirst workgroup start to last workgroup end: {span:.2f} µs")


if __name__ == "__main__":
    main()
