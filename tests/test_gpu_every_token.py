"""Token-only calls (kcap = 0, as the server calls) on rows that sample from every token (top_k = 0 or >= V,
sampler.cpp:26-35: the segment kernel's whole-row path) against the oracle: tokens and kept counts, except where the
oracle's draw lies within 1e-6 of a cumulative boundary. Vocabulary sizes from 1 to 262144, temperatures, penalties
(rep < 1 too), softcap, min-p / top-p combinations, ties, NaN and infinite rows, draws at the extremes of u."""
import os
import sys

import numpy as np
import pytest
import torch

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

from ferro_amd import workloads as W  # noqa: E402
import ferro_amd as F  # noqa: E402
from oracle import oracle as O  # noqa: E402
from parity_util import bf16_valued, boundary_row  # noqa: E402

pytestmark = pytest.mark.gpu
NT = min(16, os.cpu_count() or 1)


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module", autouse=True)
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    F.sampler.Context.default()
    F.sampler.ROUTE = "host"
    yield
    torch.cuda.synchronize()


def _case(rows, params, hists, us, name):
    B = len(rows)
    logits = np.stack(rows).astype(np.float32)
    hist = np.concatenate([np.asarray(h, np.int32) for h in hists]) if hists else np.zeros(0, np.int32)
    off = np.concatenate([[0], np.cumsum([len(h) for h in hists])]).astype(np.int64)
    return W.Workload(name, logits, params, hist, off, np.asarray(us, np.float64), np.zeros(B, np.uint64))


def check(w, max_near=None):
    """Token-only call (kcap = 0) on the host route; the oracle with every candidate's probability. With every token
    a candidate, a row's cumulative sums step by less than 1e-6 wherever its probabilities are that small, so many
    draws count as near a boundary; rows may differ only there, and the count of those that do is printed."""
    say(f"case {w.name}: B={w.B} V={w.V}")
    x = torch.from_numpy(w.logits).cuda()
    out = F.sample_batch(x, w.params, w.u, hist=w.hist, hist_off=w.hist_off, kcap=0)
    torch.cuda.synchronize()
    g = {k: v.cpu().numpy() for k, v in out.items() if v is not None and not k.startswith("_")}
    o = O.sample_batch(w.logits, w.hist, w.hist_off, w.params, w.u, kcap=w.V, nthreads=NT)
    assert F.device_error() == 0
    near = differ = 0
    for b in range(w.B):
        p = w.params[b]
        m = int(o["ncand"][b])
        edge = m > 0 and boundary_row(o["cand_probs"][b, :m], int(o["keep"][b]), w.u[b], float(p["top_p"]),
                                      float(p["min_p"]))
        near += int(edge)
        if g["tok"][b] != o["tok"][b] or g["keep"][b] != o["keep"][b]:
            assert edge, (f"{w.name} row {b}: tok {g['tok'][b]} vs {o['tok'][b]}, keep {g['keep'][b]} vs "
                          f"{o['keep'][b]}")
            differ += 1
    say(f"  {w.name}: {near} rows near a boundary, {differ} of them differ")
    if max_near is not None:
        assert near <= max_near
    return g, o


def test_cfg3_rows_every_token():
    check(W.config3_all_tokens())


def test_bf16_valued_rows_every_token():
    w = W.config3_all_tokens()
    w.logits = bf16_valued(w.logits)
    w.name += "_bf16"
    check(w)


@pytest.mark.parametrize("V", [1, 7, 4096, 16384, 16385, 100003])
def test_vocab_sizes(V):
    rng = np.random.default_rng(V)
    B = 12
    rows = [(rng.standard_normal(V) * 2).astype(np.float32) for _ in range(B)]
    p = W.make_params(B, temperature=0.9, top_k=0, top_p=0.9, min_p=0.0, repetition_penalty=1.0)
    p["top_p"] = [1.0, 0.9, 0.5, 0.0, 0.99, 1.0, 0.7, 0.95, 1.0, 0.3, 0.8, 0.999][:B]
    p["min_p"] = [0.0, 0.0, 0.0, 0.0, 0.05, 0.2, 0.01, 0.5, 2.0, 0.1, 0.0, 0.001][:B]
    p["top_k"][1] = V + 5                                # k >= V is every token too
    check(_case(rows, p, [[]] * B, rng.random(B), f"vocab_{V}"))


@pytest.mark.parametrize("T", [0.05, 0.8, 3.0])
def test_temperatures_and_penalties(T):
    rng = np.random.default_rng(int(T * 100))
    V, B = 262144, 8
    rows, hists = [], []
    for b in range(B):
        r = (rng.standard_normal(V) * 1.5).astype(np.float32)
        r[rng.choice(V, 8, replace=False)] += rng.uniform(4, 12, 8).astype(np.float32)   # spikes
        rows.append(r)
        h = rng.integers(0, V, 600).astype(np.int32)
        h[:4] = np.argsort(-r)[:4]                       # the top tokens are penalised
        hists.append(h)
    p = W.make_params(B, temperature=T, top_k=0, top_p=0.95, min_p=0.0, repetition_penalty=1.1)
    p["repetition_penalty"][5] = 0.8                     # raises the penalised logits
    p["repetition_penalty"][6] = 1.0
    p["min_p"][3] = 0.05
    p["top_p"][4] = 1.0
    p["softcap"][7] = 30.0
    p["repeat_last_n"][2] = 64
    check(_case(rows, p, hists, rng.random(B), f"temperature_{T}"))


def test_ties_and_special_rows():
    """All-equal rows (every element in one bucket: refining rounds over the ids), a few distinct values, NaN and
    infinities."""
    V = 50000
    rng = np.random.default_rng(8)
    rows = []
    rows.append(np.zeros(V, np.float32))                              # all equal
    r = np.full(V, -1.0, np.float32); r[rng.choice(V, 3000, replace=False)] = 2.0; rows.append(r)
    r = np.round(rng.standard_normal(V) * 2).astype(np.float32); rows.append(r)      # integer-valued
    r = np.full(V, np.nan, np.float32); rows.append(r)                # every logit NaN
    r = (rng.standard_normal(V)).astype(np.float32); r[::7] = np.nan; rows.append(r)
    r = (rng.standard_normal(V)).astype(np.float32); r[123] = np.inf; rows.append(r)   # +inf maximum
    r = np.full(V, -np.inf, np.float32); rows.append(r)               # every logit -inf
    r = (rng.standard_normal(V)).astype(np.float32); r[::3] = -np.inf; rows.append(r)
    r = np.zeros(V, np.float32); r[V - 1] = 1e-3; r[0] = -0.0; rows.append(r)
    B = len(rows)
    p = W.make_params(B, temperature=1.0, top_k=0, top_p=0.9, min_p=0.0, repetition_penalty=1.0)
    p["top_p"][0] = 1.0
    p["min_p"][1] = 0.5
    p["top_p"][2] = 0.6
    p["min_p"][8] = 0.9
    check(_case(rows, p, [[]] * B, rng.random(B), "ties_special"))


@pytest.mark.parametrize("u", [0.0, 1e-12, 0.5, 1.0 - 2 ** -53])
def test_draw_extremes(u):
    rng = np.random.default_rng(11)
    V, B = 131072, 4
    rows = [(rng.standard_normal(V) * 3).astype(np.float32) for _ in range(B)]
    p = W.make_params(B, temperature=0.7, top_k=0, top_p=1.0, min_p=0.0, repetition_penalty=1.0)
    p["top_p"] = [1.0, 0.95, 0.5, 1.0]
    p["min_p"] = [0.0, 0.0, 0.0, 0.1]
    check(_case(rows, p, [[]] * B, np.full(B, u), f"draw_{u}"))


def test_deterministic_and_batch_invariant():
    w = W.config3_all_tokens(seed=5, B=16)
    x = torch.from_numpy(w.logits).cuda()
    a = F.sample_batch(x, w.params, w.u, hist=w.hist, hist_off=w.hist_off, kcap=0)["tok"].cpu().numpy()
    b = F.sample_batch(x, w.params, w.u, hist=w.hist, hist_off=w.hist_off, kcap=0)["tok"].cpu().numpy()
    assert np.array_equal(a, b)
    one = F.sample_batch(x[3:4].contiguous(), w.params[3:4], w.u[3:4], hist=w.hist[w.hist_off[3]:w.hist_off[4]],
                         hist_off=np.array([0, w.hist_off[4] - w.hist_off[3]], np.int64), kcap=0)["tok"].cpu().numpy()
    assert one[0] == a[3]


@pytest.mark.parametrize("seed", range(6))
def test_randomized(seed):
    rng = np.random.default_rng(100 + seed)
    B = int(rng.integers(1, 40))
    V = int(rng.integers(1, 300000))
    rows, hists = [], []
    for b in range(B):
        r = (rng.standard_normal(V) * rng.uniform(0.5, 4)).astype(np.float32)
        if rng.random() < 0.3:
            r[rng.choice(V, min(V, 5), replace=False)] += 10
        if rng.random() < 0.2:
            r = np.round(r)
        rows.append(r)
        hists.append(rng.integers(0, V, int(rng.integers(0, 800))).astype(np.int32))
    p = W.make_params(B, temperature=1.0, top_k=0, repetition_penalty=1.0)
    p["temperature"] = rng.uniform(0.1, 2.0, B)
    p["top_p"] = np.where(rng.random(B) < 0.3, 1.0, rng.uniform(0.0, 1.0, B))
    p["min_p"] = np.where(rng.random(B) < 0.6, 0.0, rng.uniform(0.0, 0.5, B))
    p["repetition_penalty"] = np.where(rng.random(B) < 0.5, 1.0, rng.uniform(0.8, 1.5, B))
    p["repeat_last_n"] = rng.choice([-1, 0, 16, 128], B)
    check(_case(rows, p, hists, rng.random(B), f"random_{seed}"))


def _spiky(rng, V, B):
    """Rows whose mass sits in a few spikes far above a N(0, 1.5) body: the case sampled from the logits within 16 T
    of the maximum (the rest summed), with targets inside the short list."""
    rows = []
    for b in range(B):
        r = (rng.standard_normal(V) * 1.5).astype(np.float32)
        n = int(rng.integers(1, 40))
        r[rng.choice(V, n, replace=False)] = rng.uniform(12, 40, n).astype(np.float32)
        if b % 5 == 0:
            r[rng.choice(V, 3, replace=False)] = r.max()      # ties at the maximum
        rows.append(r)
    return rows


@pytest.mark.parametrize("V", [262144, 100003])
def test_short_list_rows(V):
    rng = np.random.default_rng(V + 1)
    B = 24
    rows = _spiky(rng, V, B)
    p = W.make_params(B, temperature=1.0, top_k=0, repetition_penalty=1.0)
    p["temperature"] = rng.choice([0.3, 0.8, 1.0, 2.0], B)
    p["top_p"] = rng.choice([1.0, 0.95, 0.5, 0.99, 0.0], B)
    p["min_p"] = rng.choice([0.0, 0.0, 0.05, 1e-9, 0.5], B)      # 1e-9: min-p's boundary below the list
    p["top_k"][::7] = V + 3
    us = rng.random(B)
    us[::6] = 1.0 - 2 ** -53
    us[1::6] = 0.0
    hists = [np.argsort(-rows[b])[:3].astype(np.int32) if b % 3 == 0 else [] for b in range(B)]
    p["repetition_penalty"][::3] = 1.3                         # the top tokens penalised
    check(_case(rows, p, hists, us, f"short_list_{V}"))


def test_short_list_outputs_and_repeat():
    """Candidate outputs (kcap = 64) of short-list rows against the oracle (ids exact, probabilities to 1e-5
    relative), and a second call bit-identical (the short list's sums do not depend on the waves' timing)."""
    from parity_util import compare
    rng = np.random.default_rng(77)
    V, B, kcap = 262144, 12, 64
    rows = _spiky(rng, V, B)
    p = W.make_params(B, temperature=0.8, top_k=0, top_p=0.95, repetition_penalty=1.0)
    p["top_p"][::4] = 1.0
    p["min_p"][1::4] = 0.02
    w = _case(rows, p, [[]] * B, rng.random(B), "short_list_outputs")
    x = torch.from_numpy(w.logits).cuda()
    outs = []
    for _ in range(2):
        o = F.sample_batch(x, w.params, w.u, kcap=kcap)
        torch.cuda.synchronize()
        outs.append({k: v.cpu().numpy() for k, v in o.items() if v is not None and not k.startswith("_")})
    assert F.device_error() == 0
    ora = O.sample_batch(w.logits, w.hist, w.hist_off, w.params, w.u, kcap=kcap, nthreads=NT)
    compare(outs[0], ora, w.params, w.u, kcap)
    for k in ("tok", "keep", "cand_ids", "cand_probs"):
        assert np.array_equal(outs[0][k], outs[1][k]), k


@pytest.mark.parametrize("T", [1.0, 2.5])
def test_flat_rows_crowded_bins(T):
    """Flat rows (N(0, 1), or N(0, 2) at T 2.5): top-p's crossing and the draw fall in coarse bins holding thousands
    of logits, which the segments narrow with one level of finer bins before the exact walk. Also 2048 < k < V."""
    rng = np.random.default_rng(int(T * 10))
    V, B = 262144, 10
    rows = [(rng.standard_normal(V) * (1.0 if T < 2 else 2.0)).astype(np.float32) for _ in range(B)]
    p = W.make_params(B, temperature=T, top_k=0, repetition_penalty=1.0)
    p["top_p"] = [0.95, 0.5, 1.0, 0.9, 0.99, 0.7, 0.95, 0.8, 1.0, 0.6]
    p["min_p"] = [0.0, 0.0, 0.0, 0.05, 0.0, 0.3, 0.0, 0.0, 0.01, 0.0]
    p["top_k"][6] = 50000
    p["top_k"][7] = 3000
    hists = [rng.integers(0, V, 200).astype(np.int32) if b % 4 == 0 else [] for b in range(B)]
    p["repetition_penalty"][::4] = 1.2
    us = rng.random(B)
    us[0] = 1.0 - 2 ** -53
    check(_case(rows, p, hists, us, f"flat_T{T}"))
