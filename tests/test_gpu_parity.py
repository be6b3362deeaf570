"""GPU parity: the gfx950 kernels (through the C ABI) against the CPU oracle on identical seeded inputs.

Full configuration sizes are used where the oracle finishes in seconds (all five). Edge cases follow what the
reference's own code paths allow: empty histories, windows and scopes, out-of-range history ids, ties (incl.
-0/+0 and all-equal rows), top_k >= V, V = 1, V not a multiple of 4, NaN at index 0 for greedy.
"""
import ctypes
import os
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from oracle import oracle as O  # noqa: E402
from ferro_amd import workloads as W  # noqa: E402
import ferro_amd as F  # noqa: E402
from parity_util import bf16_valued, boundary_row, compare, oracle_decode_loop  # noqa: E402

NT = min(16, os.cpu_count() or 1)


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True, params=["host", "device"])
def gpu(request):
    """Every test runs twice: with the host copy of the parameters (fs_sample_batch_hp: the small-k kernel for the
    batches it fits) and with the device copy only (fs_sample_batch: the fused kernel for every batch)."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    F.sampler.Context.default()
    F.sampler.ROUTE = request.param
    say(f"== route {request.param}")
    yield
    F.sampler.ROUTE = "host"
    torch.cuda.synchronize()


def run_gpu(w, kcap):
    x = torch.from_numpy(w.logits).cuda()
    out = F.sample_batch(x, w.params, w.u, hist=w.hist, hist_off=w.hist_off, kcap=kcap)
    torch.cuda.synchronize()
    return {k: v.cpu().numpy() for k, v in out.items() if v is not None and not k.startswith("_")}


def run_oracle(w, kcap):
    return O.sample_batch(w.logits, w.hist, w.hist_off, w.params, w.u, kcap=kcap, nthreads=NT)


def check(w, kcap=None):
    if kcap is None:
        kk = np.where((w.params["top_k"] > 0) & (w.params["top_k"] < w.V), w.params["top_k"], w.V)
        kcap = int(min(max(kk.max(), 1), 2048))
    say(f"case {w.name}: B={w.B} V={w.V} kcap={kcap}")
    g = run_gpu(w, kcap)
    o = run_oracle(w, kcap)
    nb = compare(g, o, w.params, w.u, kcap)
    say(f"  {w.name}: {int(nb)} rows near a cumulative boundary, {nb.diverged} of them differ from the oracle")
    assert F.device_error() == 0
    return g, o, nb


def test_cfg1_single_row():
    g, o, nb = check(W.config1())
    assert nb == 0


def test_cfg1_golden_seeds():
    """The full config-1 row under 32 seeds: GPU tokens equal the reference's own (tests/golden)."""
    gold = np.load(os.path.join(os.path.dirname(__file__), "golden", "sampler_golden.npz"), allow_pickle=False)
    w = W.config1()
    n = len(gold["cfg1_seed"])
    x = torch.from_numpy(np.repeat(w.logits, n, axis=0)).cuda()
    hist = np.tile(w.hist, n)
    off = np.arange(n + 1, dtype=np.int64) * len(w.hist)
    u = np.array([W.first_u(int(s)) for s in gold["cfg1_seed"]])
    out = F.sample_batch(x, np.repeat(w.params, n), u, hist=hist, hist_off=off)
    np.testing.assert_array_equal(out["tok"].cpu().numpy(), gold["cfg1_tok"])


def test_cfg2_greedy_frequency_presence():
    w = W.config2()
    g, o, nb = check(w, kcap=1)
    np.testing.assert_array_equal(g["tok"], o["tok"])
    for b in w.meta["tie_rows"]:
        row = O.penalize(w.logits[b], w.hist[w.hist_off[b]:w.hist_off[b + 1]], w.params[b])
        assert g["tok"][b] == int(np.flatnonzero(row == row.max())[0])


def test_cfg2_argmax_entry_point():
    w = W.config2()
    x = torch.from_numpy(w.logits).cuda()
    tok = F.argmax_batch(x, hist=w.hist, hist_off=w.hist_off, params=w.params).cpu().numpy()
    o = run_oracle(w, 1)
    np.testing.assert_array_equal(tok, o["tok"])
    tok0 = F.argmax_batch(x).cpu().numpy()
    np.testing.assert_array_equal(tok0, w.logits.argmax(axis=1))


def test_cfg3_serving_batch_full():
    g, o, nb = check(W.config3())
    say(f"cfg3 boundary rows: {nb}")
    assert nb <= 1


def test_cfg4_verify_full():
    w = W.config4()
    say(f"case {w.name}: rows={w.B} V={w.V}")
    x = torch.from_numpy(w.logits).cuda()
    tok, acc = F.verify(x, w.rows, w.row_off, w.params, u=w.u, hist=w.hist, hist_off=w.hist_off)
    otok, oacc = O.verify(w.logits, w.rows, w.row_off, w.hist, w.hist_off, w.params, w.u)
    np.testing.assert_array_equal(tok.cpu().numpy(), otok)
    np.testing.assert_array_equal(acc.cpu().numpy(), oacc)
    assert (oacc > 1).any() and (oacc < 17).any()


@pytest.mark.parametrize("seed", [0, 1])
def test_verify_windows_lengths_and_eos(seed):
    """Verification windows without a penalty (the small-k kernel on the host route): streams of 1 to 40 rows (the
    one-atomic exchange takes windows of up to 32 rows, longer ones the token walk), drafts that match the row's
    argmax for a while and then stop, an eos token inside a window, greedy and sampled streams."""
    rng = np.random.default_rng(seed + 40)
    V = 8192
    lens = [1, 2, 5, 17, 31, 32, 33, 40]
    S = len(lens)
    row_off = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    R = int(row_off[-1])
    x = (rng.standard_normal((R, V)) * 2).astype(np.float32)
    am = np.argmax(x, axis=1)
    rows = rng.integers(0, V, R).astype(np.int32)
    for st in range(S):
        r0, m = int(row_off[st]), lens[st]
        good = int(rng.integers(0, m + 1))                     # drafts equal to the previous row's argmax
        for r in range(1, min(good, m)):
            rows[r0 + r] = am[r0 + r - 1]
    eos = int(am[int(row_off[3]) + 2])                          # stream 3's third row yields eos
    p = W.make_params(S, temperature=0.0, repetition_penalty=1.0)
    p["temperature"][1::3] = 0.9
    p["top_k"][1::3] = 40
    u = rng.random(R)
    hist = np.zeros(0, np.int32)
    hist_off = np.zeros(S + 1, np.int64)
    tok, acc = F.verify(torch.from_numpy(x).cuda(), rows, row_off, p, u=u, hist=hist, hist_off=hist_off, eos_id=eos)
    otok, oacc = O.verify(x, rows, row_off, hist, hist_off, p, u, eos_id=eos)
    np.testing.assert_array_equal(tok.cpu().numpy(), otok)
    np.testing.assert_array_equal(acc.cpu().numpy(), oacc)
    assert F.device_error() == 0


def test_verify_sampled_with_penalties():
    rng = np.random.default_rng(7)
    S, M, V = 6, 5, 3000
    x = (rng.standard_normal((S * M, V)) * 2).astype(np.float32)
    rows = rng.integers(0, 50, S * M).astype(np.int32)          # drafts from a small id range: penalties bite
    row_off = np.arange(0, S * M + 1, M, dtype=np.int64)
    hs = [rng.integers(0, 50, 30).astype(np.int32) for _ in range(S)]
    hist = np.concatenate(hs)
    off = np.arange(S + 1, dtype=np.int64) * 30
    p = W.make_params(S, temperature=0.9, top_k=20, top_p=0.9, repetition_penalty=1.4, frequency_penalty=0.2,
                      presence_penalty=0.1, repeat_last_n=40)
    p["temperature"][0] = 0.0
    u = rng.random(S * M)
    tok, acc = F.verify(torch.from_numpy(x).cuda(), rows, row_off, p, u=u, hist=hist, hist_off=off, eos_id=7)
    otok, oacc = O.verify(x, rows, row_off, hist, off, p, u, eos_id=7)
    np.testing.assert_array_equal(tok.cpu().numpy(), otok)
    np.testing.assert_array_equal(acc.cpu().numpy(), oacc)


def test_cfg5_heterogeneous_full():
    g, o, nb = check(W.config5())
    say(f"cfg5 boundary rows: {nb}")
    assert nb <= 3


@pytest.mark.parametrize("which", ["cfg3", "cfg5"])
def test_bf16_valued_rows(which):
    w = W.config3() if which == "cfg3" else W.config5(B=96)
    w.logits = bf16_valued(w.logits)
    w.name += "_bf16"
    g, o, nb = check(w)
    assert nb <= 3


def _case(rows, params, hists, us, name):
    B = len(rows)
    V = len(rows[0])
    logits = np.stack(rows).astype(np.float32)
    hist = np.concatenate([np.asarray(h, np.int32) for h in hists]) if hists else np.zeros(0, np.int32)
    off = np.concatenate([[0], np.cumsum([len(h) for h in hists])]).astype(np.int64)
    return W.Workload(name, logits, params, hist, off, np.asarray(us, np.float64), np.zeros(B, np.uint64))


def test_known_answer_through_gpu():
    row = np.array([0, 9, 10, 9.5, 6, 0], np.float32)
    want = {(-1, 0): 4, (-1, 2): 2, (2, 0): 1, (0, 0): 2, (2, 2): 2}
    p = W.make_params(5, temperature=0.0, repetition_penalty=2.0)
    for i, (ln, fr) in enumerate(want):
        p["repeat_last_n"][i] = ln
        p["penalty_from"][i] = fr
    w = _case([row] * 5, p, [[1, 2, 3]] * 5, np.zeros(5), "known_answer")
    g = run_gpu(w, 1)
    assert list(g["tok"]) == list(want.values())


def test_combined_penalties_hand_computed_on_device():
    """Repetition + frequency + presence over windows cut by repeat_last_n and penalty_from, on the device: the
    in-place penalty pass reproduces the hand-computed rows bit for bit, and the sampler's fused penalties give the
    same candidate order and probabilities (k = V, so every penalised logit is a candidate)."""
    row = np.array([4.0, -1.5, 3.0, 0.5, -2.0, 6.0, 1.0, -0.25, 2.5, 8.0], np.float32)
    h = [5, 5, 2, 9, 5, 1, 3, 9, 9, 7, 2, 12, -1, 5]
    cases = [(9, 2, [4.0, -3.75, 0.75, -0.5, -2.0, 2.25, 1.0, -1.25, 2.5, 2.75]),
             (9, 8, [4.0, -1.5, 0.75, 0.5, -2.0, 2.25, 1.0, -1.25, 2.5, 3.25]),
             (-1, 0, [4.0, -3.75, 0.25, -0.5, -2.0, 0.75, 1.0, -1.25, 2.5, 2.25])]
    B = len(cases)
    p = W.make_params(B, temperature=1.0, top_k=0, repetition_penalty=2.0, frequency_penalty=0.5,
                      presence_penalty=0.25)
    for i, (ln, fr, _) in enumerate(cases):
        p["repeat_last_n"][i] = ln
        p["penalty_from"][i] = fr
    hist = np.array(h * B, np.int32)
    hoff = np.arange(B + 1, dtype=np.int64) * len(h)
    x = torch.from_numpy(np.stack([row] * B)).cuda()
    y = F.sampler.penalize_batch(x.clone(), p, hist=hist, hist_off=hoff)
    torch.cuda.synchronize()
    want = np.array([c[2] for c in cases], np.float32)
    np.testing.assert_array_equal(y.cpu().numpy(), want)
    res = F.sample_batch(x, p, np.full(B, 0.5), hist=hist, hist_off=hoff, kcap=10)
    torch.cuda.synchronize()
    for i in range(B):
        order = sorted(range(10), key=lambda j: (-want[i][j], j))
        assert list(res["cand_ids"][i].cpu().numpy()) == order, i
        e = np.exp((want[i][order] - want[i][order[0]]).astype(np.float64))
        np.testing.assert_allclose(res["cand_probs"][i].cpu().numpy(), e / e.sum(), rtol=1e-12)
    assert F.device_error() == 0


@pytest.mark.parametrize("V", [1, 2, 6, 17, 1000, 4097, 8193, 65537, 100003])
def test_odd_vocab_sizes(V):
    rng = np.random.default_rng(V)
    B = 6
    rows = [(rng.standard_normal(V) * 2).astype(np.float32) for _ in range(B)]
    p = W.make_params(B, temperature=0.8, top_k=40, top_p=0.9, repetition_penalty=1.2)
    p["temperature"][0] = 0.0
    p["top_k"][1] = 0 if V <= 2048 else 2048
    p["top_k"][2] = V + 5 if V <= 2048 else 7
    hists = [rng.integers(0, V, 20) for _ in range(B)]
    g, o, nb = check(_case(rows, p, hists, rng.random(B), f"odd_V{V}"))
    assert nb == 0


def test_ties_and_signed_zeros():
    rng = np.random.default_rng(11)
    V = 40000
    rows = []
    rows.append(np.full(V, 1.5, np.float32))                                  # all equal: ties everywhere
    r = (np.round(rng.standard_normal(V) * 2) / 2).astype(np.float32)       # heavy ties
    rows.append(r)
    z = np.zeros(V, np.float32)
    z[rng.random(V) < 0.5] = -0.0                                            # -0 and +0 are equal
    rows.append(z)
    r2 = rng.standard_normal(V).astype(np.float32)
    r2[rng.choice(V, 500, replace=False)] = np.float32(9.0)                  # 500-way tie at the top
    rows.append(r2)
    B = len(rows)
    p = W.make_params(B, temperature=1.0, top_k=64, top_p=0.95, repetition_penalty=1.0)
    g, o, nb = check(_case(rows, p, [[]] * B, rng.random(B), "ties"))
    p2 = W.make_params(B, temperature=0.0, repetition_penalty=1.0)
    g2, o2, _ = check(_case(rows, p2, [[]] * B, np.zeros(B), "ties_greedy"), kcap=1)
    assert list(g2["tok"]) == [0, int(np.argmax(r)), 0, int(np.flatnonzero(r2 == 9.0)[0])]
    p3 = W.make_params(B, temperature=0.7, top_k=2048, repetition_penalty=1.0)
    check(_case(rows, p3, [[]] * B, rng.random(B), "ties_k2048"))


def test_greedy_nan_at_zero():
    V = 9000
    x = np.random.default_rng(3).standard_normal((2, V)).astype(np.float32)
    x[0, 0] = np.nan
    x[1, 5] = np.nan
    tok = F.argmax_batch(torch.from_numpy(x).cuda()).cpu().numpy()
    assert tok[0] == 0
    assert tok[1] == int(np.nanargmax(np.where(np.arange(V) == 5, -np.inf, x[1])))


def test_penalty_windows_and_out_of_range_ids():
    rng = np.random.default_rng(5)
    V, B = 20000, 12
    rows = [(rng.standard_normal(V) * 2).astype(np.float32) for _ in range(B)]
    hists = []
    for b in range(B):
        h = rng.integers(-5, V + 5, int(rng.integers(0, 3000))).astype(np.int32)
        h[:5] = np.argsort(-rows[b])[:5]                # the top tokens are penalised
        hists.append(h)
    hists[3] = np.zeros(0, np.int32)                    # empty history
    p = W.make_params(B, temperature=1.0, top_k=50, top_p=0.9, repetition_penalty=1.5,
                      frequency_penalty=0.3, presence_penalty=0.2)
    p["repeat_last_n"] = [-1, 0, 1, 7, 100, 5000, -1, -1, 64, -1, 3, -1]
    p["penalty_from"] = [0, 0, 0, 3, 10, 0, 2999, 100000, 0, 0, 0, 1]
    p["repetition_penalty"][9] = 0.7
    p["frequency_penalty"][10] = 0.0
    p["presence_penalty"][10] = 0.0
    p["temperature"][11] = 0.0
    g, o, nb = check(_case(rows, p, hists, rng.random(B), "penalty_windows"))
    assert nb == 0


def test_penalised_top_of_a_segment_below_the_bound():
    """rep >= 1 on the small-k kernel: the segment's bound is taken over the raw logits and the penalty applied to the
    handed-over ones. Here the window holds most of a segment's largest logits and a strong penalty drops them below
    that bound, so fewer than k candidates stay at or above it: the segment must take its exact path. Also rep < 1
    (penalised before the bound) and greedy rows."""
    rng = np.random.default_rng(17)
    V, B = 65536, 8
    rows, hists = [], []
    for b in range(B):
        r = (rng.standard_normal(V) * 1.5).astype(np.float32)
        hot = rng.choice(16384, 200, replace=False) + 16384 * (b % 4)     # 200 large logits in one segment
        r[hot] = rng.uniform(10.0, 20.0, 200).astype(np.float32)
        order = hot[np.argsort(-r[hot])]
        rows.append(r)
        hists.append(order[:150].astype(np.int32))                          # its 150 largest are penalised
    p = W.make_params(B, temperature=1.0, top_k=64, top_p=1.0, repetition_penalty=3.0)
    p["top_k"] = [64, 64, 40, 8, 4, 2, 64, 1]
    p["repetition_penalty"][6] = 0.5                                        # rep < 1 raises the penalised logits
    p["temperature"][7] = 0.0
    g, o, nb = check(_case(rows, p, hists, rng.random(B), "penalised_top_of_a_segment"))
    assert nb == 0


def test_count_penalties_by_wave_and_by_table():
    """Frequency / presence counts (sampler.cpp:11-18 plus the extension) on 8-tile segments (B=64 x V=262144), where
    each segment buckets its window ids by tile and every wave counts its own logits, next to the per-tile table
    that a segment with more than 2048 window ids keeps: Zipf windows, a 6000-id window inside segment 0, one id
    repeated 300 times, ids on every wave's logits of one tile, a one-id window and an empty one; greedy, k <= 64
    and k > 64 rows, and whole-row (top_k = 0, k > 2048) rows with the 6000-id window. (A window with more than
    2048 ids in a segment was once counted twice: the gathered ids and then the whole window again.)"""
    V, B = 262144, 64
    rng = np.random.default_rng(64)
    rows = list(W.mixture_logits(rng, B, V))
    hists = [W.zipf_ids(rng, V, 1024) for _ in range(B)]
    for b in range(0, B, 8):
        hists[b] = rng.integers(0, 8 * 4096, 6000).astype(np.int32)           # > 2048 ids in segment 0
    for b in range(1, B, 8):
        top = int(np.argmax(rows[b]))
        hists[b] = np.concatenate([np.full(300, top, np.int32), W.zipf_ids(rng, V, 200)])   # a count of 300
    for b in range(2, B, 8):
        t = int(rng.integers(0, V // 4096)) * 4096                            # one tile, every wave's logits
        hists[b] = (t + np.arange(0, 4096, 7)).astype(np.int32)
    hists[3] = np.array([int(np.argmax(rows[3]))], np.int32)
    hists[4] = np.zeros(0, np.int32)
    p = W.make_params(B, temperature=0.9, top_k=40, top_p=0.95, repetition_penalty=1.1,
                      frequency_penalty=0.6, presence_penalty=0.4)
    p["top_k"][::3] = 700
    p["temperature"][::5] = 0.0
    p["repetition_penalty"][::4] = 1.0
    p["presence_penalty"][1::4] = 0.0
    p["top_k"][48], p["top_k"][56] = 0, 3000                                 # whole-row path, long windows
    g, o, nb = check(_case(rows, p, hists, rng.random(B), "count_penalties"), kcap=700)
    assert nb <= 1


@pytest.mark.parametrize("V", [65536, 262144])
def test_count_overflow_is_reported(V):
    """A window holding one id 70000 times overflows the 16-bit penalty counts: the call reports
    FS_DEVERR_COUNT_OVERFLOW (small-k kernel at V=65536 on the host route, fused kernel otherwise), and the next
    clean call reports nothing."""
    from ferro_amd._lib import FS_DEVERR_COUNT_OVERFLOW
    rng = np.random.default_rng(V)
    x = torch.from_numpy(rng.standard_normal((2, V)).astype(np.float32)).cuda()
    hist = np.concatenate([np.full(70000, 123, np.int32), np.arange(10, dtype=np.int32)])
    hist_off = np.array([0, 70000, 70010], np.int64)
    p = W.make_params(2, temperature=0.0, repetition_penalty=1.0, frequency_penalty=0.5)
    F.sample_batch(x, p, np.zeros(2), hist=hist, hist_off=hist_off)
    torch.cuda.synchronize()
    assert F.device_error() & FS_DEVERR_COUNT_OVERFLOW
    hist2 = np.arange(20, dtype=np.int32)
    F.sample_batch(x, p, np.zeros(2), hist=hist2, hist_off=np.array([0, 10, 20], np.int64))
    torch.cuda.synchronize()
    assert F.device_error() == 0


@pytest.mark.parametrize("B,V", [(8, 65536), (40, 65536), (64, 262144)])
def test_greedy_rows_with_every_penalty(B, V):
    """Greedy rows with repetition (above and below 1), frequency and presence penalties, windows cut by
    repeat_last_n / penalty_from, the row's maximum repeated 300 times, ids past V and negative ids, an id on every
    logit of a 4096-logit segment, and penalties that lower the maximum below its runner-up in another segment. On the
    host route the small-k kernel takes them (greedy rows apply the penalties before their maximum; frequency /
    presence counts on 4096-logit segments: B=8 and B=40 at V=65536); at B=64 x V=262144 the fused kernel does."""
    rng = np.random.default_rng(B + 7)
    rows = [rng.standard_normal(V).astype(np.float32) * 2 for _ in range(B)]
    hists = []
    for b in range(B):
        top = int(np.argmax(rows[b]))
        second = int(np.argsort(rows[b])[-2])
        kind = b % 8
        if kind == 0:
            h = np.concatenate([np.full(300, top, np.int32), W.zipf_ids(rng, V, 200)])
        elif kind == 1:
            h = np.array([top, top, second, V + 5, -3, top], np.int32)
        elif kind == 2:
            t = int(rng.integers(0, V // 4096)) * 4096
            h = (t + np.arange(4096)).astype(np.int32)                   # every logit of one segment
        elif kind == 3:
            h = np.zeros(0, np.int32)
        elif kind == 4:
            h = np.concatenate([W.zipf_ids(rng, V, 700), np.full(5, top, np.int32)])
        else:
            h = W.zipf_ids(rng, V, 256)
        hists.append(h)
    p = W.make_params(B, temperature=0.0, repetition_penalty=1.1, frequency_penalty=0.5, presence_penalty=0.3)
    p["repetition_penalty"][2::8] = 0.8                                      # rep < 1 raises the flagged logits
    p["frequency_penalty"][3::8] = 0.0
    p["presence_penalty"][5::8] = 0.0
    p["frequency_penalty"][6::8] = -0.5                                      # negative: the counted logits rise
    p["repeat_last_n"][4::8] = 3                                             # only the last three ids
    p["penalty_from"][5::8] = 100
    p["top_k"][7::8] = 1                                                     # greedy through top_k = 1 (T > 0)
    p["temperature"][7::8] = 0.9
    g, o, nb = check(_case(rows, p, hists, rng.random(B), "greedy_penalties"), kcap=1)
    assert nb == 0


@pytest.mark.parametrize("B,V", [(203, 65536), (130, 262144)])
def test_balanced_layouts(B, V):
    """Batches with 16 to 64 rows per XCD, where each XCD apportions its segment workgroups over its rows by their
    sampling settings (XCDs holding one row more or less when B is not a multiple of 8): greedy, small and large
    k, k > 2048 and top_k = 0 (whole-row rows whose segments meet at row barriers), penalties and softcap mixed."""
    rng = np.random.default_rng(B)
    x = W.mixture_logits(rng, B, V)
    p = W.make_params(B, temperature=0.9)
    p["temperature"] = rng.choice([0.0, 0.5, 0.9, 1.4], B)
    p["top_k"] = rng.choice([1, 8, 64, 200, 1000, 2048, 3000, 0], B)
    p["top_p"] = rng.choice([1.0, 0.9], B)
    p["min_p"] = rng.choice([0.0, 0.0, 0.05], B)
    p["repetition_penalty"] = rng.choice([1.0, 1.2], B)
    p["frequency_penalty"] = rng.choice([0.0, 0.5], B)
    p["presence_penalty"] = rng.choice([0.0, 0.3], B)
    p["softcap"][::7] = 30.0
    hists = [W.zipf_ids(rng, V, int(rng.integers(0, 600))) for _ in range(B)]
    g, o, nb = check(_case(list(x), p, hists, rng.random(B), f"balanced_B{B}_V{V}"), kcap=256)
    assert nb <= 2


@pytest.mark.parametrize("which", ["cfg3", "cfg5", "topk0"])
def test_token_only_calls(which):
    """Calls without candidate outputs (kcap = 0, as the server and bench.py call): tokens and kept counts equal
    the oracle's, except where the draw lies within 1e-6 of a cumulative boundary (counted)."""
    w = {"cfg3": W.config3, "cfg5": W.config5, "topk0": W.config3_all_tokens}[which]()
    kk = np.where((w.params["top_k"] > 0) & (w.params["top_k"] < w.V), w.params["top_k"], w.V)
    kcap = int(min(max(kk.max(), 1), w.V))
    say(f"case {w.name}: B={w.B} V={w.V}, GPU kcap=0, oracle kcap={kcap}")
    g = run_gpu(w, 0)
    o = run_oracle(w, kcap)
    assert F.device_error() == 0
    near = differ = 0
    for b in range(w.B):
        p = w.params[b]
        if p["temperature"] <= 0 or p["top_k"] == 1:
            assert g["tok"][b] == o["tok"][b], f"row {b} greedy token"
            continue
        m = int(o["ncand"][b])
        edge = boundary_row(o["cand_probs"][b, :m], int(o["keep"][b]), w.u[b], float(p["top_p"]), float(p["min_p"]))
        near += int(edge)
        if g["tok"][b] != o["tok"][b] or g["keep"][b] != o["keep"][b]:
            assert edge, f"row {b}: tok {g['tok'][b]} vs {o['tok'][b]}, keep {g['keep'][b]} vs {o['keep'][b]}"
            differ += 1
    say(f"  {w.name}: {near} rows near a boundary, {differ} of them differ")
    assert near <= 2


def test_large_k_full_vocab():
    """k > 2048 (top_k = 0 is ferro's k = n, sampler.cpp:26): the whole-row path, with every candidate's
    probability compared (kcap = V) and the draw at the extremes of u."""
    V = 65536
    rng = np.random.default_rng(21)
    B = 10
    rows = [(rng.standard_normal(V) * 2).astype(np.float32) for _ in range(B)]
    rows[6] = (np.round(rows[6] * 2) / 2).astype(np.float32)             # heavy ties
    p = W.make_params(B, temperature=1.0, top_k=0, top_p=1.0, repetition_penalty=1.0)
    p["temperature"][1], p["top_p"][1] = 0.7, 0.9
    p["temperature"][2], p["min_p"][2] = 1.5, 0.05
    p["top_k"][3], p["top_p"][3], p["repetition_penalty"][3] = 5000, 0.95, 1.3
    p["top_k"][4], p["temperature"][4] = 2049, 0.8
    p["temperature"][5], p["top_p"][5], p["min_p"][5] = 2.0, 0.5, 0.01
    p["frequency_penalty"][5], p["presence_penalty"][5], p["repetition_penalty"][5] = 0.3, 0.2, 1.1
    p["top_k"][7] = V - 1
    hists = [rng.integers(0, V, 200) for _ in range(B)]
    u = rng.random(B)
    u[8], u[9] = 0.0, 1.0 - 2.0 ** -40
    g, o, nb = check(_case(rows, p, hists, u, "large_k"), kcap=V)
    say(f"large_k boundary rows: {nb}")
    assert nb <= 1


def test_large_k_serving_rows_mixed_with_topk():
    """cfg5-shaped rows (V = 262144, H = 1024, frequency / presence) where some rows ask for top_k = 0."""
    w = W.config5(B=12)
    w.params["top_k"][::3] = 0
    w.params["temperature"][::3] = np.maximum(w.params["temperature"][::3], 0.3)
    g, o, nb = check(w, kcap=16)
    assert nb == 0


def test_buffer_pressure_multi_tile_segments():
    """Segments of 8 tiles (B = 256, V = 65536) with k up to 2048: the candidate buffer is compacted under load and
    the row bound is refreshed from counts at every check. Some rows rise tile after tile (every logit beats the
    running bound: the buffer overflows and the segment is streamed again in safe mode); some are constant
    (every logit ties)."""
    rng = np.random.default_rng(31)
    B, V = 256, 65536
    x = (rng.standard_normal((B, V)) * 1.5).astype(np.float32)
    x[::17] = np.sort(x[::17], axis=1)                                # ascending rows
    x[5] = 0.25
    p = W.make_params(B, temperature=0.9, top_k=2048, top_p=0.97, repetition_penalty=1.1)
    p["top_k"][1::4] = 1500
    p["top_k"][2::4] = 300
    p["top_k"][3::8] = 64
    p["frequency_penalty"][::5], p["presence_penalty"][::5] = 0.4, 0.2
    hists = [rng.integers(0, V, 300) for _ in range(B)]
    u = rng.random(B)
    g, o, nb = check(_case(list(x), p, hists, u, "buffer_pressure"), kcap=2048)
    say(f"buffer_pressure boundary rows: {nb}")
    assert nb <= 8                              # 256 rows of up to 2048 fp64 probabilities: draws near a c_i


def test_candidate_sort_tie_clusters():
    """The candidate sort bins the composites (key, id) over their span; a cluster of tied logits inside a spread
    of distinct ones puts more entries in one bin than the binned sort handles, and the sort falls back to the
    bitonic network. Rows mix both, for k on the small-list path (<= 512 reach the threshold) and on the KMAX
    path, with the candidate outputs compared in full."""
    rng = np.random.default_rng(47)
    B, V = 32, 65536
    x = (rng.standard_normal((B, V)) * 2.0).astype(np.float32)
    for b in range(0, B, 2):                                        # ties: 60 .. 1900 logits at one value
        n = int(60 + (b * 61) % 1840)
        idx = rng.choice(V, n, replace=False)
        x[b, idx] = np.float32(x[b].max() - 0.5 - 0.1 * (b % 3))
    x[3, :3000] = np.float32(4.0)                                   # a constant block above a tail
    x[9, ::2] = np.float32(-1.0)
    p = W.make_params(B, temperature=0.8, top_k=2048, top_p=0.99, repetition_penalty=1.0)
    p["top_k"][1::4] = 100
    p["top_k"][2::4] = 300
    p["top_k"][3::4] = 700
    u = rng.random(B)
    g, o, nb = check(_case(list(x), p, [np.zeros(0, np.int64)] * B, u, "tie_clusters"), kcap=2048)
    say(f"tie_clusters boundary rows: {nb}")
    assert nb <= 6                              # tied probabilities: many equal steps of the cumulative sum


def test_large_k_candidate_chunks():
    """k > 2048 (top_k = 0: the whole row): candidates are written in sorted chunks of 2048 past the first."""
    rng = np.random.default_rng(53)
    B, V = 4, 9000
    x = (rng.standard_normal((B, V)) * 1.5).astype(np.float32)
    x[1, 100:4000] = np.float32(0.5)
    p = W.make_params(B, temperature=1.0, top_k=0, top_p=0.9, repetition_penalty=1.0)
    u = rng.random(B)
    g, o, nb = check(_case(list(x), p, [np.zeros(0, np.int64)] * B, u, "large_chunks"), kcap=5000)
    assert nb <= 1


def test_large_k_coarse_bins_min_p_ties():
    """Large k through coarse key bins: top_k = 0 and 2048 < k < V (the k-th composite narrowed inside its bin),
    top-p on and off, min-p binding and not, penalties; rows with a block of > 2048 tied logits (a bin the LDS
    gather cannot hold: the exact multi-pass fallback) and with -inf entries."""
    rng = np.random.default_rng(61)
    B, V = 12, 20000
    x = (rng.standard_normal((B, V)) * 1.5).astype(np.float32)
    x[2, 1000:4500] = np.float32(5.0)                                # 3500 ties above the rest: top-p crosses inside
    x[5, ::3] = np.float32(-np.inf)
    x[7, 5000:7600] = np.float32(-0.3)
    p = W.make_params(B, temperature=0.9, top_k=0, top_p=0.9, repetition_penalty=1.1)
    p["top_k"][1::3] = 3000
    p["top_k"][2::6] = 2500
    p["top_p"][::4] = 1.0
    p["min_p"][1::4] = 0.05
    p["min_p"][3::4] = 0.3
    p["top_k"][2], p["top_p"][2] = 0, 0.5
    p["frequency_penalty"][::5] = 0.3
    hists = [rng.integers(0, V, 400) for _ in range(B)]
    u = rng.random(B)
    g, o, nb = check(_case(list(x), p, hists, u, "large_k_bins"), kcap=3000)
    say(f"large_k_bins boundary rows: {nb}")
    assert nb <= 2


def test_large_k_extremes_from_segments_and_tail():
    """top_k = 0 rows take their extremes and ordered count from the segments' published summaries plus the row's
    partial last tile: the maximum or the minimum in that tail (penalised), a segment holding only -inf, a segment
    of one repeated value, and a row shorter than one tile (no segments). Every candidate's order is compared."""
    rng = np.random.default_rng(71)
    for V in (3 * 4096 + 37, 1000):
        B = 6
        x = (rng.standard_normal((B, V)) * 2).astype(np.float32)
        x[0, V - 3] = np.float32(14.0)                               # the maximum in the tail, penalised below
        x[1, V - 1] = np.float32(-40.0)                              # the minimum in the tail
        x[2, 4096:8192 if V > 8192 else V // 2] = np.float32(-np.inf)
        x[2, V - 20] = np.float32(9.0)
        x[3, : min(4096, V // 2)] = np.float32(1.25)
        x[5, V - 2] = np.float32(12.0)
        p = W.make_params(B, temperature=1.0, top_k=0, top_p=1.0, repetition_penalty=1.3)
        p["top_p"][1] = 0.9
        p["min_p"][2] = 0.02
        p["temperature"][3], p["top_p"][3] = 0.7, 0.95
        p["frequency_penalty"][4], p["presence_penalty"][4] = 0.5, 0.25
        p["frequency_penalty"][5], p["presence_penalty"][5] = 2.0, 1.0
        hists = [rng.integers(0, V, 150) for _ in range(B)]
        hists[0] = np.concatenate([hists[0], [V - 3] * 3])
        hists[5] = np.concatenate([hists[5], [V - 2] * 4, [V - 1]])
        g, o, nb = check(_case(list(x), p, hists, rng.random(B), f"large_k_tail{V}"), kcap=V)
        say(f"large_k_tail{V} boundary rows: {nb}")
        assert nb <= 1


def test_device_logits_handoff_in_place():
    """The producer side of the boundary (ferro copies the lm_head output to the host first,
    model_lfm2_lm.cpp:477-480): logits computed on the device by an lm_head matmul land in a padded [B, ld] buffer
    (ld > V, as a model's aligned output) and are sampled from that buffer in place - no host copy and no repack.
    The oracle samples the same logits, copied to the host for it alone."""
    torch.manual_seed(5)
    B, d, V, ld = 16, 256, 50000, 50048
    hidden = torch.randn(B, d, device="cuda")
    w_head = torch.randn(d, V, device="cuda") * 0.08
    out = torch.zeros(B, ld, device="cuda")
    out[:, :V] = hidden @ w_head
    fed, fed_ld, n = F.sampler._check_logits(out, V)
    assert fed.data_ptr() == out.data_ptr() and fed_ld == ld and n == V     # the model's own buffer, unrepacked
    rng = np.random.default_rng(17)
    p = W.make_params(B, temperature=0.7, top_k=64, top_p=0.9, repetition_penalty=1.1)
    p["top_k"][::4] = 0
    p["temperature"][3] = 0.0
    hists = [rng.integers(0, V, 128) for _ in range(B)]
    hist = np.concatenate(hists).astype(np.int32)
    hoff = np.concatenate([[0], np.cumsum([len(h) for h in hists])]).astype(np.int64)
    u = rng.random(B)
    res = F.sample_batch(out, p, u, hist=hist, hist_off=hoff, V=V, kcap=64)
    torch.cuda.synchronize()
    g = {k: v.cpu().numpy() for k, v in res.items() if v is not None and not k.startswith("_")}
    w = _case(list(out[:, :V].cpu().numpy()), p, hists, u, "handoff")
    ref = run_oracle(w, 64)
    nb = compare(g, ref, p, u, 64)
    assert nb <= 1
    # the same buffer passed as the view out[:, :V] (B > 1: not contiguous, row stride ld): read in place too
    view = out[:, :V]
    assert not view.is_contiguous()
    fed, fed_ld, _ = F.sampler._check_logits(view, None)
    assert fed.data_ptr() == out.data_ptr() and fed_ld == ld
    res2 = F.sample_batch(view, p, u, hist=hist, hist_off=hoff, kcap=64)
    torch.cuda.synchronize()
    g2 = {k: v.cpu().numpy() for k, v in res2.items() if v is not None and not k.startswith("_")}
    for k in ("tok", "keep"):
        np.testing.assert_array_equal(g2[k], g[k], err_msg=f"view {k}")
    for b in range(B):                                  # the candidates each row defines (greedy rows: one)
        m = min(int(ref["ncand"][b]), 64)
        np.testing.assert_array_equal(g2["cand_ids"][b, :m], g["cand_ids"][b, :m], err_msg=f"view ids row {b}")
        np.testing.assert_array_equal(g2["cand_probs"][b, :m], g["cand_probs"][b, :m], err_msg=f"view probs row {b}")
    pg = W.make_params(B, temperature=0.0, repetition_penalty=1.1)
    np.testing.assert_array_equal(F.argmax_batch(view, hist=hist, hist_off=hoff, params=pg).cpu().numpy(),
                                  F.argmax_batch(out, hist=hist, hist_off=hoff, params=pg, V=V).cpu().numpy())
    assert F.device_error() == 0


@pytest.mark.parametrize("seed", range(16))
def test_randomized_sweep(seed):
    """Seeded random batches against the oracle: B not a multiple of 8, V from 1 to ~70000 (rows shorter than a
    tile, exact tiles, ragged tails), k from 1 to V and 0, top-p, min-p, repetition / frequency / presence
    penalties with windows and scopes, -inf entries, NaN in greedy rows (ferro's candidate sort is undefined with
    NaN; its greedy scan is not), and the Gemma 4 softcap on unclipped rows (the device restates the host C
    library's tanhf bit for bit, so capped rows are held to the same exact bar)."""
    rng = np.random.default_rng(1000 + seed)
    for case in range(4):
        B = int(rng.integers(1, 40))
        V = int(rng.choice([1, 3, 100, 4095, 4096, 4097, 12288, 20000, 65536, 70001]))
        x = (rng.standard_normal((B, V)) * rng.uniform(0.5, 4.0)).astype(np.float32)
        p = W.make_params(B, temperature=0.8)
        p["temperature"] = rng.choice([0.0, 0.3, 0.8, 1.5], B)
        p["top_k"] = rng.choice([0, 1, 5, 40, 64, 300, 2048, 3000, V + 5], B)
        if V > 10:
            for b in range(0, B, 5):
                if p["temperature"][b] <= 0 or p["top_k"][b] == 1:    # NaN: defined for ferro's greedy scan only
                    x[b, rng.integers(0, V, 3)] = np.float32(np.nan)  # (its candidate sort has no order for it)
                x[b, rng.integers(0, V, 2)] = np.float32(-np.inf)
            if B > 2:
                x[2, : V // 3] = np.float32(1.25)                       # a tied block
        p["top_p"] = rng.choice([1.0, 0.95, 0.6], B)
        p["min_p"] = rng.choice([0.0, 0.0, 0.05], B)
        p["repetition_penalty"] = rng.choice([1.0, 1.1, 1.3], B)
        p["frequency_penalty"] = rng.choice([0.0, 0.0, 0.4], B)
        p["presence_penalty"] = rng.choice([0.0, 0.2], B)
        p["repeat_last_n"] = rng.choice([-1, 0, 16], B)
        p["penalty_from"] = rng.choice([0, 0, 3], B)
        p["softcap"] = rng.choice([0.0, 0.0, 30.0, 2.5], B)
        hists = [rng.integers(-2, V + 2, int(rng.integers(0, 300))) for _ in range(B)]
        u = rng.random(B)
        kk = np.where((p["top_k"] > 0) & (p["top_k"] < V), p["top_k"], V)
        kcap = int(min(max(int(kk.max()), 1), 2048))
        g, o, nb = check(_case(list(x), p, hists, u, f"sweep{seed}.{case}"), kcap=kcap)
        assert nb <= 3


def test_verify_large_k():
    rng = np.random.default_rng(8)
    S, M, V = 3, 4, 3000
    x = (rng.standard_normal((S * M, V)) * 3).astype(np.float32)
    rows = rng.integers(0, V, S * M).astype(np.int32)
    row_off = np.arange(0, S * M + 1, M, dtype=np.int64)
    x[np.arange(S * M - 1), rows[1:]] += 30.0                        # drafts the model agrees with
    p = W.make_params(S, temperature=0.5, top_k=0, top_p=0.9, repetition_penalty=1.0)
    u = rng.random(S * M)
    tok, acc = F.verify(torch.from_numpy(x).cuda(), rows, row_off, p, u=u)
    otok, oacc = O.verify(x, rows, row_off, np.zeros(0, np.int32), np.zeros(S + 1, np.int64), p, u)
    np.testing.assert_array_equal(tok.cpu().numpy(), otok)
    np.testing.assert_array_equal(acc.cpu().numpy(), oacc)
    assert F.device_error() == 0


def test_batch_invariance_and_determinism():
    w = W.config3(B=16)
    g1, _, _ = check(w, kcap=64)
    g2 = run_gpu(w, 64)
    for k in g1:
        np.testing.assert_array_equal(g1[k], g2[k])
    # each row alone (a different chunking path) gives the same result
    for b in [0, 7, 15]:
        one = W.Workload("one", w.logits[b:b + 1], w.params[b:b + 1], w.hist[w.hist_off[b]:w.hist_off[b + 1]],
                         np.array([0, w.hist_off[b + 1] - w.hist_off[b]]), w.u[b:b + 1], w.seeds[b:b + 1])
        g = run_gpu(one, 64)
        for k in g1:
            np.testing.assert_array_equal(g[k][0], g1[k][b])


def test_sampler_shim_reproduces_reference_streams():
    """ferro_amd.Sampler (the ferro::Sampler mirror) replays the reference's own 40-call streams token for token."""
    gold = np.load(os.path.join(os.path.dirname(__file__), "golden", "sampler_golden.npz"), allow_pickle=False)
    params = gold["stream_params"].view(W.PARAMS_DTYPE) if hasattr(W, "PARAMS_DTYPE") else \
        gold["stream_params"].view(F.PARAMS_DTYPE)
    for s in range(len(params)):
        q = params[s]
        sp = F.SamplerParams(temperature=float(q["temperature"]), top_k=int(q["top_k"]), top_p=float(q["top_p"]),
                             min_p=float(q["min_p"]), repetition_penalty=float(q["repetition_penalty"]),
                             repeat_last_n=int(q["repeat_last_n"]), penalty_from=int(q["penalty_from"]),
                             seed=int(gold["stream_seed"][s]))
        smp = F.Sampler(sp)
        hist = list(gold["stream_h0"][s])
        for i, row in enumerate(gold["stream_x"][s]):
            t = smp.sample(torch.from_numpy(row).cuda(), row.size, hist)
            assert t == gold["stream_tok"][s][i], (s, i)
            hist.append(t)


def test_greedy_infinities_and_nan_rows():
    """ferro's scan (sampler.cpp:21): the first index strictly above logits[0]'s running best; -inf / NaN rows."""
    V = 3 * 4096 + 77                                   # full tiles plus a partial tail
    rows = []
    r = np.full(V, -np.inf, np.float32); rows.append(r)                      # all -inf -> 0
    r = np.full(V, -np.inf, np.float32); r[V - 5] = np.nan; rows.append(r)   # -inf and NaN -> 0
    r = np.full(V, np.nan, np.float32); r[4100] = -np.inf; rows.append(r)    # NaN at 0 -> 0
    r = np.full(V, -np.inf, np.float32); r[V - 3] = -1.0; rows.append(r)     # max in the tail
    r = np.full(V, -np.inf, np.float32); r[5000] = np.inf; r[V - 2] = np.inf; rows.append(r)   # +inf tie
    x = np.stack(rows)
    tok = F.argmax_batch(torch.from_numpy(x).cuda()).cpu().numpy()
    want = [O.sample(row, [], O.make_params(temperature=0.0, repetition_penalty=1.0))[0] for row in rows]
    assert list(tok) == want == [0, 0, 0, V - 3, 5000]
    # the same rows as greedy sampling rows (host route: the small-k kernel's greedy lists)
    p = W.make_params(len(rows), temperature=0.0, repetition_penalty=1.0)
    out = F.sample_batch(torch.from_numpy(x).cuda(), p, np.zeros(len(rows)))
    assert list(out["tok"].cpu().numpy()) == want


def _first_max(row):
    """ferro's greedy scan (sampler.cpp:19-23) restated with numpy: index 0 unless a later logit is strictly larger
    than every earlier one; NaN never compares larger."""
    if np.isnan(row[0]):
        return 0
    r = np.where(np.isnan(row), -np.inf, row)
    return int(np.argmax(r))            # np.argmax: the first index of the maximum


@pytest.mark.parametrize("V", [1, 3, 5, 4095, 4097, 65537])
def test_argmax_without_parameters_odd_vocab(V):
    """fs_argmax_batch without parameters (the small-k kernel's greedy path) on vocabularies that end inside a group
    of four, inside a segment or just past one; rows with NaN at 0, ties and -inf."""
    rng = np.random.default_rng(V)
    x = rng.standard_normal((6, V)).astype(np.float32)
    x[0, 0] = np.nan
    x[1, :] = -np.inf
    x[2, V - 1] = 50.0
    x[3, rng.integers(0, V, 3)] = 20.0
    if V > 2:
        x[4, 1] = np.nan
    want = [_first_max(r) for r in x]
    tok = F.argmax_batch(torch.from_numpy(x).cuda()).cpu().numpy()
    assert list(tok) == want


def test_greedy_batch_ties_across_segments():
    """A full-size greedy batch (B=64 x V=262144): maxima tied across segment boundaries, inside one lane's four
    logits, at the row's ends, +-0 and infinities; tokens must be the first maximum of each row."""
    rng = np.random.default_rng(21)
    B, V = 64, 262144
    x = rng.standard_normal((B, V)).astype(np.float32)
    seg = 16384
    for b in range(B):
        kind = b % 8
        if kind == 0:                                   # a tie in two segments: the lower one wins
            i, j = sorted(rng.choice(V, 2, replace=False))
            x[b, i] = x[b, j] = 7.5
        elif kind == 1:                                 # a tie at both sides of a segment boundary
            s = int(rng.integers(1, V // seg)) * seg
            x[b, s - 1] = x[b, s] = 9.0
        elif kind == 2:                                 # a tie inside one group of four
            g = int(rng.integers(0, V // 4)) * 4
            x[b, g + 1] = x[b, g + 3] = 8.0
        elif kind == 3:                                 # the maximum at the very end
            x[b, V - 1] = 10.0
        elif kind == 4:                                 # +0 and -0 as the maximum
            x[b] = -np.abs(x[b]) - 1.0
            x[b, 777] = -0.0
            x[b, 100000] = 0.0
        elif kind == 5:                                 # +inf twice
            x[b, 5000] = np.inf
            x[b, 200000] = np.inf
        elif kind == 6:                                 # NaN on the maximum's left and at index 0's right
            x[b, 1] = np.nan
            x[b, 3000] = 6.0
            x[b, 2999] = np.nan
        else:                                           # many equal maxima spread over every segment
            x[b, rng.choice(V, 300, replace=False)] = 5.0
    want = [_first_max(r) for r in x]
    p = W.make_params(B, temperature=0.0, repetition_penalty=1.0)
    out = F.sample_batch(torch.from_numpy(x).cuda(), p, np.zeros(B))
    assert list(out["tok"].cpu().numpy()) == want
    tok = F.argmax_batch(torch.from_numpy(x).cuda()).cpu().numpy()
    assert list(tok) == want


def test_sampled_rows_with_an_infinite_maximum():
    """A sampled row whose maximum is -inf or +inf: exp((l - mx) / T) is NaN for every logit (inf - inf), so ferro's
    sums are NaN, min-p and top-p cut nothing (their comparisons are false) and the walk ends on the last kept
    candidate (sampler.cpp:37-49). Every candidate path: small k, k <= 2048, large k and every token; with and
    without min-p / top-p."""
    V = 3 * 4096 + 77
    rng = np.random.default_rng(23)
    rows, B = [], 0
    for kind in ("neg", "pos"):
        for k in (5, 100, 3000, 0):
            for mp, tp in ((0.0, 1.0), (0.1, 0.9)):
                if kind == "neg":
                    r = np.full(V, -np.inf, np.float32)
                else:
                    r = (rng.standard_normal(V)).astype(np.float32)
                    r[[17, V - 9]] = np.inf
                rows.append((r, k, mp, tp))
    B = len(rows)
    p = W.make_params(B, temperature=0.9, top_k=0, repetition_penalty=1.0)
    for b, (_, k, mp, tp) in enumerate(rows):
        p["top_k"][b], p["min_p"][b], p["top_p"][b] = k, mp, tp
    w = _case([r for r, *_ in rows], p, [[]] * B, rng.random(B), "infinite_max")
    g = run_gpu(w, 0)
    o = run_oracle(w, 0)
    assert F.device_error() == 0
    bad = [(b, rows[b][1:], (int(g["tok"][b]), int(g["keep"][b])), (int(o["tok"][b]), int(o["keep"][b])))
           for b in range(B) if (g["tok"][b], g["keep"][b]) != (o["tok"][b], o["keep"][b])]
    assert not bad, bad


def test_penalize_in_place_matches_oracle():
    """fs_penalize_batch leaves each row exactly as ferro's sample() leaves its host row (sampler.cpp:11-18), with
    the frequency/presence extension, per-row windows and scopes (cfg5 rows: V=262144, H=1024)."""
    w = W.config5()
    B = 48
    x = torch.from_numpy(w.logits[:B].copy()).cuda()
    p = w.params[:B].copy()
    p["repeat_last_n"][:8] = [-1, 0, 1, 7, 100, 5000, -1, 64]
    p["penalty_from"][8:12] = [0, 3, 1000, 2000]
    off = w.hist_off[:B + 1]
    F.penalize_batch(x, p, hist=w.hist[:off[-1]], hist_off=off)
    got = x.cpu().numpy()
    changed = 0
    for b in range(B):
        want = O.penalize(w.logits[b], w.hist[off[b]:off[b + 1]], p[b])
        changed += int((want != w.logits[b]).sum())
        np.testing.assert_array_equal(got[b].view(np.uint32), want.view(np.uint32), err_msg=f"row {b}")
    assert changed > 1000
    assert F.device_error() == 0


def test_sampler_shim_writes_penalised_row_back():
    """Like ferro::Sampler::sample, the mirror leaves a host (numpy) or device row penalised in place."""
    rng = np.random.default_rng(3)
    V = 70000
    row = (rng.standard_normal(V) * 2).astype(np.float32)
    hist = list(rng.integers(0, V, 300)) + [5, 5, 5]
    sp = F.SamplerParams(temperature=0.7, top_k=40, repetition_penalty=1.3, frequency_penalty=0.25, seed=9)
    want = O.penalize(row, np.asarray(hist, np.int32), F.params_array(sp)[0])
    assert (want != row).sum() > 250
    host = row.copy()
    F.Sampler(sp).sample(host, V, hist)
    np.testing.assert_array_equal(host, want)
    dev = torch.from_numpy(row.copy()).cuda()
    F.Sampler(sp).sample(dev, V, hist)
    np.testing.assert_array_equal(dev.cpu().numpy(), want)
    kept = row.copy()
    F.Sampler(sp, write_back=False).sample(kept, V, hist)
    np.testing.assert_array_equal(kept, row)


def test_cpp_dropin_shim_replays_reference_streams(tmp_path):
    """include/ferro_sampler.hpp's ferro_amd::Sampler, driven from C++ like lm_cli.cpp:129-130, reproduces the
    reference's own seeded 40-call streams and leaves every host row penalised in place as ferro does."""
    import subprocess
    exe = os.path.join(os.path.dirname(__file__), "cpp", "shim_replay")
    if not os.path.exists(exe):
        pytest.fail("tests/cpp/shim_replay is not built (run __graft_entry__.build())")
    gold = np.load(os.path.join(os.path.dirname(__file__), "golden", "sampler_golden.npz"), allow_pickle=False)
    params = gold["stream_params"].view(F.PARAMS_DTYPE)
    X = gold["stream_x"]
    S, steps, V = X.shape
    inp, outp = tmp_path / "in.bin", tmp_path / "out.bin"
    with open(inp, "wb") as f:
        f.write(np.int64(S).tobytes())
        for s in range(S):
            h0 = gold["stream_h0"][s].astype(np.int32)
            f.write(params[s:s + 1].tobytes())
            f.write(np.array([gold["stream_seed"][s]], np.uint64).tobytes())
            f.write(np.array([V, steps, h0.size], np.int64).tobytes())
            f.write(h0.tobytes())
            f.write(np.ascontiguousarray(X[s], np.float32).tobytes())
    say(f"case cpp shim: S={S} steps={steps} V={V}")
    r = subprocess.run([exe, str(inp), str(outp)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    buf = np.fromfile(outp, np.uint8)
    pos = 0
    for s in range(S):
        tok = buf[pos:pos + 4 * steps].view(np.int32); pos += 4 * steps
        rows = buf[pos:pos + 4 * steps * V].view(np.float32).reshape(steps, V); pos += 4 * steps * V
        np.testing.assert_array_equal(tok, gold["stream_tok"][s])
        hist = list(gold["stream_h0"][s])
        for i in range(steps):
            want = O.penalize(X[s, i], np.asarray(hist, np.int32), params[s])
            np.testing.assert_array_equal(rows[i], want, err_msg=f"stream {s} step {i}")
            hist.append(int(tok[i]))
    assert pos == buf.size


def _host_draws(seed, n):
    r = F.Rng(int(seed))
    return r.next_u(n)


def test_device_draw_streams_match_libstdcxx():
    """fs_drng: per-stream std::mt19937_64 + generate_canonical on the device equals the host engine (libstdc++)
    bit for bit, across twists; greedy streams consume nothing."""
    seeds = np.array([1, 5489, 2**63 + 7, 123456789, 42, 7], dtype=np.uint64)
    S = len(seeds)
    p = W.make_params(S, temperature=0.8, top_k=40)
    p["temperature"][3] = 0.0                                  # greedy stream
    p["top_k"][5] = 1                                          # greedy through top_k == 1
    d = F.DeviceRng(seeds)
    got = np.stack([d.draw(p).cpu().numpy() for _ in range(700)])   # 700 calls: crosses two twists
    for s_ in range(S):
        if s_ in (3, 5):
            assert (got[:, s_] == 0).all()
        else:
            np.testing.assert_array_equal(got[:, s_], _host_draws(seeds[s_], 700))
    # the greedy streams start drawing exactly where they were once they sample
    p2 = p.copy()
    p2["temperature"][3] = 0.9
    np.testing.assert_array_equal(d.draw(p2).cpu().numpy()[3], _host_draws(seeds[3], 1)[0])
    assert d.error() == 0


def test_device_draw_rows_peek_and_skip():
    """A verify window: rows of a stream draw in row order; peek leaves the engine; skip consumes the accepted count
    (also across a twist)."""
    seeds = np.array([11, 22, 33], dtype=np.uint64)
    p = W.make_params(3, temperature=1.0, top_k=0)
    d = F.DeviceRng(seeds)
    one = np.array([0, 1, 2, 3], dtype=np.int64)
    for _ in range(300):                                       # bring the engines near the end of the state
        d.draw(p, row_off=one)
    m = 17
    row_off = np.arange(0, 3 * m + 1, m, dtype=np.int64)
    peek = d.draw(p, row_off=row_off, peek=True).cpu().numpy().reshape(3, m)
    for s_ in range(3):
        np.testing.assert_array_equal(peek[s_], _host_draws(seeds[s_], 300 + m)[300:])
    again = d.draw(p, row_off=row_off, peek=True).cpu().numpy().reshape(3, m)
    np.testing.assert_array_equal(again, peek)                 # peek consumed nothing
    acc = np.array([5, 17, 0], dtype=np.int32)
    d.skip(acc, p)
    nxt = d.draw(p).cpu().numpy()
    for s_ in range(3):
        assert nxt[s_] == _host_draws(seeds[s_], 300 + int(acc[s_]) + 1)[-1]
    assert d.error() == 0


def test_device_draws_replay_reference_streams():
    """ferro's own seeded 40-call streams (tests/golden): device draws + fs_sample_batch give the reference tokens."""
    gold = np.load(os.path.join(os.path.dirname(__file__), "golden", "sampler_golden.npz"), allow_pickle=False)
    params = gold["stream_params"].view(F.PARAMS_DTYPE)
    X = gold["stream_x"]
    S, steps, V = X.shape
    d = F.DeviceRng(gold["stream_seed"])
    hists = [list(gold["stream_h0"][s_]) for s_ in range(S)]
    for i in range(steps):
        u = d.draw(params)
        hist = np.concatenate([np.asarray(h, np.int32) for h in hists])
        off = np.concatenate([[0], np.cumsum([len(h) for h in hists])]).astype(np.int64)
        tok = F.sample_batch(torch.from_numpy(np.ascontiguousarray(X[:, i])).cuda(), params, u, hist=hist,
                             hist_off=off)["tok"].cpu().numpy()
        np.testing.assert_array_equal(tok, gold["stream_tok"][:, i], err_msg=f"step {i}")
        for s_ in range(S):
            hists[s_].append(int(tok[s_]))


@pytest.mark.parametrize("seed", [30, 31, 32])
def test_softcap_fused_read(seed):
    """Gemma 4's final-logit softcap (cap 30) fused into the read, on every path: top-k, greedy, large k, penalties,
    and a row tail, on unclipped logits (saturating ones and +-inf included), to the same exact bar as uncapped rows:
    the device's tanhf is the host C library's, restated (model_gemma4_gpu.cpp:282-283 caps the host row with it)."""
    rng = np.random.default_rng(seed)
    V = 262144 + 77
    B = 8
    x = (W.mixture_logits(rng, B, V) * np.float32(rng.uniform(1.0, 40.0))).astype(np.float32)
    x[0, rng.integers(0, V, 50)] = np.float32(1e4)                 # saturated: every one of them caps to 30
    x[5, rng.integers(0, V, 5)] = np.float32(np.inf)
    x[6, rng.integers(0, V, 5)] = np.float32(-np.inf)
    p = W.make_params(B, temperature=0.8, top_k=64, top_p=0.95, repetition_penalty=1.05)
    p["softcap"] = 30.0
    p["temperature"][1] = 0.0
    p["top_k"][2] = 0
    p["top_k"][7] = 1500
    p["frequency_penalty"][3], p["presence_penalty"][3] = 0.4, 0.2
    hists = [rng.integers(0, V, 300) for _ in range(B)]
    g, o, nb = check(_case(list(x), p, hists, rng.random(B), f"softcap{seed}"), kcap=64)
    assert nb <= 1
    t2 = F.argmax_batch(torch.from_numpy(x).cuda(), params=p, hist=np.concatenate(hists).astype(np.int32),
                        hist_off=np.concatenate([[0], np.cumsum([len(h) for h in hists])]).astype(np.int64))
    np.testing.assert_array_equal(t2.cpu().numpy(), [O.sample(x[b], hists[b], O.make_params(
        temperature=0.0, repetition_penalty=1.05, softcap=30.0, frequency_penalty=float(p["frequency_penalty"][b]),
        presence_penalty=float(p["presence_penalty"][b])))[0] for b in range(B)])


def test_softcap_matches_host_libm_on_every_float():
    """fs_softcap_batch (the sampler's fused cap) against the model's host loop, cap * tanhf(x / cap) with the C
    library's tanhf (model_gemma4_gpu.cpp:282-283): bit-identical on all 2^32 float inputs at cap 1 (tanhf itself),
    and on 2^26 random bit patterns at caps 30 and 0.375. NaN inputs give NaN (payloads are not compared)."""
    from ferro_amd._lib import lib
    L = lib()
    chunk = 1 << 27
    dev = torch.device("cuda", 0)
    d_in = torch.empty(chunk, dtype=torch.int32, device=dev)
    d_out = torch.empty(chunk, dtype=torch.float32, device=dev)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    base = np.arange(chunk, dtype=np.uint32)
    nth = min(16, os.cpu_count() or 1)
    bad = 0

    def run(bits, cap):
        n = bits.size
        d_in[:n].copy_(torch.from_numpy(bits.view(np.int32)))
        rc = L.fs_softcap_batch(ctypes.c_void_p(d_in.data_ptr()), ctypes.c_void_p(d_out.data_ptr()), n,
                                ctypes.c_float(cap), st)
        assert rc == 0
        ref = torch.from_numpy(O.softcap(bits.view(np.float32), cap, nth).view(np.int32)).to(dev)
        got = d_out[:n].view(torch.int32)
        differ = (got != ref) & ~(torch.isnan(d_out[:n]) & torch.isnan(ref.view(torch.float32)))
        return int(differ.sum().item())

    for c in range((1 << 32) // chunk):
        bad += run(base + np.uint32(c * chunk), 1.0)
    say(f"softcap cap 1: {bad} of 2^32 inputs differ from the host C library")
    assert bad == 0
    rng = np.random.default_rng(5)
    for cap in (30.0, 0.375):
        bits = rng.integers(0, 1 << 32, 1 << 26, dtype=np.uint64).astype(np.uint32)
        n = run(bits, cap)
        say(f"softcap cap {cap}: {n} of 2^26 random inputs differ")
        assert n == 0


def test_lookup_draft_matches_oracle():
    """fs_lookup_draft (server.cpp:552-564) on histories with copied runs, eos tokens and per-stream kmax / min_n,
    including long histories."""
    rng = np.random.default_rng(52)
    E = 7
    hists = []
    for s_ in range(40):
        L = int(rng.integers(0, 60)) if s_ < 30 else int(rng.integers(2000, 6000))
        base = list(rng.integers(0, 12 if s_ % 3 == 0 else 400, L))
        for _ in range(int(rng.integers(0, 4))):          # copy runs so that tails recur
            if len(base) > 8:
                a_ = int(rng.integers(0, len(base) - 6))
                base += base[a_:a_ + int(rng.integers(2, 7))]
        hists.append(np.asarray(base, np.int32))
    off = np.concatenate([[0], np.cumsum([len(h) for h in hists])]).astype(np.int64)
    hist = np.concatenate(hists).astype(np.int32)
    kmax = rng.integers(0, 17, len(hists)).astype(np.int32)
    min_n = rng.integers(2, 4, len(hists)).astype(np.int32)
    draft, nd = F.lookup_draft(hist, off, kmax, min_n=min_n, eos_id=E, draft_ld=16)
    draft, nd = draft.cpu().numpy(), nd.cpu().numpy()
    hits = 0
    for s_, h in enumerate(hists):
        want = O.lookup_draft(h, int(kmax[s_]), eos=E, min_n=int(min_n[s_]))
        assert nd[s_] == len(want), s_
        np.testing.assert_array_equal(draft[s_, :nd[s_]], want)
        hits += len(want) > 0
    assert hits >= 10


def test_device_decode_loop_with_history_append():
    """Decode steps entirely on the device: fs_drng_draw, fs_sample_batch over the device histories, then
    fs_hist_append (gen_token's push_back, server.cpp:342) feeding the next step. Tokens and the final histories
    equal the oracle's loop (sample each stream, then append)."""
    rng = np.random.default_rng(505)
    S, V, steps = 6, 5000, 10
    p = W.make_params(S, temperature=0.8, top_k=40, top_p=0.9, repetition_penalty=1.4)
    p["temperature"][1] = 0.0
    p["top_k"][2] = 0
    p["repeat_last_n"][3] = 6
    p["frequency_penalty"][4], p["presence_penalty"][4] = 0.5, 0.3
    seeds = [101, 202, 303, 404, 505, 606]
    hist0 = [list(rng.integers(0, V, int(rng.integers(0, 40)))) for _ in range(S)]
    hist0[5] = []
    rows = [(rng.standard_normal((S, V)) * 2.5).astype(np.float32) for _ in range(steps)]
    want, want_hist, want_off = oracle_decode_loop(rows, p, seeds, hist0)
    d = F.DeviceRng(np.array(seeds, np.uint64))
    hist = torch.from_numpy(np.concatenate([np.asarray(h, np.int32) for h in hist0])).cuda()
    off = torch.from_numpy(np.concatenate([[0], np.cumsum([len(h) for h in hist0])]).astype(np.int64)).cuda()
    got = []
    for k in range(steps):
        say(f"decode step {k}")
        u = d.draw(p)
        tok = F.sample_batch(torch.from_numpy(rows[k]).cuda(), p, u, hist=hist, hist_off=off)["tok"]
        got.append(tok)
        hist, off = F.hist_append(hist, off, tok)
    np.testing.assert_array_equal(torch.stack(got).cpu().numpy(), want)
    o = off.cpu().numpy()
    np.testing.assert_array_equal(o, want_off)
    np.testing.assert_array_equal(hist[:o[-1]].cpu().numpy(), want_hist)
    assert F.device_error() == 0


def test_history_append_verify_window_and_limits():
    """fs_hist_append fed fs_verify's outputs as they are (tok, row_off, accepted): each stream gains its accepted
    prefix. Counts outside [0, rows] are clamped and flagged; an output past out_cap is not written and flagged."""
    rng = np.random.default_rng(9)
    Sn, M, V = 4, 5, 3000
    x = (rng.standard_normal((Sn * M, V)) * 3).astype(np.float32)
    rows = rng.integers(0, V, Sn * M).astype(np.int32)
    row_off = np.arange(0, Sn * M + 1, M, dtype=np.int64)
    x[np.arange(Sn * M - 1), rows[1:]] += 30.0
    x[2 * M + 1, rows[2 * M + 2]] -= 60.0                            # stream 2 rejects its second draft
    p = W.make_params(Sn, temperature=0.0)
    hists = [rng.integers(0, V, int(n)).astype(np.int32) for n in (0, 7, 30, 3)]
    h = np.concatenate(hists)
    ho = np.concatenate([[0], np.cumsum([len(a) for a in hists])]).astype(np.int64)
    tok, acc = F.verify(torch.from_numpy(x).cuda(), rows, row_off, p, hist=h, hist_off=ho)
    out, oo = F.hist_append(torch.from_numpy(h).cuda(), torch.from_numpy(ho).cuda(), tok, row_off=row_off, count=acc)
    wh, wo = O.hist_append(h, ho, tok.cpu().numpy(), row_off=row_off, count=acc.cpu().numpy())
    np.testing.assert_array_equal(oo.cpu().numpy(), wo)
    np.testing.assert_array_equal(out[:wo[-1]].cpu().numpy(), wh)
    assert acc.cpu().numpy()[2] == 2 and F.device_error() == 0
    # counts out of range: clamped, flagged
    bad = np.array([-1, 9, 2, 5], np.int32)
    out, oo = F.hist_append(torch.from_numpy(h).cuda(), torch.from_numpy(ho).cuda(), tok, row_off=row_off, count=bad)
    wh, wo = O.hist_append(h, ho, tok.cpu().numpy(), row_off=row_off, count=bad)
    np.testing.assert_array_equal(oo.cpu().numpy(), wo)
    np.testing.assert_array_equal(out[:wo[-1]].cpu().numpy(), wh)
    assert F.device_error() == 4
    # capacity: the first out_cap ids are written, the offsets are complete, the overflow is flagged
    cap = int(wo[-1]) - 3
    out, oo = F.hist_append(torch.from_numpy(h).cuda(), torch.from_numpy(ho).cuda(), tok, row_off=row_off, count=bad,
                            out_cap=cap)
    np.testing.assert_array_equal(oo.cpu().numpy(), wo)
    np.testing.assert_array_equal(out[:cap].cpu().numpy(), wh[:cap])
    assert F.device_error() == 4


def test_history_append_many_streams():
    """fs_hist_append over 1500 streams (the offset scan runs in chunks of 512 with a carry): ragged histories,
    empty ones, rows of 0-6 per stream and random accepted counts, against the oracle; and no streams at all."""
    rng = np.random.default_rng(77)
    S = 1500
    lens = rng.integers(0, 40, S)
    lens[::7] = 0
    h = rng.integers(0, 100000, int(lens.sum())).astype(np.int32)
    ho = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    nrows = rng.integers(0, 7, S)
    row_off = np.concatenate([[0], np.cumsum(nrows)]).astype(np.int64)
    tok = rng.integers(0, 100000, int(row_off[-1])).astype(np.int32)
    cnt = np.array([rng.integers(0, r + 1) for r in nrows], np.int32)
    out, oo = F.hist_append(torch.from_numpy(h).cuda(), torch.from_numpy(ho).cuda(), torch.from_numpy(tok).cuda(),
                            row_off=row_off, count=cnt)
    wh, wo = O.hist_append(h, ho, tok, row_off=row_off, count=cnt)
    np.testing.assert_array_equal(oo.cpu().numpy(), wo)
    np.testing.assert_array_equal(out[:wo[-1]].cpu().numpy(), wh)
    # one token per stream (decode), on a sub-view whose offsets do not start at 0
    out, oo = F.hist_append(torch.from_numpy(h).cuda(), torch.from_numpy(ho[5:]).cuda(),
                            torch.from_numpy(tok[:S - 5]).cuda())
    wh, wo = O.hist_append(h, ho[5:], tok[:S - 5])
    np.testing.assert_array_equal(oo.cpu().numpy(), wo)
    np.testing.assert_array_equal(out[:wo[-1]].cpu().numpy(), wh)
    out, oo = F.hist_append(torch.zeros(0, dtype=torch.int32).cuda(), torch.zeros(1, dtype=torch.int64).cuda(),
                            torch.zeros(0, dtype=torch.int32).cuda())
    assert oo.cpu().numpy().tolist() == [0]
    out, oo = F.hist_append(torch.zeros(0, dtype=torch.int32).cuda(), torch.zeros(4, dtype=torch.int64).cuda(),
                            torch.tensor([5, 6, 7], dtype=torch.int32).cuda())      # streams, all histories empty
    assert oo.cpu().numpy().tolist() == [0, 1, 2, 3] and out[:3].cpu().numpy().tolist() == [5, 6, 7]
    assert F.device_error() == 0


def test_strided_inputs_are_packed_before_the_abi():
    """Wrapper inputs given as strided views (a column of a token matrix, every other draw) are copied to packed
    arrays, never read as if packed: results equal those of the packed inputs."""
    rng = np.random.default_rng(91)
    S = 9
    lens = rng.integers(1, 12, S)
    h = rng.integers(0, 5000, int(lens.sum())).astype(np.int32)
    ho = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    toks = torch.from_numpy(rng.integers(0, 5000, (S, 3)).astype(np.int32)).cuda()
    col = toks[:, 1]                                        # stride 3
    assert not col.is_contiguous()
    out, oo = F.hist_append(torch.from_numpy(h).cuda(), torch.from_numpy(ho).cuda(), col)
    wh, wo = O.hist_append(h, ho, toks[:, 1].cpu().numpy().copy())
    np.testing.assert_array_equal(oo.cpu().numpy(), wo)
    np.testing.assert_array_equal(out[:wo[-1]].cpu().numpy(), wh)
    w = W.config3(B=4, V=8192)
    u2 = torch.from_numpy(np.stack([w.u, np.full(w.B, 0.5)], axis=1).reshape(-1)).cuda()[::2]   # stride 2
    assert not u2.is_contiguous()
    a = F.sample_batch(torch.from_numpy(w.logits).cuda(), w.params, u2, hist=w.hist, hist_off=w.hist_off, kcap=8)
    b = F.sample_batch(torch.from_numpy(w.logits).cuda(), w.params, w.u, hist=w.hist, hist_off=w.hist_off, kcap=8)
    np.testing.assert_array_equal(a["tok"].cpu().numpy(), b["tok"].cpu().numpy())
    with pytest.raises(F.SamplerError):
        F.sampler._ptr(col)


def test_sampled_rows_with_nan_follow_the_policy():
    """Sampled (non-greedy) rows holding NaN logits, where ferro's order is unspecified, against the oracle's
    stated policy (NaN ranks below every number and is never a candidate): scattered NaNs with k below the count of
    numbers on the fused path, top_k = 0 over the numbers, rows with fewer numbers than k, a row of NaNs only (token
    0, nothing kept), through every path (one-tile rows, multi-tile rows, penalties)."""
    rng = np.random.default_rng(404)
    for V, B in ((3000, 12), (65536, 10)):
        x = (rng.standard_normal((B, V)) * 2).astype(np.float32)
        x[rng.random((B, V)) < 0.02] = np.nan
        p = W.make_params(B, temperature=0.8, top_k=40, top_p=0.95, repetition_penalty=1.1)
        p["top_k"][1] = 500
        p["top_k"][2] = 0
        p["top_p"][2] = 0.9
        p["top_k"][3] = 2048
        few = rng.choice(V, 30, replace=False)            # 30 numbers, the rest NaN; k = 40 > 30
        x[4] = np.nan
        x[4, few] = rng.standard_normal(30).astype(np.float32)
        x[5] = np.nan                                     # no numbers at all
        p["min_p"][6] = 0.05
        hists = [rng.integers(0, V, 50).astype(np.int32) for _ in range(B)]
        w = _case(list(x), p, hists, rng.random(B), f"nan_rows_V{V}")
        g, o, nb = check(w, kcap=64)
        assert g["tok"][5] == 0 and g["keep"][5] == 0
        assert nb <= 1


def test_golden_rows_through_gpu():
    """The reference's own 160 single-call vectors (tokens of ferro::Sampler, tests/golden: V 1..3000, ties, signed
    zeros, every parameter regime) through fs_sample_batch, rows grouped by V: tokens equal the reference's except
    where the draw lies within 1e-6 of a cumulative boundary (counted)."""
    gold = np.load(os.path.join(os.path.dirname(__file__), "golden", "sampler_golden.npz"), allow_pickle=False)
    params = gold["rows_params"].view(O.PARAMS_DTYPE)
    xo, ho = gold["rows_x_off"], gold["rows_h_off"]
    n = len(gold["rows_tok"])
    Vs = np.diff(xo)
    near = differ = 0
    for V in sorted(set(Vs.tolist())):
        idx = np.nonzero(Vs == V)[0]
        rows = [gold["rows_x"][xo[i]:xo[i + 1]] for i in idx]
        hists = [gold["rows_h"][ho[i]:ho[i + 1]] for i in idx]
        u = np.array([W.first_u(int(gold["rows_seed"][i])) for i in idx])
        w = _case(rows, params[idx].copy(), hists, u, f"golden_V{V}")
        g, o, nb = check(w, kcap=min(int(V), 2048))
        near += int(nb)
        diff = g["tok"] != gold["rows_tok"][idx]
        differ += int(diff.sum())
        assert int(diff.sum()) <= nb.diverged, f"V={V}: tokens differ from the reference away from a boundary"
    say(f"golden rows: {n}, near a boundary {near}, tokens differing from the reference {differ}")
    assert differ <= 2
