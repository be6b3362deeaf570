"""Pins the CPU oracle (oracle/sampler_oracle.c) before it is trusted as the GPU checker.

- reference known-answer test: tests/test_kernels.cpp:348-358 (penalty window / scope, five cases);
- golden vectors written by the compiled reference sampler (tests/golden/sampler_golden.npz): 160 single calls,
  two 40-call streams (draw-stream consumption), the full config-1 row under 32 seeds;
- brute force: a full numpy lexsort gives the candidate order for tiny rows (membership, order, ties, +-0);
- closed forms: top-p keeps the crossing element, min-p, greedy, u at the CDF edges, the extension's arithmetic;
- the verification rule (server.cpp:627-637) on hand-built windows;
- the live reference (if oracle/_ref is built) on fresh random rows.
"""
import math
import os

import numpy as np
import pytest

from oracle import oracle as O
from ferro_amd import workloads as W
from parity_util import bf16_valued, oracle_decode_loop

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "sampler_golden.npz")


def test_known_answer_penalty_window_scope():
    # tests/test_kernels.cpp:348-358: logits {0,9,10,9.5,6,0}, history {1,2,3}, penalty 2, greedy
    row = np.array([0, 9, 10, 9.5, 6, 0], np.float32)
    want = {(-1, 0): 4, (-1, 2): 2, (2, 0): 1, (0, 0): 2, (2, 2): 2}
    for (last_n, frm), tok in want.items():
        p = O.make_params(temperature=0.0, repetition_penalty=2.0, repeat_last_n=last_n, penalty_from=frm)
        assert O.sample(row, [1, 2, 3], p)[0] == tok, (last_n, frm)


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN, allow_pickle=False)


def test_golden_rows(golden):
    g = golden
    params = g["rows_params"].view(O.PARAMS_DTYPE)
    n = len(g["rows_tok"])
    assert n == 160
    bad = []
    for i in range(n):
        x = g["rows_x"][g["rows_x_off"][i]:g["rows_x_off"][i + 1]]
        h = g["rows_h"][g["rows_h_off"][i]:g["rows_h_off"][i + 1]]
        u = W.first_u(int(g["rows_seed"][i]))
        tok = O.sample(x, h, params[i], u)[0]
        if tok != g["rows_tok"][i]:
            bad.append(i)
    assert not bad


def test_golden_streams(golden):
    g = golden
    params = g["stream_params"].view(O.PARAMS_DTYPE)
    for s in range(len(params)):
        p = params[s]
        mt = W.MT19937_64(int(g["stream_seed"][s]))
        greedy = p["temperature"] <= 0 or p["top_k"] == 1
        hist = list(g["stream_h0"][s])
        for i, row in enumerate(g["stream_x"][s]):
            u = 0.0 if greedy else W.canonical(mt.next())     # one draw per non-greedy call, none for greedy
            tok = O.sample(row, np.array(hist, np.int32), p, u)[0]
            assert tok == g["stream_tok"][s][i], (s, i)
            hist.append(tok)


def test_golden_cfg1(golden):
    w = W.config1()
    for s, t in zip(golden["cfg1_seed"], golden["cfg1_tok"]):
        assert O.sample(w.logits[0], w.hist, w.params[0], W.first_u(int(s)))[0] == t


def test_mt64_and_canonical():
    # std::mt19937_64 with the default seed 5489: the standard fixes the 10000th output (C++11 [rand.predef])
    mt = W.MT19937_64(5489)
    for _ in range(9999):
        mt.next()
    assert mt.next() == 9981545732273789042
    # the C restatement agrees with the Python one
    a, b = O.MT64(12345), W.MT19937_64(12345)
    for _ in range(700):
        assert a.next() == b.next()
    assert W.canonical(0) == 0.0
    assert W.canonical(2**64 - 1) == float(np.nextafter(1.0, 0.0))
    assert O.canonical(2**64 - 1) == W.canonical(2**64 - 1)
    assert O.canonical(2**63) == 0.5


def brute_order(x):
    """Candidate order by brute force: value desc, id asc; -0 == +0 (add 0.0 folds -0 onto +0)."""
    v = x.astype(np.float64) + 0.0
    return np.lexsort((np.arange(len(x)), -v))


@pytest.mark.parametrize("seed", range(40))
def test_topk_membership_and_order_brute_force(seed):
    rng = np.random.default_rng(seed)
    V = int(rng.integers(1, 200))
    x = (np.round(rng.standard_normal(V) * 3) / 2).astype(np.float32)     # ties
    x[rng.random(V) < 0.2] = -0.0
    k = int(rng.integers(1, V + 3))
    p = O.make_params(temperature=1.0, top_k=k if k != 1 else 2, repetition_penalty=1.0)
    tok, ids, probs, keep, ncand = O.sample(x, [], p, 0.5, kcap=V)
    kk = p["top_k"][0] if 0 < p["top_k"][0] < V else V
    assert ncand == kk
    np.testing.assert_array_equal(ids, brute_order(x)[:kk])


def test_softmax_topp_minp_closed_form():
    # 4 candidates with logits log(4), log(3), log(2), log(1) at T=1 -> p = .4 .3 .2 .1
    x = np.log(np.array([1, 4, 2, 3], np.float64)).astype(np.float32)
    p = O.make_params(temperature=1.0, top_k=0, repetition_penalty=1.0)
    tok, ids, probs, keep, ncand = O.sample(x, [], p, 0.0, kcap=4)
    np.testing.assert_array_equal(ids, [1, 3, 2, 0])
    np.testing.assert_allclose(probs, [0.4, 0.3, 0.2, 0.1], rtol=1e-6)
    assert keep == 4 and tok == 1
    # top-p keeps the element whose cumulative sum crosses: .4 < .5 <= .7 -> keep 2
    p["top_p"] = 0.5
    assert O.sample(x, [], p, 0.0, kcap=4)[3] == 2
    p["top_p"] = 0.4                  # .4 >= .4 (within float rounding of the stored top_p) -> keep 1 or 2
    assert O.sample(x, [], p, 0.0, kcap=4)[3] in (1, 2)
    p["top_p"] = 1.0
    p["min_p"] = 0.6                  # thr = .24: keeps .4 .3
    assert O.sample(x, [], p, 0.0, kcap=4)[3] == 2
    p["min_p"] = 2.0                  # thr above pr[0]: keep shrinks to 1
    assert O.sample(x, [], p, 0.999, kcap=4)[3] == 1
    # draw: u*tot against the cumulative sums .4 .7 .9 1.0
    p["min_p"] = 0.0
    for u, want in [(0.0, 1), (0.39, 1), (0.41, 3), (0.69, 3), (0.71, 2), (0.89, 2), (0.91, 0), (0.999999, 0)]:
        assert O.sample(x, [], p, u)[0] == want, u


def test_greedy_ties_nan_and_topk1():
    p = O.make_params(temperature=0.0, repetition_penalty=1.0)
    assert O.sample(np.array([1, 3, 3, 2], np.float32), [], p)[0] == 1
    assert O.sample(np.array([-0.0, 0.0], np.float32), [], p)[0] == 0
    assert O.sample(np.array([np.nan, 5, 6], np.float32), [], p)[0] == 0      # nothing compares > NaN at 0
    assert O.sample(np.array([1, np.nan, 6], np.float32), [], p)[0] == 2
    p = O.make_params(temperature=1.0, top_k=1, repetition_penalty=1.0)        # top_k 1 is greedy
    assert O.sample(np.array([1, 3, 3, 2], np.float32), [], p, 0.99)[0] == 1


def test_frequency_presence_extension():
    row = np.array([2.0, -1.0, 0.5, 3.0], np.float32)
    h = [0, 0, 0, 1, 3, 3]
    # freq = pres = 0 must leave ferro's repetition step alone, bit for bit
    p = O.make_params(repetition_penalty=1.3)
    base = O.penalize(row, h, p)
    p2 = O.make_params(repetition_penalty=1.3, frequency_penalty=0.0, presence_penalty=0.0)
    np.testing.assert_array_equal(O.penalize(row, h, p2).view(np.uint32), base.view(np.uint32))
    # llama.cpp convention after the repetition step: l -= cnt*freq + pres (float32 ops)
    p3 = O.make_params(repetition_penalty=1.0, frequency_penalty=0.5, presence_penalty=0.25)
    out = O.penalize(row, h, p3)
    f32 = np.float32
    np.testing.assert_array_equal(out, np.array([f32(2.0) - (f32(3) * f32(0.5) + f32(0.25)),
                                                 f32(-1.0) - (f32(1) * f32(0.5) + f32(0.25)),
                                                 f32(0.5),
                                                 f32(3.0) - (f32(2) * f32(0.5) + f32(0.25))], np.float32))


def test_combined_penalties_hand_computed():
    """Repetition, frequency and presence penalties together, over a window that repeat_last_n and penalty_from cut
    through repeated ids (sampler.cpp:11-18 plus the llama.cpp-convention extension after it). Every value is exact
    in fp32 (rep 2, freq 0.5, pres 0.25), so the expected rows are written out by hand."""
    row = np.array([4.0, -1.5, 3.0, 0.5, -2.0, 6.0, 1.0, -0.25, 2.5, 8.0], np.float32)
    h = [5, 5, 2, 9, 5, 1, 3, 9, 9, 7, 2, 12, -1, 5]        # 12 and -1 lie outside [0, V): never penalised
    # window h[14-9 .. 14) = [1, 3, 9, 9, 7, 2, 12, -1, 5]: the 5s at positions 0, 1, 4 fall before it
    #   id 1: -1.5 * 2 = -3.0, then - (1*0.5 + 0.25) = -3.75        id 3: 0.5 / 2 = 0.25, - 0.75 = -0.5
    #   id 9:  8.0 / 2 =  4.0, then - (2*0.5 + 0.25) =  2.75        id 7: -0.25 * 2 = -0.5, - 0.75 = -1.25
    #   id 2:  3.0 / 2 =  1.5, - 0.75 = 0.75                        id 5: 6.0 / 2 = 3.0, - 0.75 = 2.25
    p = O.make_params(repetition_penalty=2.0, frequency_penalty=0.5, presence_penalty=0.25, repeat_last_n=9,
                      penalty_from=2)
    want = np.array([4.0, -3.75, 0.75, -0.5, -2.0, 2.25, 1.0, -1.25, 2.5, 2.75], np.float32)
    np.testing.assert_array_equal(O.penalize(row, h, p), want)
    # penalty_from 8 moves the window start past repeat_last_n's: h[8 .. 14) = [9, 7, 2, 12, -1, 5]
    p = O.make_params(repetition_penalty=2.0, frequency_penalty=0.5, presence_penalty=0.25, repeat_last_n=9,
                      penalty_from=8)
    want2 = np.array([4.0, -1.5, 0.75, 0.5, -2.0, 2.25, 1.0, -1.25, 2.5, 3.25], np.float32)
    np.testing.assert_array_equal(O.penalize(row, h, p), want2)
    # whole history (repeat_last_n -1, penalty_from 0): ids 5 x4, 9 x3, 2 x2, 1, 3, 7 x1
    #   id 5: 3.0 - (4*0.5 + 0.25) = 0.75     id 9: 4.0 - 1.75 = 2.25     id 2: 1.5 - 1.25 = 0.25
    p = O.make_params(repetition_penalty=2.0, frequency_penalty=0.5, presence_penalty=0.25, repeat_last_n=-1)
    want3 = np.array([4.0, -3.75, 0.25, -0.5, -2.0, 0.75, 1.0, -1.25, 2.5, 2.25], np.float32)
    np.testing.assert_array_equal(O.penalize(row, h, p), want3)
    # the greedy token of the penalised row
    p = O.make_params(temperature=0.0, repetition_penalty=2.0, frequency_penalty=0.5, presence_penalty=0.25,
                      repeat_last_n=9, penalty_from=2)
    assert O.sample(row, h, p)[0] == 0


def test_verify_rule_hand_built():
    V = 8
    # stream 0: rows predict 5, 6, 7; drafts fed are [x, 5, 6] -> both drafts accepted -> acc 3
    # stream 1: rows predict 1, 2; drafts fed [x, 3] -> first draft rejected -> acc 1
    # stream 2: rows predict 4 (= eos), 0; drafts fed [x, 4] -> eos ends the window at row 0 -> acc 1
    preds = [5, 6, 7, 1, 2, 4, 0]
    logits = np.zeros((7, V), np.float32)
    logits[np.arange(7), preds] = 10.0
    rows = np.array([0, 5, 6, 0, 3, 0, 4], np.int32)
    row_off = np.array([0, 3, 5, 7], np.int64)
    p = O.make_params(3, temperature=0.0, repetition_penalty=1.0)
    tok, acc = O.verify(logits, rows, row_off, np.zeros(0, np.int32), np.zeros(4, np.int64), p, np.zeros(7),
                        eos_id=4)
    assert list(tok) == preds
    assert list(acc) == [3, 1, 1]


def test_verify_row_history_includes_drafts():
    # repetition penalty on the drafts: row 1 sees history [base..., draft1]; its argmax moves off draft1
    V = 4
    logits = np.array([[0, 0, 5, 0], [0, 0, 5, 4.9]], np.float32)
    rows = np.array([1, 2], np.int32)
    p = O.make_params(1, temperature=0.0, repetition_penalty=2.0)
    tok, acc = O.verify(logits, rows, np.array([0, 2]), np.array([1], np.int32), np.array([0, 1]), p, np.zeros(2))
    assert list(tok) == [2, 3] and list(acc) == [2]


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (needs /root/reference)")
def test_live_reference_random():
    rng = np.random.default_rng(99)
    for s in range(1, 200):
        V = int(rng.integers(1, 5000))
        x = (rng.standard_normal(V) * rng.uniform(0.5, 5)).astype(np.float32)
        if s % 3 == 0:
            x = (np.round(x) / 2).astype(np.float32)
        h = rng.integers(0, V, int(rng.integers(0, 300))).astype(np.int32)
        p = O.make_params(temperature=float(rng.choice([0, 0.2, 0.8, 1.5])), top_k=int(rng.integers(0, 300)),
                          top_p=float(rng.uniform(0.3, 1.0)), min_p=float(rng.choice([0, 0.1])),
                          repetition_penalty=float(rng.uniform(0.8, 1.6)),
                          repeat_last_n=int(rng.choice([-1, 0, 5, 64])), penalty_from=int(rng.choice([0, 3])))
        assert O.sample(x, h, p, W.first_u(s))[0] == O.ref_sample_stream(p, s, [x], [h])[0], s


def test_softcap_closed_form():
    """softcap (the model's final-logit transform, model_gemma4_gpu.cpp:282-283): sampling raw logits with softcap
    set equals sampling the capped row (numpy's float32 tanh, an independent implementation) with softcap off."""
    rng = np.random.default_rng(17)
    row = (rng.standard_normal(5000) * 12).astype(np.float32)
    cap = np.float32(30.0)
    capped = (cap * np.tanh(row / cap)).astype(np.float32)
    for kw in [dict(temperature=0.8, top_k=50, top_p=0.9), dict(temperature=0.0), dict(temperature=1.2, top_k=0)]:
        p0 = O.make_params(repetition_penalty=1.2, **kw)
        p1 = O.make_params(repetition_penalty=1.2, softcap=30.0, **kw)
        h = rng.integers(0, 5000, 40).astype(np.int32)
        t0, ids0, pr0, k0, n0 = O.sample(capped, h, p0, 0.37, kcap=64)
        t1, ids1, pr1, k1, n1 = O.sample(row, h, p1, 0.37, kcap=64)
        assert t0 == t1 and k0 == k1 and n0 == n1
        np.testing.assert_array_equal(ids0, ids1)
        np.testing.assert_allclose(pr0, pr1, rtol=1e-5)          # tanh implementations differ by ulps
    assert (O.penalize(row, h, p1) == O.penalize(row, h, p0)).all()   # the penalty pass alone ignores softcap


def test_lookup_draft_known_answers():
    """server.cpp:552-564 on hand-built histories: the most recent match of the last n tokens (n = 4, 3, 2) wins;
    a match followed by eos is passed over; the draft stops before eos and at kmax."""
    h = [1, 2, 3, 4, 5, 1, 2, 3]                      # no 4-token repeat; the 3-token tail [1,2,3] occurs at 0
    assert list(O.lookup_draft(h, 3)) == [4, 5, 1]
    assert list(O.lookup_draft(h, 10)) == [4, 5, 1, 2, 3]
    E = 99
    h = [7, 8, 9, 2, 5, 7, 8, 9, E, 6, 7, 8, 9]       # most recent [7,8,9] is followed by eos: skipped
    assert list(O.lookup_draft(h, 8, eos=E)) == [2, 5, 7, 8, 9]
    assert list(O.lookup_draft(h, 8)) == [E, 6, 7, 8, 9]  # no eos: the most recent match wins
    h = [4, 4, 4, 4, 4]                               # self-overlapping repeat: n = 4 matches at p = 0
    assert list(O.lookup_draft(h, 5)) == [4]
    assert list(O.lookup_draft([1, 2, 3, 1, 2], 4, min_n=3)) == []      # only a 2-token repeat
    assert list(O.lookup_draft([1, 2, 3, 1, 2], 4, min_n=2)) == [3, 1, 2]
    assert list(O.lookup_draft([5], 4)) == [] and list(O.lookup_draft([], 4)) == []
    assert list(O.lookup_draft([5, 5], 4)) == []      # n = min(4, L-1) = 1 < min_n
    assert list(O.lookup_draft([1, 2, 1, 2], 0)) == []  # kmax = 0: nothing to draft


def test_hist_append_known_answers():
    """gen_token's push_back (server.cpp:342) on CSR histories: one token per stream (the decode loop), the accepted
    prefix of a verify window (server.cpp:627-637), empty histories, counts clamped to the stream's rows."""
    out, off = O.hist_append([1, 2, 3, 9], [0, 3, 3, 4], [7, 8, 6])
    assert list(off) == [0, 4, 5, 7] and list(out) == [1, 2, 3, 7, 8, 9, 6]
    # verify window: stream rows [0, 3) and [3, 5), accepted 2 and 1 -> tokens 10, 11 and 13
    out, off = O.hist_append([5, 6], [0, 1, 2], [10, 11, 12, 13, 14], row_off=[0, 3, 5], count=[2, 1])
    assert list(off) == [0, 3, 5] and list(out) == [5, 10, 11, 6, 13]
    # rebased input offsets, count 0, a count past the stream's rows (clamped)
    out, off = O.hist_append([0, 0, 4, 4], [2, 3, 4], [1, 2, 3], row_off=[0, 1, 3], count=[0, 9])
    assert list(off) == [0, 1, 4] and list(out) == [4, 4, 2, 3]


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (needs /root/reference)")
def test_decode_loop_with_append_matches_reference():
    """The oracle's decode loop (sample, then append) against ferro's own Sampler objects, one per stream, each fed
    its growing history the way gen_token keeps it (hist.push_back, server.cpp:342)."""
    rng = np.random.default_rng(404)
    S, V, steps = 5, 700, 12
    params = W.make_params(S, temperature=0.9, top_k=40, top_p=0.9, repetition_penalty=1.3)
    params["temperature"][1] = 0.0
    params["top_k"][3] = 0
    params["repeat_last_n"][4] = 8
    seeds = [11, 22, 33, 44, 55]
    hist0 = [list(rng.integers(0, V, int(rng.integers(0, 30)))) for _ in range(S)]
    rows = [(rng.standard_normal((S, V)) * 2).astype(np.float32) for _ in range(steps)]
    toks, _, _ = oracle_decode_loop(rows, params, seeds, hist0)
    R = O.ref()
    for s in range(S):
        p = np.ascontiguousarray(params[s:s + 1], O.PARAMS_DTYPE)
        h = [int(t) for t in hist0[s]]
        obj = R.ref_sampler_new(O._ptr(p), seeds[s])
        try:
            for k in range(steps):
                x = rows[k][s].copy()
                hh = np.asarray(h, np.int32)
                t = R.ref_sampler_sample(obj, O._ptr(x), V, O._ptr(hh), hh.size)
                assert t == toks[k, s], (s, k)
                h.append(t)
        finally:
            R.ref_sampler_free(obj)


def test_nan_policy_numbers_only():
    """The oracle's NaN policy (ferro's comparator is no strict weak order with a NaN, so its candidates are
    unspecified there): NaN ranks below every number and is never a candidate. Checked against a brute-force sort
    of the numbers: the candidates are the first min(k, #numbers) numbers (value desc, id asc), softmax over them;
    a row of NaNs only gives token 0 with nothing kept."""
    rng = np.random.default_rng(5)
    for trial in range(40):
        V = int(rng.integers(2, 300))
        x = (rng.standard_normal(V) * 2).astype(np.float32)
        x[rng.random(V) < rng.uniform(0.05, 0.9)] = np.nan
        k = int(rng.choice([1, 3, 40, 0, V + 5]))
        p = O.make_params(temperature=0.7, top_k=k, top_p=1.0, repetition_penalty=1.0)
        tok, ids, probs, keep, ncand = O.sample(x, [], p[0], 0.37, kcap=V)
        num = [i for i in range(V) if x[i] == x[i]]
        if not num:
            assert (tok, keep, ncand) == (0, 0, 0)
            continue
        if k == 1:
            continue                                   # greedy: ferro's scan, defined with NaN (never moves onto it)
        order = sorted(num, key=lambda i: (-float(x[i]), i))
        kk = min(k if 0 < k < V else V, len(num))
        assert ncand == kk
        np.testing.assert_array_equal(ids, order[:kk])
        mx = np.float32(x[order[0]])
        e = np.array([np.exp(np.float64(np.float32(x[i] - mx)) / np.float64(np.float32(0.7))) for i in order[:kk]])
        np.testing.assert_allclose(probs, e / e.sum(), rtol=1e-13)
        assert x[tok] == x[tok]                        # a number is drawn


def test_bf16_valued_matches_torch_rounding():
    """The bf16-valued test rows (round to nearest even) agree with torch's float32 -> bfloat16 conversion, ties and
    specials included."""
    import torch
    rng = np.random.default_rng(11)
    x = (rng.standard_normal(1 << 16) * 3).astype(np.float32)
    bits = x.view(np.uint32)
    bits[:256] = (bits[:256] & 0xFFFF0000) | 0x8000         # exactly halfway: ties to even
    x[256:260] = [np.inf, -np.inf, 0.0, -0.0]
    want = torch.from_numpy(x.copy()).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(bf16_valued(x).view(np.uint32), want.view(np.uint32))
