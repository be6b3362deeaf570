"""fs_decode_step(_hp): one decode step in one launch - each stream's draw from its device mt19937_64 stream, the sampled
token, and the token appended to the stream's history (server.cpp:603-606, then gen_token's push_back at :342) -
against the oracle's decode loop (sample each stream with its own std::mt19937_64 draws, then append), which is
pinned against ferro's Sampler objects. Includes steps across the engine's twists (every 312 draws), large rows
whose segments read the draw (k > 2048 and top_k = 0), greedy streams (no draw consumed) and the capacity check."""
import os
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

from ferro_amd import workloads as W  # noqa: E402
import ferro_amd as F  # noqa: E402
from parity_util import oracle_decode_loop  # noqa: E402


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module", autouse=True, params=["host", "device"])
def gpu(request):
    """Every test runs twice: with the host copy of the parameters (fs_decode_step_hp: the small-k kernel for the
    batches it fits) and with the device copy only (fs_decode_step: the fused kernel)."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    F.sampler.Context.default()
    F.sampler.ROUTE = request.param
    say(f"== route {request.param}")
    yield
    F.sampler.ROUTE = "host"
    torch.cuda.synchronize()


def _hist(hist0):
    h = torch.from_numpy(np.concatenate([np.asarray(x, np.int32) for x in hist0] + [np.zeros(0, np.int32)])).cuda()
    o = torch.from_numpy(np.concatenate([[0], np.cumsum([len(x) for x in hist0])]).astype(np.int64)).cuda()
    return h, o


def _run(rows, p, seeds, hist0):
    d = F.DeviceRng(np.array(seeds, np.uint64))
    hist, off = _hist(hist0)
    got = []
    for k, x in enumerate(rows):
        tok, keep, hist, off = F.decode_step(torch.from_numpy(x).cuda(), p, d, hist=hist, hist_off=off)
        got.append(tok)
    torch.cuda.synchronize()
    assert F.device_error() == 0
    return torch.stack(got).cpu().numpy(), hist, off


def _check(rows, p, seeds, hist0):
    want, want_hist, want_off = oracle_decode_loop(rows, p, seeds, hist0)
    got, hist, off = _run(rows, p, seeds, hist0)
    np.testing.assert_array_equal(got, want)
    o = off.cpu().numpy()
    np.testing.assert_array_equal(o, want_off)
    np.testing.assert_array_equal(hist[:o[-1]].cpu().numpy(), want_hist)


def test_decode_steps_match_the_oracle_loop():
    rng = np.random.default_rng(606)
    S, V, steps = 6, 5000, 10
    p = W.make_params(S, temperature=0.8, top_k=40, top_p=0.9, repetition_penalty=1.4)
    p["temperature"][1] = 0.0                          # greedy: draws nothing
    p["top_k"][2] = 0                                  # every token a candidate
    p["repeat_last_n"][3] = 6
    p["frequency_penalty"][4], p["presence_penalty"][4] = 0.5, 0.3
    seeds = [11, 22, 33, 44, 55, 66]
    hist0 = [list(rng.integers(0, V, int(rng.integers(0, 40)))) for _ in range(S)]
    hist0[5] = []
    rows = [(rng.standard_normal((S, V)) * 2.5).astype(np.float32) for _ in range(steps)]
    _check(rows, p, seeds, hist0)


def test_decode_steps_across_twists():
    """330 steps: every sampling stream crosses two of its engine's twists (the first draw twists, then every 312th);
    a greedy stream keeps its engine untouched."""
    rng = np.random.default_rng(7)
    S, V, steps = 3, 700, 330
    p = W.make_params(S, temperature=1.0, top_k=20, top_p=1.0, repetition_penalty=1.0)
    p["temperature"][2] = 0.0
    seeds = [9, 10, 12]
    rows = [(rng.standard_normal((S, V)) * 2).astype(np.float32) for _ in range(steps)]
    _check(rows, p, seeds, [[], [1, 2, 3], []])


def test_decode_steps_large_rows():
    """V = 262144 rows of every kind: large k and top_k = 0 (their segments read the draw too), k > 64, k <= 64,
    greedy, spiky rows that take the short list."""
    rng = np.random.default_rng(8)
    S, V, steps = 8, 262144, 3
    p = W.make_params(S, temperature=0.9, top_k=0, top_p=0.95, repetition_penalty=1.1)
    p["top_k"] = [0, 5000, 300, 40, 1, 0, 2100, 64]
    p["temperature"][4] = 0.0
    p["frequency_penalty"][6] = 0.2
    seeds = list(range(100, 100 + S))
    rows = []
    for k in range(steps):
        x = (rng.standard_normal((S, V)) * 1.5).astype(np.float32)
        x[5, rng.choice(V, 10, replace=False)] += 25.0                 # row 5: the short list
        rows.append(x)
    hist0 = [list(rng.integers(0, V, 300)) for _ in range(S)]
    _check(rows, p, seeds, hist0)


def test_decode_step_capacity():
    """An output buffer one id short: FS_DEVERR_HIST_APPEND, the ids past it not written."""
    rng = np.random.default_rng(5)
    S, V = 4, 5000
    p = W.make_params(S, temperature=0.7, top_k=10)
    d = F.DeviceRng(np.arange(1, S + 1, dtype=np.uint64))
    hist, off = _hist([[1, 2], [3], [], [4, 5, 6]])
    x = torch.from_numpy((rng.standard_normal((S, V))).astype(np.float32)).cuda()
    tok, keep, out, oo = F.decode_step(x, p, d, hist=hist, hist_off=off, out_cap=6 + S - 1)
    torch.cuda.synchronize()
    bits = F.device_error()
    assert bits & 4, bits                               # FS_DEVERR_HIST_APPEND
    np.testing.assert_array_equal(oo.cpu().numpy(), [0, 3, 5, 6, 10])
    assert F.device_error() == 0


def test_decode_steps_small_k_serving_rows():
    """Serving rows that the small-k kernel takes on the host route: top-k 40-64 with top-p and repetition windows,
    greedy rows among them (one with frequency / presence counts), then an all-greedy batch (the greedy-only kernel:
    no draw consumed, tokens appended)."""
    rng = np.random.default_rng(64)
    S, V, steps = 12, 65536, 5
    p = W.make_params(S, temperature=0.8, top_k=64, top_p=0.95, repetition_penalty=1.1)
    p["top_k"][3::4] = 40
    p["temperature"][1] = 0.0
    p["temperature"][5] = 0.0
    p["frequency_penalty"][5], p["presence_penalty"][5] = 0.4, 0.2
    p["repeat_last_n"][7] = 8
    seeds = list(range(500, 500 + S))
    hist0 = [list(W.zipf_ids(rng, V, int(rng.integers(0, 300)))) for _ in range(S)]
    rows = [W.mixture_logits(rng, S, V) for _ in range(steps)]
    _check(rows, p, seeds, hist0)
    g = W.make_params(4, temperature=0.0, repetition_penalty=1.2)
    _check([W.mixture_logits(rng, 4, V) for _ in range(3)], g, [1, 2, 3, 4], [[5, 6], [], [7], [8, 8, 8]])
