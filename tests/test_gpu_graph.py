"""GPU: sampling calls captured into a HIP graph and replayed.

A serving loop can record its sampling calls into a graph once and replay it every step (bench.py times the
headline that way). Once warm, fs_sample_batch and fs_sample_batch_static launch one kernel and nothing else, so
they capture as they run. The kernels leave their workspace (row histograms, counters) at zero, which a replay
relies on. Each replay is checked against the eager outputs of the same calls, with eager calls on other inputs
between the replays, for a small mixed batch (greedy, small k, k in (64, 2048], top_k = 0, penalties, a partial
last tile) and for a batch large enough for the balanced segment layout.
"""
import ctypes
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from ferro_amd import workloads as W  # noqa: E402
from ferro_amd._lib import lib  # noqa: E402
from ferro_amd.sampler import Context  # noqa: E402


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    yield
    torch.cuda.synchronize()


def P(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def mixed(seed, B, V):
    rng = np.random.default_rng(seed)
    x = W.mixture_logits(rng, B, V)
    hs = [W.zipf_ids(rng, V, 200) for _ in range(B)]
    p = W.make_params(B, temperature=0.9, top_k=50, top_p=0.9, repetition_penalty=1.1)
    r = rng.random(B)
    p["temperature"][r < 0.1] = 0.0
    p["top_k"][(r >= 0.1) & (r < 0.3)] = 700
    p["top_k"][(r >= 0.3) & (r < 0.35)] = 0
    p["frequency_penalty"][(r >= 0.35) & (r < 0.5)] = 0.5
    p["presence_penalty"][(r >= 0.35) & (r < 0.5)] = 0.25
    return W.Workload(f"mixed_B{B}_V{V}", x, p, np.concatenate(hs).astype(np.int32),
                      np.arange(B + 1, dtype=np.int64) * 200, rng.random(B), np.zeros(B, np.uint64))


class Call:
    """Device inputs and outputs of one sampling call."""

    def __init__(self, w, kcap):
        dev = torch.device("cuda", 0)
        ld = w.V + (-w.V) % 4
        self.x = torch.zeros((w.B, ld), dtype=torch.float32, device=dev)
        self.x[:, :w.V] = torch.from_numpy(w.logits).to(dev)
        self.params = torch.from_numpy(w.params.view(np.uint8).copy()).to(dev)
        self.hist = torch.from_numpy(w.hist).to(dev)
        self.hoff = torch.from_numpy(w.hist_off).to(dev)
        self.u = torch.from_numpy(w.u).to(dev)
        self.B, self.V, self.kcap = w.B, w.V, kcap
        self.tok = torch.empty(w.B, dtype=torch.int32, device=dev)
        self.keep = torch.empty(w.B, dtype=torch.int32, device=dev)
        self.ids = torch.empty((w.B, kcap), dtype=torch.int32, device=dev)
        self.probs = torch.empty((w.B, kcap), dtype=torch.float64, device=dev)

    def launch(self, entry, ctx, stream):
        rc = entry(ctx.h, P(self.x), self.x.stride(0), self.B, self.V, P(self.hist), P(self.hoff), P(self.params),
                   P(self.u), P(self.tok), self.kcap, P(self.ids), P(self.probs), P(self.keep),
                   ctypes.c_void_p(stream.cuda_stream))
        assert rc == 0, f"rc {rc}"

    def poison(self):
        for t in (self.tok, self.keep, self.ids):
            t.fill_(-7)
        self.probs.fill_(-7.0)

    def out(self):
        return {k: getattr(self, k).cpu().numpy().copy() for k in ("tok", "keep", "ids", "probs")}


def check_clean(ctx):
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    bits = ctypes.c_int32(-1)
    assert lib().fs_device_error(ctx.h, st, ctypes.byref(bits)) == 0
    assert bits.value == 0, f"device error bits {bits.value}"


@pytest.mark.parametrize("static", [False, True])
@pytest.mark.parametrize("B,V", [(24, 70001), (136, 65536)])
def test_graph_replays_match_eager(B, V, static):
    say(f"graph replay: B={B} V={V} static={static}")
    L = lib()
    entry = L.fs_sample_batch_static if static else L.fs_sample_batch
    ctx = Context.default(torch.device("cuda", 0))
    calls = [Call(mixed(100 + B + i, B, V), kcap=16) for i in range(2)]
    other = Call(mixed(7, B, V), kcap=16)
    cur = torch.cuda.current_stream()
    want = []
    for c in calls:                                    # eager (also warms the workspace up)
        c.poison()                                     # outputs a call leaves unwritten compare as -7
        c.launch(entry, ctx, cur)
        torch.cuda.synchronize()
        want.append(c.out())
    check_clean(ctx)
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(cur)
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            for c in calls:
                c.launch(entry, ctx, side)
    cur.wait_stream(side)
    torch.cuda.synchronize()
    for rep in range(3):
        for c in calls:
            c.poison()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for i, c in enumerate(calls):
            got = c.out()
            for k in want[i]:
                np.testing.assert_array_equal(got[k], want[i][k], err_msg=f"replay {rep} call {i} {k}")
        other.launch(entry, ctx, cur)                  # eager work between the replays
        torch.cuda.synchronize()
        check_clean(ctx)
    del g


def test_replay_after_the_context_grew():
    """A captured call keeps the workspace addresses it was recorded with. An eager call on the same context that
    needs a larger workspace then replaces the buffers: they are retired (kept until the context is destroyed), not
    freed, so the replay still runs on valid memory and matches its eager outputs."""
    say("graph replay after growth: capture B=24, eager B=300, replay")
    L = lib()
    ctx = Context()
    small = Call(mixed(301, 24, 65536), kcap=16)
    big = Call(mixed(302, 300, 65536), kcap=16)
    cur = torch.cuda.current_stream()
    small.poison()
    small.launch(L.fs_sample_batch, ctx, cur)
    torch.cuda.synchronize()
    want = small.out()
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(cur)
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            small.launch(L.fs_sample_batch, ctx, side)
    cur.wait_stream(side)
    torch.cuda.synchronize()
    big.launch(L.fs_sample_batch, ctx, cur)            # grows every workspace buffer of the context
    torch.cuda.synchronize()
    check_clean(ctx)
    for rep in range(2):
        small.poison()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = small.out()
        for k in want:
            np.testing.assert_array_equal(got[k], want[k], err_msg=f"replay {rep} {k}")
    del g
