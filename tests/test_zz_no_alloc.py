"""GPU: fs_sample_batch_static (the entry point that allocates nothing) against fs_sample_batch.

Both entry points run the same kernels; the static one binds the device's file-scope workspace instead of the
context's allocated one. Every output (tokens, candidate ids, probabilities, kept counts) must be identical, on
three calls in a row, each with a smaller batch than the one before (the workspace keeps the previous call's
contents), and the device error bits must stay clear. A batch past the static limits is refused with FS_E_LIMIT.
"""
import ctypes
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from ferro_amd import workloads as W  # noqa: E402
from ferro_amd._lib import FS_E_LIMIT, lib  # noqa: E402
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


def run(entry, ctx, w, kcap):
    dev = torch.device("cuda", 0)
    ld = w.V + (-w.V) % 4                              # rows 16-byte aligned: the ABI's layout rule
    x = torch.zeros((w.B, ld), dtype=torch.float32, device=dev)
    x[:, :w.V] = torch.from_numpy(w.logits).to(dev)
    params = torch.from_numpy(w.params.view(np.uint8).copy()).to(dev)
    hist = torch.from_numpy(w.hist).to(dev)
    hoff = torch.from_numpy(w.hist_off).to(dev)
    u = torch.from_numpy(w.u).to(dev)
    B, V = w.B, w.V
    tok = torch.full((B,), -7, dtype=torch.int32, device=dev)
    keep = torch.full((B,), -7, dtype=torch.int32, device=dev)
    ids = torch.full((B, kcap), -7, dtype=torch.int32, device=dev)
    probs = torch.full((B, kcap), -7.0, dtype=torch.float64, device=dev)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = entry(ctx.h, P(x), x.stride(0), B, V, P(hist), P(hoff), P(params), P(u), P(tok), kcap, P(ids), P(probs),
               P(keep), st)
    assert rc == 0, f"rc {rc}"
    torch.cuda.synchronize()
    bits = ctypes.c_int32(-1)
    assert lib().fs_device_error(ctx.h, st, ctypes.byref(bits)) == 0
    assert bits.value == 0, f"device error bits {bits.value}"
    return {k: v.cpu().numpy() for k, v in dict(tok=tok, keep=keep, ids=ids, probs=probs).items()}


def mixed(seed, B, V):
    """Greedy, small-k, k in (64, 2048], top_k = 0 and penalised rows, with a partial last tile."""
    rng = np.random.default_rng(seed)
    x = W.mixture_logits(rng, B, V)
    hs = [W.zipf_ids(rng, V, 300) for _ in range(B)]
    p = W.make_params(B, temperature=0.9, top_k=50, top_p=0.9, repetition_penalty=1.1)
    p["temperature"][0] = 0.0
    p["top_k"][1] = 700
    p["top_k"][2] = 0
    p["frequency_penalty"][3] = 0.5
    p["presence_penalty"][3] = 0.25
    return W.Workload(f"mixed_B{B}_V{V}", x, p, np.concatenate(hs).astype(np.int32),
                      np.arange(B + 1, dtype=np.int64) * 300, rng.random(B), np.zeros(B, np.uint64))


def test_static_entry_matches_allocating_entry():
    L = lib()
    ctx_a, ctx_s = Context(), Context()
    # cfg5 (balanced layout, every (row, segment) slot of the static workspace), then cfg3, then a small ragged batch
    for w, kcap in ((W.config5(), 2048), (W.config3(), 64), (mixed(7, 5, 70001), 96)):
        say(f"case {w.name}: B={w.B} V={w.V} kcap={kcap}, fs_sample_batch_static then fs_sample_batch")
        got = run(L.fs_sample_batch_static, ctx_s, w, kcap)
        ref = run(L.fs_sample_batch, ctx_a, w, kcap)
        for k in ref:
            assert np.array_equal(got[k], ref[k]), f"{w.name}: {k} differs between the entry points"
        assert (got["tok"] >= 0).all() and (got["tok"] < w.V).all()


def test_static_entry_takes_every_batch_up_to_its_limit():
    """Every B = 1..512 at V = 262144 fits the static workspace (fewer segments per row where its 512 (row, segment)
    slots would run out) and gives fs_sample_batch's tokens."""
    L = lib()
    ctx_a, ctx_s = Context(), Context()
    dev = torch.device("cuda", 0)
    Bmax, V = 512, 262144
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    x = torch.randn((Bmax, V), generator=g, device=dev, dtype=torch.float32) * 1.5
    p = W.make_params(Bmax, temperature=0.8, top_k=64, top_p=0.95, repetition_penalty=1.0)
    p["temperature"][::7] = 0.0
    params = torch.from_numpy(p.view(np.uint8).copy()).to(dev)
    u = torch.rand(Bmax, generator=g, device=dev, dtype=torch.float64)
    ta = torch.empty(Bmax, dtype=torch.int32, device=dev)
    ts = torch.empty(Bmax, dtype=torch.int32, device=dev)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    say(f"case sweep: B = 1..{Bmax}, V={V}")
    for B in range(1, Bmax + 1):
        ts.fill_(-7)
        rs = L.fs_sample_batch_static(ctx_s.h, P(x), V, B, V, None, None, P(params), P(u), P(ts), 0, None, None, None,
                                      st)
        ra = L.fs_sample_batch(ctx_a.h, P(x), V, B, V, None, None, P(params), P(u), P(ta), 0, None, None, None, st)
        assert rs == 0 and ra == 0, f"B={B}: rc static {rs}, allocating {ra}"
        if B % 32 == 1 or B in (17, 23, 33, 46, 73, 97, 511, 512):
            torch.cuda.synchronize()
            assert torch.equal(ts[:B], ta[:B]), f"B={B}: tokens differ between the entry points"
    torch.cuda.synchronize()
    for c in (ctx_a, ctx_s):
        bits = ctypes.c_int32(-1)
        assert lib().fs_device_error(c.h, st, ctypes.byref(bits)) == 0 and bits.value == 0


def test_static_entry_refuses_batches_past_its_limit():
    L = lib()
    ctx = Context()
    w = mixed(3, 513, 4096)
    say(f"case limit: B={w.B} V={w.V}")
    dev = torch.device("cuda", 0)
    x = torch.zeros((w.B, w.V), dtype=torch.float32, device=dev)
    params = torch.from_numpy(w.params.view(np.uint8).copy()).to(dev)
    u = torch.zeros(w.B, dtype=torch.float64, device=dev)
    tok = torch.empty(w.B, dtype=torch.int32, device=dev)
    rc = L.fs_sample_batch_static(ctx.h, P(x), x.stride(0), w.B, w.V, None, None, P(params), P(u), P(tok), 0, None,
                                  None, None, None)
    assert rc == FS_E_LIMIT
