"""GPU: the merge's bounded wait for a row's segments, forced to give up from the host.

fs_set_wait_limit(ctx, FS_WAIT_GIVE_UP) makes every merging workgroup give up without polling; segments that are
still streaming then finish after their merge has moved on. The merge must raise FS_DEVERR_INTERNAL, mark the
context dirty and compute its row from the logits alone (exact), every kernel exiting normally. The next call on the
context sees the give-up through its host-mapped flag, clears the workspace ahead of its own launch, runs normally
and returns FS_W_RECOVERED; fs_device_error still reports the give-up. Calls with a one-poll limit (whether a merge
gives up then depends on timing) must match the oracle too.
"""
import os
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from oracle import oracle as O  # noqa: E402
from ferro_amd import workloads as W  # noqa: E402
import ferro_amd as F  # noqa: E402
from ferro_amd._lib import FS_DEVERR_INTERNAL, FS_WAIT_GIVE_UP, RecoveredWarning  # noqa: E402
from parity_util import compare  # noqa: E402

NT = min(16, os.cpu_count() or 1)


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    yield
    torch.cuda.synchronize()


def mixed_batch(seed=11, B=12, V=65536):
    """Greedy, small-k, k in (64, 2048], top_k = 0 and penalised rows over V = 16 full tiles."""
    rng = np.random.default_rng(seed)
    x = W.mixture_logits(rng, B, V)
    hs = [W.zipf_ids(rng, V, 200) for _ in range(B)]
    hist = np.concatenate(hs).astype(np.int32)
    off = np.arange(B + 1, dtype=np.int64) * 200
    p = W.make_params(B, temperature=0.8, top_k=40, top_p=0.95, repetition_penalty=1.1)
    p["temperature"][0] = 0.0                          # greedy
    p["top_k"][1] = 1                                  # greedy through top_k == 1
    p["top_k"][2] = 500
    p["top_k"][3] = 0                                  # every token a candidate
    p["top_p"][3] = 0.9
    p["frequency_penalty"][4] = 0.4
    p["presence_penalty"][4] = 0.2
    p["min_p"][5] = 0.05
    u = rng.random(B)
    return W.Workload("handoff_mixed", x, p, hist, off, u, np.zeros(B, np.uint64))


def run_and_check(w, ctx, kcap=64):
    x = torch.from_numpy(w.logits).cuda()
    out = F.sample_batch(x, w.params, w.u, hist=w.hist, hist_off=w.hist_off, kcap=kcap, ctx=ctx, route="device")
    torch.cuda.synchronize()
    g = {k: v.cpu().numpy() for k, v in out.items() if v is not None and not k.startswith("_")}
    o = O.sample_batch(w.logits, w.hist, w.hist_off, w.params, w.u, kcap=kcap, nthreads=NT)
    nb = compare(g, o, w.params, w.u, kcap)
    assert nb <= 1


def test_merge_give_up_is_exact_and_resets():
    w = mixed_batch()
    ctx = F.sampler.Context()
    say(f"case give-up: B={w.B} V={w.V}, every merge gives up")
    ctx.set_wait_limit(FS_WAIT_GIVE_UP)
    run_and_check(w, ctx)                          # merges give up: rows computed alone, tokens still exact
    torch.cuda.synchronize()                       # the give-up has reached the host-mapped flag
    ctx.set_wait_limit(0)
    say("case recovery: the next call clears the workspace and says so")
    w2 = mixed_batch(seed=12)
    with pytest.warns(RecoveredWarning):
        run_and_check(w2, ctx)
    bits = F.device_error(ctx)
    assert bits & FS_DEVERR_INTERNAL, f"the forced give-up was not reported (bits {bits})"
    say("case after recovery: normal merges")
    w3 = mixed_batch(seed=13)
    run_and_check(w3, ctx)
    assert F.device_error(ctx) == 0
    say("case one poll: a give-up depends on timing; tokens exact either way")
    ctx.set_wait_limit(1)
    import warnings
    with warnings.catch_warnings():
        warnings.simplefilter("ignore", RecoveredWarning)
        run_and_check(mixed_batch(seed=14), ctx)
        ctx.set_wait_limit(0)
        run_and_check(mixed_batch(seed=15), ctx)
    F.device_error(ctx)


def test_verify_give_up_is_exact():
    """The fused kernel's verify path (the small-k kernel of fs_verify_hp never waits, so it never gives up)."""
    w = W.config4(S=6, M=9)
    ctx = F.sampler.Context()
    say(f"case verify give-up: rows={w.B} V={w.V}")
    ctx.set_wait_limit(FS_WAIT_GIVE_UP)
    x = torch.from_numpy(w.logits).cuda()
    tok, acc = F.verify(x, w.rows, w.row_off, w.params, u=w.u, hist=w.hist, hist_off=w.hist_off, ctx=ctx,
                      route="device")
    otok, oacc = O.verify(w.logits, w.rows, w.row_off, w.hist, w.hist_off, w.params, w.u)
    np.testing.assert_array_equal(tok.cpu().numpy(), otok)
    np.testing.assert_array_equal(acc.cpu().numpy(), oacc)
    ctx.set_wait_limit(0)
    assert F.device_error(ctx) & FS_DEVERR_INTERNAL
    tok, acc = F.verify(x, w.rows, w.row_off, w.params, u=w.u, hist=w.hist, hist_off=w.hist_off, ctx=ctx,
                      route="device")
    np.testing.assert_array_equal(tok.cpu().numpy(), otok)
    np.testing.assert_array_equal(acc.cpu().numpy(), oacc)
    assert F.device_error(ctx) == 0
