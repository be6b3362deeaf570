"""CPU checks of the C ABI library: it loads, exports every symbol include/ferro_sampler.h declares, rejects bad
arguments before touching the device, and its host draw source is libstdc++'s mt19937_64 + generate_canonical
(the reference Sampler's stream, src/sampler.h:25,32)."""
import ctypes
import os
import re

import numpy as np
import pytest

from ferro_amd import _lib
from ferro_amd import workloads as W

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ferro_sampler.h")


def declared_symbols():
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(fs_[a-z_0-9]+)\s*\(", txt)))


def test_header_symbols_exported_and_bound():
    L = _lib.lib()
    syms = declared_symbols()
    assert "fs_sample_batch" in syms and "fs_verify" in syms and "fs_argmax_batch" in syms
    for s in syms:
        assert hasattr(L, s), s
        assert s in _lib.SIGNATURES, s
    assert set(_lib.SIGNATURES) == set(syms)


def test_params_layout_matches_header():
    txt = open(HEADER).read()
    body = txt[txt.index("typedef struct fs_row_params {"):txt.index("} fs_row_params;")]
    fields = re.findall(r"\b(?:float|int32_t)\s+(\w+);", body)
    assert tuple(fields) == _lib.PARAMS_DTYPE.names


def test_invalid_arguments_rejected_without_device():
    L = _lib.lib()
    P = ctypes.c_void_p
    assert L.fs_sample_batch(None, None, 0, 0, 0, None, None, None, None, None, 0, None, None, None, None) \
        == _lib.FS_E_INVALID
    assert L.fs_verify(None, None, 0, 0, 0, 0, None, None, None, None, None, None, -1, None, None, None) \
        == _lib.FS_E_INVALID
    assert L.fs_argmax_batch(None, None, 0, 0, 0, None, None, None, None, None) == _lib.FS_E_INVALID
    assert L.fs_penalize_batch(None, None, 0, 0, 0, None, None, None, None) == _lib.FS_E_INVALID
    assert L.fs_rng_create(1, None) == _lib.FS_E_INVALID
    assert L.fs_drng_create(0, None, None, None) == _lib.FS_E_INVALID
    assert L.fs_drng_draw(None, None, None, None, 0, None) == _lib.FS_E_INVALID
    assert L.fs_drng_skip(None, None, None, None) == _lib.FS_E_INVALID
    h = P()
    assert L.fs_create(ctypes.byref(h)) == _lib.FS_OK
    fake = P(16)   # never dereferenced: argument checks fail first
    # history append: no context / offsets / tokens / outputs, negative capacity, outputs aliasing inputs
    assert L.fs_hist_append(None, 1, fake, fake, fake, None, None, P(32), 4, P(48), None) == _lib.FS_E_INVALID
    assert L.fs_hist_append(h, 1, fake, None, fake, None, None, P(32), 4, P(48), None) == _lib.FS_E_INVALID
    assert L.fs_hist_append(h, 1, fake, fake, fake, None, None, P(32), -1, P(48), None) == _lib.FS_E_INVALID
    assert L.fs_hist_append(h, 1, fake, fake, fake, None, None, None, 4, P(48), None) == _lib.FS_E_INVALID
    assert L.fs_hist_append(h, 1, fake, P(48), fake, None, None, P(32), 4, P(48), None) == _lib.FS_E_INVALID
    assert L.fs_hist_append(h, 1, fake, fake, fake, None, None, fake, 4, P(48), None) == _lib.FS_E_INVALID
    assert L.fs_hist_append(h, 1, None, fake, fake, None, None, P(32), 4, P(48), None) == _lib.FS_E_INVALID
    assert L.fs_hist_append(h, 1, fake, fake, None, None, None, P(32), 4, P(48), None) == _lib.FS_E_INVALID
    # misaligned logits / ld not a multiple of 4 / ld < V / V < 1
    assert L.fs_sample_batch(h, P(4), 8, 1, 8, None, None, fake, None, fake, 0, None, None, None, None) \
        == _lib.FS_E_INVALID
    assert L.fs_sample_batch(h, fake, 6, 1, 6, None, None, fake, None, fake, 0, None, None, None, None) \
        == _lib.FS_E_INVALID
    assert L.fs_sample_batch(h, fake, 4, 1, 8, None, None, fake, None, fake, 0, None, None, None, None) \
        == _lib.FS_E_INVALID
    assert L.fs_sample_batch(h, fake, 4, 1, 0, None, None, fake, None, fake, 0, None, None, None, None) \
        == _lib.FS_E_INVALID
    # candidate outputs without kcap
    assert L.fs_sample_batch(h, fake, 8, 1, 8, None, None, fake, None, fake, 0, fake, None, None, None) \
        == _lib.FS_E_INVALID
    assert _lib.lib().fs_strerror(_lib.FS_E_INVALID) == b"invalid argument"


@pytest.mark.parametrize("seed", [1, 5489, 2**63 + 7, 123456789])
def test_rng_is_libstdcxx_stream(seed):
    from ferro_amd.sampler import Rng
    r = Rng(seed)
    got = r.next_u(700)
    mt = W.MT19937_64(seed)
    want = np.array([W.canonical(mt.next()) for _ in range(700)])
    np.testing.assert_array_equal(got, want)
    # copy continues the same stream independently
    c = r.copy()
    np.testing.assert_array_equal(c.next_u(5), r.next_u(5))


def test_planner_layouts_on_mocked_devices():
    """fs_plan_layout: the segment grid on MI355X (256 CUs, 8 XCDs), and its XCD-count guard on mocked devices."""
    rc, nseg, st, slots = _lib.plan_layout(256, 8, 64, 262144)      # the headline batch: 8 segments of 8 tiles
    assert (rc, nseg, st, slots) == (_lib.FS_OK, 8, 8, 512)
    rc, nseg, st, slots = _lib.plan_layout(256, 8, 272, 65536)      # cfg4: one segment per row
    assert (rc, nseg, st) == (_lib.FS_OK, 1, 16)
    for x in (1, 2, 4, 8):                                           # every partition mode keeps the hand-off
        rc, nseg, _, _ = _lib.plan_layout(32 * x, x, 64, 262144)
        assert rc == _lib.FS_OK and nseg >= 1, x
    for x in (0, 3, 5, 6, 7, 12, 16):                                # counts that do not divide 8: every row alone
        rc, nseg, st, slots = _lib.plan_layout(256, x, 64, 262144)
        assert (rc, nseg, slots) == (_lib.FS_OK, 0, 0), x
    rc, nseg, _, _ = _lib.plan_layout(256, 8, 4, 1000)              # rows shorter than a tile: no segments
    assert (rc, nseg) == (_lib.FS_OK, 0)


@pytest.mark.parametrize("V", [262144, 151936, 65536, 4096 * 600])
def test_static_planner_fits_every_batch(V):
    """fs_sample_batch_static takes every B <= 512 (fewer segments where its 512 slots would run out)."""
    for B in range(1, 513):
        rc, nseg, st, slots = _lib.plan_layout(256, 8, B, V, static_ws=True)
        assert rc == _lib.FS_OK, (B, rc)
        assert 1 <= nseg and slots <= 512 and slots == 8 * nseg * ((B + 7) // 8), (B, nseg, slots)
        assert nseg * st >= V // 4096 and (nseg - 1) * st < V // 4096, (B, nseg, st)
        d = _lib.plan_layout(256, 8, B, V)
        assert nseg <= d[1], B                                      # never more segments than fs_sample_batch
    assert _lib.plan_layout(256, 8, 513, V, static_ws=True)[0] == _lib.FS_E_LIMIT


def test_status_codes():
    L = _lib.lib()
    assert L.fs_strerror(_lib.FS_W_RECOVERED).startswith(b"ok")
    assert _lib.check(_lib.FS_OK, "x") == _lib.FS_OK
    with pytest.warns(_lib.RecoveredWarning):
        assert _lib.check(_lib.FS_W_RECOVERED, "x") == _lib.FS_W_RECOVERED
    with pytest.raises(_lib.SamplerError):
        _lib.check(_lib.FS_E_INVALID, "x")


def test_small_k_planner():
    """fs_small_k_plan: the largest segments that give every CU four workgroups, else the most workgroups."""
    def plan(cus, B, V):
        nl, ns = ctypes.c_int32(), ctypes.c_int32()
        rc = _lib.lib().fs_small_k_plan(cus, B, V, ctypes.byref(nl), ctypes.byref(ns))
        return rc, nl.value, ns.value
    assert plan(256, 64, 262144) == (_lib.FS_OK, 16, 16)           # the headline: 1024 workgroups of 64 KB
    assert plan(256, 1, 65536) == (_lib.FS_OK, 4, 16)              # one row: 16 segments of 4096 logits
    assert plan(256, 8, 65536) == (_lib.FS_OK, 4, 16)
    assert plan(256, 256, 262144) == (_lib.FS_OK, 16, 16)
    assert plan(256, 16, 262144) == (_lib.FS_OK, 4, 64)
    assert plan(256, 3, 100) == (_lib.FS_OK, 4, 1)                 # one short segment of the smallest size
    rc, nl, ns = plan(256, 2, 4 * 1024 * 16 * 64 + 1)              # more than 64 of the largest segments
    assert rc == _lib.FS_E_LIMIT
    for V in (1, 4095, 4096, 70001, 262144, 1 << 20):
        rc, nl, ns = plan(256, 4, V)
        assert rc == _lib.FS_OK and ns * 1024 * nl >= V and (ns - 1) * 1024 * nl < V and ns <= 64, V


def test_route_plan_of_the_benchmark_configurations():
    """fs_route_plan, the host parameters' kernel choice of fs_sample_batch_hp / fs_verify_hp, on every configuration
    (host only): the small-k kernel for k <= 64 batches and for greedy ones (its greedy-only form, frequency /
    presence counts only on 4096-logit segments), the fused kernel with four segments per CU for mixed k batches."""
    from ferro_amd import workloads as W
    rp = _lib.route_plan
    assert rp(256, W.config1().params, 65536) == (1, 4, 16, 0)
    assert rp(256, W.config2().params, 65536) == (2, 4, 16, 0)        # greedy, counts, NL = 4
    assert rp(256, W.config3().params, 262144) == (1, 16, 16, 0)
    w4 = W.config4()
    assert rp(256, w4.params, w4.V, total_rows=w4.B, verify=True) == (2, 16, 4, 0)
    w5 = W.config5()
    k, nl, ns, pc = rp(256, w5.params, w5.V)
    assert (k, pc, ns) == (0, 4, 4)
    k, nl, ns, pc = rp(256, W.config3_all_tokens().params, 262144)
    assert (k, pc) == (0, 2)
    g = W.make_params(64, temperature=0.0, frequency_penalty=0.5)      # counts on 16384-logit segments: fused
    assert rp(256, g, 262144)[0] == 0
    g["frequency_penalty"] = 0.0
    g["repetition_penalty"] = 1.3
    assert rp(256, g, 262144)[:2] == (2, 16)                        # greedy with a repetition penalty
    p = W.make_params(64, temperature=0.8, top_k=65)                    # k > 64: fused, uniform layout
    assert rp(256, p, 262144)[0] == 0 and rp(256, p, 262144)[3] == 2
    v = W.make_params(16, temperature=0.0, repetition_penalty=1.2)     # a window with a penalty: fused
    assert rp(256, v, 65536, total_rows=272, verify=True)[0] == 0
    with pytest.raises(_lib.SamplerError):
        rp(256, W.config3().params, 262144, total_rows=65)              # sampling: one record per row
