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
