"""ctypes binding of the gfx950 sampler library (libferro_sampler.so, C ABI of include/ferro_sampler.h).

There is no CPU fallback: if the library is missing or fails to load, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
import threading
import warnings

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libferro_sampler.so")

FS_OK = 0
FS_E_INVALID = -1
FS_E_HIP = -2
FS_E_NOMEM = -3
FS_E_DEVICE = -4
FS_E_LIMIT = -5
FS_W_RECOVERED = 1          # success; an earlier call's give-up was cleared (FS_DEVERR_INTERNAL stays set)
FS_WAIT_GIVE_UP = 0xFFFFFFFF
FS_DEVERR_COUNT_OVERFLOW = 1
FS_DEVERR_INTERNAL = 2

# fs_row_params (include/ferro_sampler.h); field order follows ferro's SamplerParams (src/sampler.h:12-21).
PARAMS_DTYPE = np.dtype([
    ("temperature", np.float32), ("top_k", np.int32), ("top_p", np.float32), ("min_p", np.float32),
    ("repetition_penalty", np.float32), ("frequency_penalty", np.float32), ("presence_penalty", np.float32),
    ("repeat_last_n", np.int32), ("penalty_from", np.int32), ("softcap", np.float32),
])
assert PARAMS_DTYPE.itemsize == 40

# Every symbol include/ferro_sampler.h declares, with its ctypes signature.
_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
SIGNATURES = {
    "fs_create": (ctypes.c_int, [_P]),
    "fs_destroy": (ctypes.c_int, [_P]),
    "fs_sample_batch": (ctypes.c_int, [_P, _P, _I64, _I32, _I32, _P, _P, _P, _P, _P, _I32, _P, _P, _P, _P]),
    "fs_sample_batch_static": (ctypes.c_int, [_P, _P, _I64, _I32, _I32, _P, _P, _P, _P, _P, _I32, _P, _P, _P, _P]),
    "fs_sample_batch_hp": (ctypes.c_int, [_P, _P, _I64, _I32, _I32, _P, _P, _P, _P, _P, _P, _I32, _P, _P, _P, _P]),
    "fs_small_k_plan": (ctypes.c_int, [_I32, _I32, _I32, _P, _P]),
    "fs_route_plan": (ctypes.c_int, [_I32, _P, _I32, _I32, _I32, _I32, _P, _P, _P, _P]),
    "fs_argmax_batch": (ctypes.c_int, [_P, _P, _I64, _I32, _I32, _P, _P, _P, _P, _P]),
    "fs_verify": (ctypes.c_int, [_P, _P, _I64, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P, _I32, _P, _P, _P]),
    "fs_verify_hp": (ctypes.c_int, [_P, _P, _I64, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P, _P, _I32, _P, _P, _P]),
    "fs_penalize_batch": (ctypes.c_int, [_P, _P, _I64, _I32, _I32, _P, _P, _P, _P]),
    "fs_softcap_batch": (ctypes.c_int, [_P, _P, _I64, ctypes.c_float, _P]),
    "fs_device_error": (ctypes.c_int, [_P, _P, _P]),
    "fs_set_wait_limit": (ctypes.c_int, [_P, ctypes.c_uint32]),
    "fs_plan_layout": (ctypes.c_int, [_I32, _I32, _I32, _I32, _I32, _P, _P, _P]),
    "fs_error_word": (ctypes.c_int, [_P, _P]),
    "fs_rng_create": (ctypes.c_int, [ctypes.c_uint64, _P]),
    "fs_rng_destroy": (ctypes.c_int, [_P]),
    "fs_rng_next_u": (ctypes.c_int, [_P, _P, _I32]),
    "fs_rng_copy": (ctypes.c_int, [_P, _P]),
    "fs_lookup_draft": (ctypes.c_int, [_P, _I32, _P, _P, _P, _P, _I32, _P, _I32, _P, _P]),
    "fs_hist_append": (ctypes.c_int, [_P, _I32, _P, _P, _P, _P, _P, _P, ctypes.c_int64, _P, _P]),
    "fs_drng_create": (ctypes.c_int, [_I32, _P, _P, _P]),
    "fs_drng_destroy": (ctypes.c_int, [_P]),
    "fs_drng_draw": (ctypes.c_int, [_P, _P, _P, _P, _I32, _P]),
    "fs_decode_step": (ctypes.c_int, [_P, _P, _P, ctypes.c_int64, _I32, _I32, _P, _P, _P, _P, _P, _P, _P,
                                      ctypes.c_int64, _P]),
    "fs_decode_step_hp": (ctypes.c_int, [_P, _P, _P, ctypes.c_int64, _I32, _I32, _P, _P, _P, _P, _P, _P, _P, _P,
                                         ctypes.c_int64, _P]),
    "fs_drng_skip": (ctypes.c_int, [_P, _P, _P, _P]),
    "fs_drng_error": (ctypes.c_int, [_P, _P, _P]),
    "fs_strerror": (ctypes.c_char_p, [ctypes.c_int]),
}

_lib = None
_lock = threading.Lock()


class SamplerError(RuntimeError):
    pass


def lib():
    """Load the library (raises if it has not been built: run ferro_amd/build.py or __graft_entry__.build())."""
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise SamplerError(f"{LIB_PATH} is missing: build it with `python ferro_amd/build.py`")
            L = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                f = getattr(L, name)
                f.restype = res
                f.argtypes = args
            _lib = L
    return _lib


class RecoveredWarning(UserWarning):
    """A call returned FS_W_RECOVERED: it succeeded after clearing the workspace an earlier call's give-up left."""


def check(rc: int, what: str) -> int:
    """Raise on a negative status; warn (RecoveredWarning) on FS_W_RECOVERED. Returns rc."""
    if rc < 0:
        msg = lib().fs_strerror(rc).decode()
        raise SamplerError(f"{what} failed: {msg} ({rc})")
    if rc == FS_W_RECOVERED:
        warnings.warn(f"{what}: {lib().fs_strerror(rc).decode()}", RecoveredWarning, stacklevel=3)
    elif rc != FS_OK:
        raise SamplerError(f"{what}: unexpected status {rc}")
    return rc


def plan_layout(cus: int, xccs: int, B: int, V: int, static_ws: bool = False):
    """fs_plan_layout: (nseg, seg_tiles, slots) the sampling call would launch on such a device (host only)."""
    n, t, sl = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int64()
    rc = lib().fs_plan_layout(cus, xccs, B, V, 1 if static_ws else 0, ctypes.byref(n), ctypes.byref(t),
                              ctypes.byref(sl))
    return rc, n.value, t.value, sl.value


def route_plan(cus: int, params, V: int, total_rows: int = None, verify: bool = False):
    """fs_route_plan: (kernel, nl, nseg, per_cu) fs_sample_batch_hp / fs_verify_hp would launch for these host
    parameter records (numpy structured array of fs_row_params); kernel 0 fused, 1 small-k, 2 greedy-only small-k."""
    import numpy as np
    p = np.ascontiguousarray(params)
    n = len(p)
    k, nl, ns, pc = (ctypes.c_int32() for _ in range(4))
    rc = lib().fs_route_plan(cus, p.ctypes.data_as(ctypes.c_void_p), n, total_rows if total_rows else n, V,
                             1 if verify else 0, ctypes.byref(k), ctypes.byref(nl), ctypes.byref(ns), ctypes.byref(pc))
    check(rc, "fs_route_plan")
    return k.value, nl.value, ns.value, pc.value
