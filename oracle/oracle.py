"""ctypes bindings for the CPU oracle (liboracle.so) and, where built, the reference sampler (_ref/libferro_ref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, as the
checker. The product package (ferro_amd/) never imports this module.

The oracle restates /root/reference/src/sampler.cpp:10-50 (see sampler_oracle.c); _ref is that file compiled
as-is by oracle/Makefile.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libferro_ref.so")

# Same layout as fs_row_params (include/ferro_sampler.h) and fso_params (sampler_oracle.h).
PARAMS_DTYPE = np.dtype([
    ("temperature", np.float32), ("top_k", np.int32), ("top_p", np.float32), ("min_p", np.float32),
    ("repetition_penalty", np.float32), ("frequency_penalty", np.float32), ("presence_penalty", np.float32),
    ("repeat_last_n", np.int32), ("penalty_from", np.int32), ("softcap", np.float32),
])
assert PARAMS_DTYPE.itemsize == 40


def make_params(n=1, temperature=0.05, top_k=50, top_p=1.0, min_p=0.0, repetition_penalty=1.05,
                frequency_penalty=0.0, presence_penalty=0.0, repeat_last_n=-1, penalty_from=0, softcap=0.0):
    """Params array with ferro's SamplerParams defaults (sampler.h:12-20)."""
    p = np.zeros(n, PARAMS_DTYPE)
    p["temperature"] = temperature
    p["top_k"] = top_k
    p["top_p"] = top_p
    p["min_p"] = min_p
    p["repetition_penalty"] = repetition_penalty
    p["frequency_penalty"] = frequency_penalty
    p["presence_penalty"] = presence_penalty
    p["repeat_last_n"] = repeat_last_n
    p["penalty_from"] = penalty_from
    p["softcap"] = softcap
    return p


_P = ctypes.c_void_p
_lib = None
_ref = None


def _ptr(a):
    return None if a is None else a.ctypes.data_as(_P)


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        L.fso_sample.restype = ctypes.c_int
        L.fso_sample.argtypes = [_P, ctypes.c_int, _P, ctypes.c_int64, _P, ctypes.c_double, _P, _P, ctypes.c_int,
                                 _P, _P]
        L.fso_penalize.restype = ctypes.c_int
        L.fso_penalize.argtypes = [_P, ctypes.c_int, _P, ctypes.c_int64, _P]
        L.fso_sample_batch.restype = None
        L.fso_sample_batch.argtypes = [_P, ctypes.c_int64, ctypes.c_int, ctypes.c_int, _P, _P, _P, _P, _P, _P, _P,
                                       ctypes.c_int, _P, _P, ctypes.c_int]
        L.fso_lookup_draft.restype = ctypes.c_int
        L.fso_lookup_draft.argtypes = [_P, ctypes.c_int64, ctypes.c_int, ctypes.c_int32, ctypes.c_int, _P]
        L.fso_verify.restype = None
        L.fso_verify.argtypes = [_P, ctypes.c_int64, ctypes.c_int, ctypes.c_int, _P, _P, _P, _P, _P, _P,
                                 ctypes.c_int32, _P, _P]
        L.fso_mt64_seed.argtypes = [_P, ctypes.c_uint64]
        L.fso_mt64_next.restype = ctypes.c_uint64
        L.fso_mt64_next.argtypes = [_P]
        L.fso_softcap.restype = None
        L.fso_softcap.argtypes = [_P, _P, ctypes.c_int64, ctypes.c_float, ctypes.c_int]
        L.fso_canonical.restype = ctypes.c_double
        L.fso_canonical.argtypes = [ctypes.c_uint64]
        _lib = L
    return _lib


def ref_available():
    return os.path.exists(REF_PATH)


def ref():
    """The reference sampler compiled from /root/reference/src/sampler.cpp (None if not built)."""
    global _ref
    if _ref is None and ref_available():
        R = ctypes.CDLL(REF_PATH)
        R.ref_sampler_new.restype = _P
        R.ref_sampler_new.argtypes = [_P, ctypes.c_uint64]
        R.ref_sampler_free.argtypes = [_P]
        R.ref_sampler_sample.restype = ctypes.c_int
        R.ref_sampler_sample.argtypes = [_P, _P, ctypes.c_int, _P, ctypes.c_int64]
        R.ref_sample_batch.restype = None
        R.ref_sample_batch.argtypes = [_P, ctypes.c_int64, ctypes.c_int, ctypes.c_int, _P, _P, _P, _P, _P,
                                       ctypes.c_int]
        _ref = R
    return _ref


# ---------------------------------------------------------------------------------------------- oracle calls
def softcap(x, cap, nthreads=1):
    """The model's host softcap loop (model_gemma4_gpu.cpp:282-283) on a copy of x (float32)."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    lib().fso_softcap(_ptr(x), _ptr(out), x.size, float(cap), int(nthreads))
    return out


def penalize(row, hist, params):
    row = np.ascontiguousarray(row, np.float32).copy()
    hist = np.ascontiguousarray(hist, np.int32)
    p = np.ascontiguousarray(params, PARAMS_DTYPE).reshape(1)
    lib().fso_penalize(_ptr(row), row.size, _ptr(hist), hist.size, _ptr(p))
    return row


def sample(row, hist, params, u=0.0, kcap=0):
    """One sample() call on a copy of `row`. Returns (tok, cand_ids[:min(k,kcap)], cand_probs, keep, ncand)."""
    row = np.ascontiguousarray(row, np.float32).copy()
    hist = np.ascontiguousarray(hist, np.int32)
    p = np.ascontiguousarray(params, PARAMS_DTYPE).reshape(1)
    ids = np.zeros(max(kcap, 1), np.int32)
    probs = np.zeros(max(kcap, 1), np.float64)
    keep = np.zeros(1, np.int32)
    ncand = np.zeros(1, np.int32)
    tok = lib().fso_sample(_ptr(row), row.size, _ptr(hist), hist.size, _ptr(p), float(u), _ptr(ids), _ptr(probs),
                           kcap, _ptr(keep), _ptr(ncand))
    m = min(int(ncand[0]), kcap)
    return tok, ids[:m], probs[:m], int(keep[0]), int(ncand[0])


def sample_batch(logits, hist, hist_off, params, u, kcap=0, nthreads=1):
    """Batch sample on a COPY of logits [B, ld] (the first n columns used; n = logits.shape[1])."""
    x = np.ascontiguousarray(logits, np.float32).copy()
    B, n = x.shape
    hist = np.ascontiguousarray(hist, np.int32)
    hist_off = np.ascontiguousarray(hist_off, np.int64)
    params = np.ascontiguousarray(params, PARAMS_DTYPE)
    u = np.ascontiguousarray(u, np.float64)
    tok = np.zeros(B, np.int32)
    keep = np.zeros(B, np.int32)
    ncand = np.zeros(B, np.int32)
    ids = np.zeros((B, kcap), np.int32) if kcap else None
    probs = np.zeros((B, kcap), np.float64) if kcap else None
    lib().fso_sample_batch(_ptr(x), n, B, n, _ptr(hist), _ptr(hist_off), _ptr(params), _ptr(u), _ptr(tok), _ptr(ids),
                           _ptr(probs), kcap, _ptr(keep), _ptr(ncand), nthreads)
    return dict(tok=tok, keep=keep, ncand=ncand, cand_ids=ids, cand_probs=probs)


def verify(logits, rows, row_off, hist, hist_off, params, u, eos_id=-1):
    x = np.ascontiguousarray(logits, np.float32).copy()
    R, n = x.shape
    rows = np.ascontiguousarray(rows, np.int32)
    row_off = np.ascontiguousarray(row_off, np.int64)
    S = row_off.size - 1
    tok = np.zeros(R, np.int32)
    acc = np.zeros(S, np.int32)
    lib().fso_verify(_ptr(x), n, S, n, _ptr(rows), _ptr(row_off), _ptr(np.ascontiguousarray(hist, np.int32)),
                     _ptr(np.ascontiguousarray(hist_off, np.int64)),
                     _ptr(np.ascontiguousarray(params, PARAMS_DTYPE)),
                     _ptr(np.ascontiguousarray(u, np.float64)), int(eos_id), _ptr(tok), _ptr(acc))
    return tok, acc


class MT64:
    """mt19937_64 restated in C (sampler_oracle.c)."""

    def __init__(self, seed):
        self._state = ctypes.create_string_buffer(312 * 8 + 8)
        lib().fso_mt64_seed(self._state, seed)

    def next(self):
        return int(lib().fso_mt64_next(self._state))


def lookup_draft(hist, kmax, eos=-1, min_n=2):
    """server.cpp:552-564 restated in C (fso_lookup_draft)."""
    h = np.ascontiguousarray(hist, np.int32)
    out = np.zeros(max(kmax, 1), np.int32)
    d = lib().fso_lookup_draft(_ptr(h), h.size, kmax, eos, min_n, _ptr(out))
    return out[:d].copy()


def hist_append(hist, hist_off, tok, row_off=None, count=None):
    """gen_token's `j.hist.push_back(id)` (server.cpp:342) for each stream's consumed tokens, in row order: the decode
    loop (server.cpp:603-606) consumes one token per stream, the verify window (server.cpp:627-637) its first
    count[s] rows. CSR in, CSR out (offsets rebased to 0). Counts outside [0, the stream's rows] are clamped, as the
    device entry point does (it also flags them)."""
    hist = np.asarray(hist, np.int32)
    off = np.asarray(hist_off, np.int64)
    tok = np.asarray(tok, np.int32)
    S = off.size - 1
    ro = np.arange(S + 1, dtype=np.int64) if row_off is None else np.asarray(row_off, np.int64)
    streams = []
    for s in range(S):
        h = list(hist[off[s]:off[s + 1]])
        rows = int(ro[s + 1] - ro[s])
        n = 1 if count is None else int(count[s])
        n = min(max(n, 0), rows)
        for i in range(n):
            h.append(int(tok[ro[s] + i]))
        streams.append(h)
    out_off = np.zeros(S + 1, np.int64)
    out_off[1:] = np.cumsum([len(h) for h in streams])
    out = np.array([t for h in streams for t in h], np.int32)
    return out, out_off


def canonical(x):
    return float(lib().fso_canonical(x))


def first_u(seed):
    """u of the first draw of Sampler(seed): generate_canonical of mt19937_64(seed)'s first output."""
    return canonical(MT64(seed).next())


# ---------------------------------------------------------------------------------------------- reference calls
def ref_sample_stream(params, seed, rows, hists):
    """Run ONE reference Sampler(params, seed) over successive (row, history) calls; returns the token list."""
    R = ref()
    p = np.ascontiguousarray(params, PARAMS_DTYPE).reshape(1)
    s = R.ref_sampler_new(_ptr(p), seed)
    try:
        out = []
        for row, h in zip(rows, hists):
            x = np.ascontiguousarray(row, np.float32).copy()
            hh = np.ascontiguousarray(h, np.int32)
            out.append(R.ref_sampler_sample(s, _ptr(x), x.size, _ptr(hh), hh.size))
        return out
    finally:
        R.ref_sampler_free(s)


def ref_sample_batch(logits, hist, hist_off, params, seeds, nthreads=1, inplace=False):
    """Each row through a fresh reference Sampler(seed[b]); rows penalised in place when inplace."""
    R = ref()
    x = logits if inplace else np.ascontiguousarray(logits, np.float32).copy()
    B, n = x.shape
    tok = np.zeros(B, np.int32)
    R.ref_sample_batch(_ptr(x), n, B, n, _ptr(np.ascontiguousarray(hist, np.int32)),
                       _ptr(np.ascontiguousarray(hist_off, np.int64)),
                       _ptr(np.ascontiguousarray(params, PARAMS_DTYPE)),
                       _ptr(np.ascontiguousarray(seeds, np.uint64)), _ptr(tok), nthreads)
    return tok


# ---------------------------------------------------------------------------------------------- parity bar
BOUNDARY = 1e-6


def near_boundary(probs, keep, u, top_p, min_p):
    """True if a sequential-vs-parallel summation difference could flip keep or the drawn index of a row: the
    oracle's candidate probabilities `probs` (candidate order), its kept count, the draw u, top_p and min_p put
    u*tot, top_p or the min-p threshold within 1e-6 (relative) of a cumulative boundary (sampler.cpp:43-49)."""
    c = np.cumsum(probs)
    if len(c) == 0:
        return False
    if top_p < 1.0 and np.any(np.abs(c - np.float64(np.float32(top_p))) <= BOUNDARY):
        return True
    if min_p > 0.0:
        thr = probs[0] * np.float64(np.float32(min_p))
        if np.any(np.abs(probs - thr) <= BOUNDARY * max(thr, 1e-300)):
            return True
    tot = c[max(keep, 1) - 1]
    return bool(np.any(np.abs(u * tot - c[:max(keep, 1)]) <= BOUNDARY))
