"""Host-side mirror of ferro's sampler interface over the gfx950 kernels.

- `SamplerParams` / `Sampler` mirror ferro::SamplerParams / ferro::Sampler (reference src/sampler.h:12-34): same
  field names, defaults and meaning; `Sampler.sample(logits, n_vocab, history)` returns the token id exactly as
  `int Sampler::sample(float*, int, const std::vector<int>&)` does, drawing from the same libstdc++ mt19937_64
  stream (one draw per non-greedy call, none for greedy: sampler.cpp:19-23, 45-46).
- `sample_batch`, `argmax_batch`, `verify` are the batched device entry points (fs_sample_batch, fs_argmax_batch,
  fs_verify) on torch CUDA tensors, launched on torch's current stream.

PyTorch only supplies device memory and streams; all sampling arithmetic runs in libferro_sampler.so.
"""
from __future__ import annotations

import ctypes
import threading
from dataclasses import dataclass

import numpy as np
import torch

from ._lib import PARAMS_DTYPE, FS_OK, SamplerError, check, lib

__all__ = ["SamplerParams", "Sampler", "Context", "Rng", "params_array", "sample_batch", "argmax_batch", "verify",
           "device_error", "PARAMS_DTYPE", "SamplerError"]


@dataclass
class SamplerParams:
    """ferro::SamplerParams (src/sampler.h:12-21) plus the frequency/presence extension (0 = off)."""
    temperature: float = 0.05
    top_k: int = 50
    top_p: float = 1.0
    min_p: float = 0.0
    repetition_penalty: float = 1.05
    repeat_last_n: int = -1
    penalty_from: int = 0
    seed: int = 0
    frequency_penalty: float = 0.0
    presence_penalty: float = 0.0
    softcap: float = 0.0              # > 0: the model's final-logit softcap, fused into the sampler's read

    def validate(self) -> None:
        """The server's range check (src/server.cpp:1071)."""
        if (self.temperature < 0 or self.top_p <= 0 or self.top_p > 1 or self.top_k < 0
                or self.repetition_penalty <= 0 or self.repeat_last_n < -1):
            raise ValueError("sampling parameter out of range")

    def is_greedy(self) -> bool:
        return np.float32(self.temperature) <= 0 or self.top_k == 1


def params_array(params) -> np.ndarray:
    """fs_row_params records from SamplerParams objects (or pass a PARAMS_DTYPE array through)."""
    if isinstance(params, np.ndarray) and params.dtype == PARAMS_DTYPE:
        return np.ascontiguousarray(params)
    if isinstance(params, SamplerParams):
        params = [params]
    out = np.zeros(len(params), PARAMS_DTYPE)
    for i, p in enumerate(params):
        out[i] = (p.temperature, p.top_k, p.top_p, p.min_p, p.repetition_penalty, p.frequency_penalty,
                  p.presence_penalty, p.repeat_last_n, p.penalty_from, p.softcap)
    return out


def _ptr(t):
    """Device pointer of a tensor the C ABI reads or writes as a packed array."""
    if t is None:
        return None
    if not t.is_contiguous():
        raise SamplerError("a non-contiguous tensor cannot be passed as a packed array")
    return ctypes.c_void_p(t.data_ptr())


def _lptr(t):
    """Device pointer of a logits matrix: rows may be strided (the C ABI takes the row stride ld), elements packed."""
    if t.dim() == 2 and t.shape[1] > 1 and t.stride(1) != 1:
        raise SamplerError("logits rows must be packed (stride 1 along the vocabulary)")
    return ctypes.c_void_p(t.data_ptr())


def _dev(x, dtype, device):
    """An input array or tensor as a packed device tensor of `dtype` (a strided view is copied, not misread)."""
    return torch.as_tensor(x, dtype=dtype, device=device).contiguous()


def _stream(stream=None):
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def _dev_params(params, device) -> torch.Tensor:
    if isinstance(params, torch.Tensor):
        if params.dtype != torch.uint8 or params.numel() % PARAMS_DTYPE.itemsize:
            raise SamplerError("params tensor must be uint8 bytes of fs_row_params records")
        return params.to(device).contiguous()
    a = params_array(params)
    return torch.from_numpy(a.view(np.uint8).copy()).to(device)


class Context:
    """An fs_context (device workspace); calls on one context are serialised by a lock."""

    _default = {}
    _dlock = threading.Lock()

    def __init__(self):
        h = ctypes.c_void_p()
        check(lib().fs_create(ctypes.byref(h)), "fs_create")
        self.h = h
        self.lock = threading.Lock()

    def __del__(self):
        h = getattr(self, "h", None)
        if h is not None and h.value:
            try:
                lib().fs_destroy(h)
            except Exception:
                pass

    def set_wait_limit(self, polls: int) -> None:
        """fs_set_wait_limit: the merge's bounded wait for a row's segments (0 = default)."""
        check(lib().fs_set_wait_limit(self.h, int(polls)), "fs_set_wait_limit")

    @classmethod
    def default(cls, device=None) -> "Context":
        dev = torch.device("cuda", torch.cuda.current_device() if device is None else torch.device(device).index or 0)
        with cls._dlock:
            if dev not in cls._default:
                cls._default[dev] = Context()
            return cls._default[dev]


class Rng:
    """fs_rng: libstdc++ std::mt19937_64 + generate_canonical, ferro::Sampler's draw stream (sampler.h:25,32)."""

    def __init__(self, seed: int = 0):
        h = ctypes.c_void_p()
        check(lib().fs_rng_create(ctypes.c_uint64(seed), ctypes.byref(h)), "fs_rng_create")
        self.h = h

    def __del__(self):
        h = getattr(self, "h", None)
        if h is not None and h.value:
            try:
                lib().fs_rng_destroy(h)
            except Exception:
                pass

    def next_u(self, n: int = 1) -> np.ndarray:
        out = np.zeros(n, np.float64)
        check(lib().fs_rng_next_u(self.h, out.ctypes.data_as(ctypes.c_void_p), n), "fs_rng_next_u")
        return out

    def copy(self) -> "Rng":
        r = Rng(1)
        check(lib().fs_rng_copy(self.h, r.h), "fs_rng_copy")
        return r


class DeviceRng:
    """fs_drng: one std::mt19937_64 draw stream per sampling stream, held on the device (ferro::Sampler's rng_,
    sampler.h:25,32). draw() gives each row of a sampling stream one generate_canonical draw, in row order; rows of
    greedy streams get 0 and consume nothing."""

    def __init__(self, seeds, device=None, stream=None):
        seeds = np.ascontiguousarray(np.asarray(seeds, dtype=np.uint64).reshape(-1))
        self.n = int(seeds.size)
        self._dev = torch.device("cuda" if device is None else device)
        h = ctypes.c_void_p()
        check(lib().fs_drng_create(self.n, seeds.ctypes.data_as(ctypes.c_void_p), _stream(stream),
                                   ctypes.byref(h)), "fs_drng_create")
        self.h = h

    def __del__(self):
        h = getattr(self, "h", None)
        if h is not None and h.value:
            try:
                lib().fs_drng_destroy(h)
            except Exception:
                pass

    def draw(self, params, row_off=None, peek=False, stream=None) -> torch.Tensor:
        p = _dev_params(params, self._dev)
        if p.numel() != self.n * PARAMS_DTYPE.itemsize:
            raise SamplerError("one params record per stream")
        ro = None
        rows = self.n
        if row_off is not None:
            ro = _dev(row_off, torch.int64, self._dev)
            if ro.numel() != self.n + 1:
                raise SamplerError("row_off must have n_streams+1 entries")
            rows = int(ro[-1].item())
        u = torch.empty(rows, dtype=torch.float64, device=self._dev)
        check(lib().fs_drng_draw(self.h, _ptr(ro), _ptr(p), _ptr(u), 1 if peek else 0, _stream(stream)),
              "fs_drng_draw")
        self._keep = (p, ro)
        return u

    def skip(self, counts, params, stream=None) -> None:
        p = _dev_params(params, self._dev)
        c = _dev(counts, torch.int32, self._dev)
        if c.numel() != self.n:
            raise SamplerError("one count per stream")
        check(lib().fs_drng_skip(self.h, _ptr(c), _ptr(p), _stream(stream)), "fs_drng_skip")
        self._keep = (p, c)

    def error(self, stream=None) -> int:
        bits = ctypes.c_int32(0)
        check(lib().fs_drng_error(self.h, _stream(stream), ctypes.byref(bits)), "fs_drng_error")
        return bits.value


def _check_logits(logits: torch.Tensor, V: int | None):
    if not (isinstance(logits, torch.Tensor) and logits.is_cuda and logits.dtype == torch.float32):
        raise SamplerError("logits must be a float32 CUDA tensor")
    if logits.dim() == 1:
        logits = logits.unsqueeze(0)
    if logits.dim() != 2:
        raise SamplerError("logits must be [B, V]")
    n = logits.shape[1] if V is None else V
    if n > logits.shape[1]:
        raise SamplerError("V exceeds the row length")
    ld = logits.stride(0) if logits.shape[0] > 1 else n + (-n) % 4
    if logits.stride(1) != 1 or ld % 4 or ld < n or logits.data_ptr() % 16:
        # the kernels take 16-byte aligned rows: repack into a padded copy
        padded = torch.zeros((logits.shape[0], n + (-n) % 4), dtype=torch.float32, device=logits.device)
        padded[:, :n] = logits[:, :n]
        logits, ld = padded, padded.stride(0)
    return logits, ld, n


def _hist_tensors(hist, hist_off, B, device):
    if hist is None:
        return None, None
    hist = _dev(hist, torch.int32, device)
    hist_off = _dev(hist_off, torch.int64, device)
    if hist_off.numel() != B + 1:
        raise SamplerError("hist_off must have B+1 entries")
    return hist, hist_off


# How sample_batch passes the parameters: "host" also hands the library their host copy (fs_sample_batch_hp, which
# picks the small-k kernel for batches it fits); "device" passes the device copy only (fs_sample_batch, the fused
# kernel for every batch). Tests run both.
ROUTE = "host"


def sample_batch(logits, params, u, hist=None, hist_off=None, V=None, kcap=0, ctx=None, stream=None, route=None):
    """fs_sample_batch(_hp) on device tensors: logits [B, ld] fp32 (rows 16-byte aligned), params (B records),
    u [B] float64 draws, hist/hist_off CSR histories. Returns dict(tok, keep, cand_ids, cand_probs) (device).
    route: "host" / "device" (default: the module's ROUTE); params given as a device tensor always go "device"."""
    logits, ld, n = _check_logits(logits, V)
    B = logits.shape[0]
    dev = logits.device
    p = _dev_params(params, dev)
    if p.numel() != B * PARAMS_DTYPE.itemsize:
        raise SamplerError("one params record per row")
    u = _dev(u, torch.float64, dev)
    hist, hist_off = _hist_tensors(hist, hist_off, B, dev)
    tok = torch.empty(B, dtype=torch.int32, device=dev)
    keep = torch.empty(B, dtype=torch.int32, device=dev)
    ids = torch.empty((B, kcap), dtype=torch.int32, device=dev) if kcap else None
    probs = torch.empty((B, kcap), dtype=torch.float64, device=dev) if kcap else None
    ctx = ctx or Context.default(dev)
    hp = None                                             # the host copy of the parameters picks the kernel
    if (route or ROUTE) == "host" and not isinstance(params, torch.Tensor):
        hp = params_array(params)
    with ctx.lock:
        if hp is not None:
            check(lib().fs_sample_batch_hp(ctx.h, _lptr(logits), ld, B, n, _ptr(hist), _ptr(hist_off), _ptr(p),
                                           hp.ctypes.data_as(ctypes.c_void_p), _ptr(u), _ptr(tok), kcap, _ptr(ids),
                                           _ptr(probs), _ptr(keep), _stream(stream)), "fs_sample_batch_hp")
        else:
            check(lib().fs_sample_batch(ctx.h, _lptr(logits), ld, B, n, _ptr(hist), _ptr(hist_off), _ptr(p),
                                        _ptr(u), _ptr(tok), kcap, _ptr(ids), _ptr(probs), _ptr(keep),
                                        _stream(stream)), "fs_sample_batch")
    return dict(tok=tok, keep=keep, cand_ids=ids, cand_probs=probs, _keepalive=(p, u, hist, hist_off))


def argmax_batch(logits, hist=None, hist_off=None, params=None, V=None, ctx=None, stream=None):
    """fs_argmax_batch: greedy token per row after the penalties of `params` (None = no penalty)."""
    logits, ld, n = _check_logits(logits, V)
    B = logits.shape[0]
    dev = logits.device
    p = _dev_params(params, dev) if params is not None else None
    hist, hist_off = _hist_tensors(hist, hist_off, B, dev)
    tok = torch.empty(B, dtype=torch.int32, device=dev)
    ctx = ctx or Context.default(dev)
    with ctx.lock:
        check(lib().fs_argmax_batch(ctx.h, _lptr(logits), ld, B, n, _ptr(hist), _ptr(hist_off), _ptr(p), _ptr(tok),
                                    _stream(stream)), "fs_argmax_batch")
    return tok


def verify(logits, rows, row_off, params, u=None, hist=None, hist_off=None, eos_id=-1, V=None, ctx=None,
           stream=None, route=None):
    """fs_verify(_hp): per-row tokens and per-stream accepted prefix lengths of a speculative window. route as for
    sample_batch ("host": the host copy of the stream parameters goes along, fs_verify_hp)."""
    logits, ld, n = _check_logits(logits, V)
    R = logits.shape[0]
    dev = logits.device
    rows = _dev(rows, torch.int32, dev)
    row_off = _dev(row_off, torch.int64, dev)
    S = row_off.numel() - 1
    p = _dev_params(params, dev)
    if p.numel() != S * PARAMS_DTYPE.itemsize:
        raise SamplerError("one params record per stream")
    u = _dev(np.zeros(R) if u is None else u, torch.float64, dev)
    hist, hist_off = _hist_tensors(hist, hist_off, S, dev)
    tok = torch.empty(R, dtype=torch.int32, device=dev)
    acc = torch.empty(S, dtype=torch.int32, device=dev)
    ctx = ctx or Context.default(dev)
    hp = None
    if (route or ROUTE) == "host" and not isinstance(params, torch.Tensor):
        hp = params_array(params)
    with ctx.lock:
        if hp is not None:
            check(lib().fs_verify_hp(ctx.h, _lptr(logits), ld, S, R, n, _ptr(rows), _ptr(row_off), _ptr(hist),
                                     _ptr(hist_off), _ptr(p), hp.ctypes.data_as(ctypes.c_void_p), _ptr(u),
                                     int(eos_id), _ptr(tok), _ptr(acc), _stream(stream)), "fs_verify_hp")
        else:
            check(lib().fs_verify(ctx.h, _lptr(logits), ld, S, R, n, _ptr(rows), _ptr(row_off), _ptr(hist),
                                  _ptr(hist_off), _ptr(p), _ptr(u), int(eos_id), _ptr(tok), _ptr(acc),
                                  _stream(stream)), "fs_verify")
    return tok, acc


def penalize_batch(logits, params, hist=None, hist_off=None, V=None, ctx=None, stream=None):
    """fs_penalize_batch: leave each row penalised in place, as ferro's sample() leaves its host row
    (sampler.cpp:11-18). logits must be a writable [B, ld] fp32 CUDA tensor; returns it."""
    target = logits
    logits, ld, n = _check_logits(logits, V)
    B = logits.shape[0]
    dev = logits.device
    p = _dev_params(params, dev)
    if p.numel() != B * PARAMS_DTYPE.itemsize:
        raise SamplerError("one params record per row")
    hist, hist_off = _hist_tensors(hist, hist_off, B, dev)
    ctx = ctx or Context.default(dev)
    with ctx.lock:
        check(lib().fs_penalize_batch(ctx.h, _lptr(logits), ld, B, n, _ptr(hist), _ptr(hist_off), _ptr(p),
                                      _stream(stream)), "fs_penalize_batch")
    t2 = target if target.dim() == 2 else target.unsqueeze(0)
    if logits.data_ptr() != t2.data_ptr():            # repacked into an aligned copy: write the rows back
        t2[:, :n].copy_(logits[:, :n])
    return target


def lookup_draft(hist, hist_off, kmax, min_n=None, eos_id=-1, draft_ld=None, ctx=None, stream=None):
    """fs_lookup_draft: prompt-lookup drafts per stream (server.cpp:552-564). Returns (draft [S, draft_ld], n [S])."""
    hist_off = _dev(hist_off, torch.int64, "cuda")
    S = hist_off.numel() - 1
    dev = hist_off.device
    hist = _dev(hist, torch.int32, dev)
    km = _dev(np.broadcast_to(np.asarray(kmax, np.int32), (S,)).copy(), torch.int32, dev)
    mn = None if min_n is None else _dev(np.broadcast_to(np.asarray(min_n, np.int32), (S,)).copy(), torch.int32, dev)
    ld = int(draft_ld if draft_ld is not None else max(int(km.max().item()) if S else 1, 1))
    draft = torch.zeros((S, ld), dtype=torch.int32, device=dev)
    nd = torch.zeros(S, dtype=torch.int32, device=dev)
    ctx = ctx or Context.default(dev)
    with ctx.lock:
        check(lib().fs_lookup_draft(ctx.h, S, _ptr(hist), _ptr(hist_off), _ptr(km), _ptr(mn), int(eos_id),
                                    _ptr(draft), ld, _ptr(nd), _stream(stream)), "fs_lookup_draft")
    return draft, nd


def hist_append(hist, hist_off, tok, row_off=None, count=None, out_cap=None, ctx=None, stream=None):
    """fs_hist_append: each stream's consumed tokens pushed onto its history (server.cpp:342), on device CSR
    histories, out of place. Stream s gains tok[row_off[s] : row_off[s] + count[s]] (row_off None: row s; count
    None: 1 per stream; fs_verify's tok / row_off / accepted fit as they are). Returns (out_hist, out_off): out_off
    [S+1] int64 rebased to 0; out_hist holds out_cap ids (default: room for every row of tok), of which
    out_off[-1] are used. Stays on the device: nothing here waits for the GPU."""
    hist_off = _dev(hist_off, torch.int64, "cuda")
    dev = hist_off.device
    S = hist_off.numel() - 1
    hist = _dev(hist, torch.int32, dev)
    if hist.numel() == 0:
        hist = torch.zeros(1, dtype=torch.int32, device=dev)     # every history empty: a valid pointer, never read
    tok = _dev(tok, torch.int32, dev)
    ro = None if row_off is None else _dev(row_off, torch.int64, dev)
    cnt = None if count is None else _dev(count, torch.int32, dev)
    if ro is not None and ro.numel() != S + 1:
        raise SamplerError(f"row_off has {ro.numel()} entries for {S} streams")
    if cnt is not None and cnt.numel() != S:
        raise SamplerError(f"count has {cnt.numel()} entries for {S} streams")
    if out_cap is None:
        out_cap = hist.numel() + tok.numel()
    out = torch.empty(max(int(out_cap), 1), dtype=torch.int32, device=dev)
    out_off = torch.empty(S + 1, dtype=torch.int64, device=dev)
    ctx = ctx or Context.default(dev)
    with ctx.lock:
        check(lib().fs_hist_append(ctx.h, S, _ptr(hist), _ptr(hist_off), _ptr(tok), _ptr(ro), _ptr(cnt), _ptr(out),
                                   int(out_cap), _ptr(out_off), _stream(stream)), "fs_hist_append")
    return out, out_off


def decode_step(logits, params, rng, hist=None, hist_off=None, out_cap=None, V=None, ctx=None, stream=None,
                route=None):
    """fs_decode_step(_hp): one decode step in one launch - each row's draw from its DeviceRng stream (row s = stream
    s), fs_sample_batch's token, and the token appended to the stream's history (server.cpp:603-606, then :342).
    Returns (tok, keep, out_hist, out_off); out_hist holds out_cap ids (default: room for one more per stream), of
    which out_off[-1] are used. Stays on the device. route as for sample_batch ("host": the host copy of the
    parameters goes along, fs_decode_step_hp)."""
    logits, ld, n = _check_logits(logits, V)
    B = logits.shape[0]
    dev = logits.device
    p = _dev_params(params, dev)
    if p.numel() != B * PARAMS_DTYPE.itemsize:
        raise SamplerError("one params record per row")
    if B > rng.n:
        raise SamplerError(f"{B} rows for {rng.n} draw streams")
    hist, hist_off = _hist_tensors(hist, hist_off, B, dev)
    if out_cap is None:
        out_cap = (hist.numel() if hist is not None else 0) + B
    tok = torch.empty(B, dtype=torch.int32, device=dev)
    keep = torch.empty(B, dtype=torch.int32, device=dev)
    out = torch.empty(max(int(out_cap), 1), dtype=torch.int32, device=dev)
    out_off = torch.empty(B + 1, dtype=torch.int64, device=dev)
    ctx = ctx or Context.default(dev)
    hp = params_array(params) if (route or ROUTE) == "host" and not isinstance(params, torch.Tensor) else None
    with ctx.lock:
        if hp is not None:
            check(lib().fs_decode_step_hp(ctx.h, rng.h, _lptr(logits), ld, B, n, _ptr(hist), _ptr(hist_off), _ptr(p),
                                          hp.ctypes.data_as(ctypes.c_void_p), _ptr(tok), _ptr(keep), _ptr(out),
                                          _ptr(out_off), int(out_cap), _stream(stream)), "fs_decode_step_hp")
        else:
            check(lib().fs_decode_step(ctx.h, rng.h, _lptr(logits), ld, B, n, _ptr(hist), _ptr(hist_off), _ptr(p),
                                       _ptr(tok), _ptr(keep), _ptr(out), _ptr(out_off), int(out_cap),
                                       _stream(stream)), "fs_decode_step")
    return tok, keep, out, out_off


def device_error(ctx=None, stream=None) -> int:
    ctx = ctx or Context.default()
    bits = ctypes.c_int32(0)
    check(lib().fs_device_error(ctx.h, _stream(stream), ctypes.byref(bits)), "fs_device_error")
    return bits.value


class Sampler:
    """Mirror of ferro::Sampler (src/sampler.h:23-34) running on the GPU.

    sample(logits, n_vocab, history) -> int, with logits a CUDA float32 tensor (device-resident, the intended
    use), a CPU tensor or a numpy float32 array (copied to the device). As in ferro (sampler.cpp:11-18) the row is
    left penalised in place, on whichever side it lives, unless the sampler was made with write_back=False (the
    token is the same either way: the kernels penalise on the fly)."""

    def __init__(self, p: SamplerParams, device=None, write_back: bool = True):
        self._p = p
        self._rng = Rng(int(p.seed))
        self._dev = torch.device("cuda" if device is None else device)
        self._rec = torch.from_numpy(params_array(p).view(np.uint8).copy()).to(self._dev)
        self._ctx = Context.default(self._dev)
        self._write_back = write_back

    def params(self) -> SamplerParams:
        return self._p

    def sample(self, logits, n_vocab: int, history) -> int:
        host = logits
        on_dev = isinstance(logits, torch.Tensor) and logits.is_cuda
        if not on_dev:
            logits = torch.as_tensor(np.asarray(logits, np.float32)).to(self._dev)
        row = logits.reshape(-1)[:n_vocab].reshape(1, -1)
        h = np.asarray(history, np.int32).reshape(-1)
        u = np.zeros(1) if self._p.is_greedy() else self._rng.next_u(1)
        hist_off = [0, h.size]
        out = sample_batch(row, self._rec, u, hist=h, hist_off=hist_off, V=n_vocab, ctx=self._ctx)
        tok = int(out["tok"].item())
        if self._write_back and h.size:
            penalize_batch(row, self._rec, hist=h, hist_off=hist_off, V=n_vocab, ctx=self._ctx)
            if not on_dev:
                pen = row.reshape(-1).cpu()
                if isinstance(host, torch.Tensor):
                    host.reshape(-1)[:n_vocab].copy_(pen)
                elif isinstance(host, np.ndarray) and host.dtype == np.float32:
                    host.reshape(-1)[:n_vocab] = pen.numpy()
        return tok
