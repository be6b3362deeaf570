"""Seeded synthetic inputs for the five measured configurations of the sampler path (host numpy arrays).

Shared by the GPU parity tests, the CPU oracle checks and bench.py, so every consumer sees identical inputs.
Conventions: "N(0, s)" is a normal with standard deviation s; Zipf(1.1) over ids 0..V-1 is P(id) ~ (id+1)^-1.1;
draws u are generate_canonical values of mt19937_64(seed_b)'s first output (the draw a fresh ferro
Sampler(seed_b) makes: src/sampler.h:25, sampler.cpp:45-46), so the reference itself can be run on the same rows.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from ._lib import PARAMS_DTYPE


# ----------------------------------------------------------------------------------------- mt19937_64 (std)
class MT19937_64:
    """std::mt19937_64 (Matsumoto & Nishimura's 64-bit Mersenne Twister, the standard's parameters)."""

    def __init__(self, seed: int):
        mt = [0] * 312
        mt[0] = seed & 0xFFFFFFFFFFFFFFFF
        for i in range(1, 312):
            mt[i] = (6364136223846793005 * (mt[i - 1] ^ (mt[i - 1] >> 62)) + i) & 0xFFFFFFFFFFFFFFFF
        self.mt, self.i = mt, 312

    def next(self) -> int:
        mt = self.mt
        if self.i >= 312:
            for k in range(312):
                x = (mt[k] & 0xFFFFFFFF80000000) | (mt[(k + 1) % 312] & 0x7FFFFFFF)
                mt[k] = mt[(k + 156) % 312] ^ (x >> 1) ^ (0xB5026F5AA96619E9 if x & 1 else 0)
            self.i = 0
        y = mt[self.i]
        self.i += 1
        y ^= (y >> 29) & 0x5555555555555555
        y ^= (y << 17) & 0x71D67FFFEDA60000
        y ^= (y << 37) & 0xFFF7EEE000000000
        y ^= y >> 43
        return y & 0xFFFFFFFFFFFFFFFF


def canonical(x: int) -> float:
    """generate_canonical<double,53> of one 64-bit output: x / 2^64 rounded to double, clamped below 1."""
    r = float(x) / 18446744073709551616.0
    return r if r < 1.0 else float(np.nextafter(1.0, 0.0))


def first_u(seed: int) -> float:
    return canonical(MT19937_64(seed).next())


# ----------------------------------------------------------------------------------------- pieces
def zipf_ids(rng: np.random.Generator, V: int, n: int, a: float = 1.1) -> np.ndarray:
    w = np.arange(1, V + 1, dtype=np.float64) ** (-a)
    cdf = np.cumsum(w)
    cdf /= cdf[-1]
    return np.minimum(np.searchsorted(cdf, rng.random(n), side="right"), V - 1).astype(np.int32)


def mixture_logits(rng: np.random.Generator, B: int, V: int) -> np.ndarray:
    """Per element: 90% N(0, 1.5), 10% Student-t(3) * 4 (configs 3 and 5)."""
    x = rng.standard_normal((B, V), dtype=np.float32) * np.float32(1.5)
    tail = rng.random((B, V)) < 0.1
    x[tail] = (rng.standard_t(3, size=int(tail.sum())) * 4.0).astype(np.float32)
    return x


def make_params(n, **kw) -> np.ndarray:
    p = np.zeros(n, PARAMS_DTYPE)
    defaults = dict(temperature=0.05, top_k=50, top_p=1.0, min_p=0.0, repetition_penalty=1.05,
                    frequency_penalty=0.0, presence_penalty=0.0, repeat_last_n=-1, penalty_from=0)
    defaults.update(kw)
    for k, v in defaults.items():
        p[k] = v
    return p


@dataclass
class Workload:
    name: str
    logits: np.ndarray            # [B, V] float32
    params: np.ndarray            # [B] (or [S] for verify) PARAMS_DTYPE
    hist: np.ndarray              # int32 CSR values
    hist_off: np.ndarray          # int64 CSR offsets
    u: np.ndarray                 # [B] float64
    seeds: np.ndarray             # [B] uint64: u[b] = first_u(seeds[b])
    rows: np.ndarray | None = None      # verify: token fed at each row
    row_off: np.ndarray | None = None   # verify: stream offsets
    meta: dict = field(default_factory=dict)

    @property
    def B(self):
        return self.logits.shape[0]

    @property
    def V(self):
        return self.logits.shape[1]

    def algorithmic_bytes(self) -> int:
        """One read of every logits row plus the history: 4V per row + 4H (per-call bytes of the roofline)."""
        return int(self.logits.nbytes + self.hist.nbytes)


def _seeds_u(seed: int, B: int):
    seeds = np.array([(seed * 1000003 + b + 1) & 0xFFFFFFFFFFFFFFFF for b in range(B)], np.uint64)
    return seeds, np.array([first_u(int(s)) for s in seeds], np.float64)


def _csr(hs):
    off = np.zeros(len(hs) + 1, np.int64)
    off[1:] = np.cumsum([len(h) for h in hs])
    return (np.concatenate(hs).astype(np.int32) if hs else np.zeros(0, np.int32)), off


# ----------------------------------------------------------------------------------------- configurations
def config1(seed: int = 1, V: int = 65536) -> Workload:
    """Single row, V=65536: N(0,2) + 8 spike tokens at +12; rep 1.1 over a 64-token uniform history; T 0.7,
    top-k 40, top-p 0.95."""
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((1, V), dtype=np.float32) * np.float32(2.0))
    spikes = rng.choice(V, 8, replace=False)
    x[0, spikes] += np.float32(12.0)
    h = rng.integers(0, V, 64).astype(np.int32)
    hist, off = _csr([h])
    p = make_params(1, temperature=0.7, top_k=40, top_p=0.95, repetition_penalty=1.1)
    seeds, u = _seeds_u(seed, 1)
    return Workload("cfg1_single_row", x, p, hist, off, u, seeds)


def config2(seed: int = 2, B: int = 8, V: int = 65536) -> Workload:
    """Greedy decode batch: N(0,2); frequency 0.5 / presence 0.3 over 256-token Zipf(1.1) histories; rep 1.0;
    T 0; 1% of rows (at least one) get an exact tie at the maximum."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((B, V), dtype=np.float32) * np.float32(2.0)
    hs = [zipf_ids(rng, V, 256) for _ in range(B)]
    ntie = max(1, int(round(0.01 * B)))
    tie_rows = rng.choice(B, ntie, replace=False)
    for b in tie_rows:
        free = np.setdiff1d(np.arange(V), hs[b])                 # unpenalised ids keep the tie exact
        i, j = np.sort(rng.choice(free, 2, replace=False))
        x[b, i] = x[b, j] = np.float32(x[b].max() + 1.0)
    hist, off = _csr(hs)
    p = make_params(B, temperature=0.0, top_k=50, repetition_penalty=1.0, frequency_penalty=0.5,
                    presence_penalty=0.3)
    seeds, u = _seeds_u(seed, B)
    return Workload("cfg2_greedy_freq_pres", x, p, hist, off, u, seeds, meta=dict(tie_rows=tie_rows))


def config3(seed: int = 3, B: int = 64, V: int = 262144) -> Workload:
    """Gemma-4-vocab serving batch (the headline): mixture logits; T 0.8, top-k 64, top-p 0.95, rep 1.05 over
    512-token Zipf histories; one draw per row."""
    rng = np.random.default_rng(seed)
    x = mixture_logits(rng, B, V)
    hist, off = _csr([zipf_ids(rng, V, 512) for _ in range(B)])
    p = make_params(B, temperature=0.8, top_k=64, top_p=0.95, repetition_penalty=1.05)
    seeds, u = _seeds_u(seed, B)
    return Workload("cfg3_gemma_serving", x, p, hist, off, u, seeds)


def config4(seed: int = 4, S: int = 16, M: int = 17, V: int = 65536, base_hist: int = 64) -> Workload:
    """Speculative verification: S streams x M rows (M-1 drafts + bonus), N(0,2), T 0, rep 1.0; the draft fed
    after row r equals row r's argmax with probability 0.8, else a uniform id."""
    rng = np.random.default_rng(seed)
    R = S * M
    x = rng.standard_normal((R, V), dtype=np.float32) * np.float32(2.0)
    am = x.argmax(axis=1)
    rows = np.zeros(R, np.int32)
    for s in range(S):
        rows[s * M] = rng.integers(0, V)
        for r in range(M - 1):
            rows[s * M + r + 1] = am[s * M + r] if rng.random() < 0.8 else rng.integers(0, V)
    row_off = np.arange(0, R + 1, M, dtype=np.int64)
    hist, off = _csr([rng.integers(0, V, base_hist).astype(np.int32) for _ in range(S)])
    p = make_params(S, temperature=0.0, top_k=50, repetition_penalty=1.0)
    seeds, u = _seeds_u(seed, R)
    return Workload("cfg4_spec_verify", x, p, hist, off, u, seeds, rows=rows, row_off=row_off)


def config5(seed: int = 5, B: int = 256, V: int = 262144, H: int = 1024) -> Workload:
    """Heterogeneous large batch: mixture logits; per row T ~ U[0.3,1.5] (5% at 0), top-k log-uniform in
    [1, 2048], top-p ~ U[0.8,1], repetition ~ U[1,1.3], frequency ~ U[0,1], presence ~ U[0,1] over 1024-token
    Zipf histories."""
    rng = np.random.default_rng(seed)
    x = mixture_logits(rng, B, V)
    hist, off = _csr([zipf_ids(rng, V, H) for _ in range(B)])
    T = rng.uniform(0.3, 1.5, B)
    T[rng.random(B) < 0.05] = 0.0
    k = np.floor(np.exp(rng.uniform(0.0, np.log(2048.0), B))).astype(np.int32).clip(1, 2048)
    p = make_params(B, temperature=T, top_k=k, top_p=rng.uniform(0.8, 1.0, B),
                    repetition_penalty=rng.uniform(1.0, 1.3, B), frequency_penalty=rng.uniform(0.0, 1.0, B),
                    presence_penalty=rng.uniform(0.0, 1.0, B))
    seeds, u = _seeds_u(seed, B)
    return Workload("cfg5_heterogeneous", x, p, hist, off, u, seeds)


CONFIGS = {1: config1, 2: config2, 3: config3, 4: config4, 5: config5}


def config3_all_tokens(seed: int = 3, B: int = 64, V: int = 262144) -> Workload:
    """cfg3's rows and parameters with top_k = 0: every token is a candidate (ferro's k = n, sampler.h:14,
    sampler.cpp:26-27), the whole-row path."""
    w = config3(seed, B, V)
    w.params["top_k"] = 0
    w.name = "cfg3_all_tokens"
    return w
