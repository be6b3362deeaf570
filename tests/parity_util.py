"""Comparison helpers for the GPU parity tests: GPU outputs vs the CPU oracle on identical inputs.

Bar (per the sampler's contract): integer outputs (argmax, top-k ids and order, accepted prefix) bit-exact;
probabilities within 1e-5 relative; sampled ids and kept-prefix lengths identical except where the oracle's
sequential sums put u*tot, top_p or the min-p threshold within 1e-6 of a boundary - such rows are counted.
"""
import numpy as np

from oracle import oracle as O

PROB_RTOL = 1e-5
BOUNDARY = O.BOUNDARY


boundary_row = O.near_boundary


def bf16_valued(x):
    """fp32 logits rounded to bfloat16 (round to nearest even) and widened back: what a model that emits bf16 logits
    hands the sampler. A V=262144 row then holds only a few thousand distinct values, so equal logits meet at every
    top-k boundary and top-p crossing (ties go to the lowest id)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


class Parity(int):
    """Rows of a comparison whose draw lies near a cumulative boundary (the int value), with .diverged: the rows
    among them whose token or kept count actually differs from the oracle's."""

    def __new__(cls, near, diverged):
        obj = super().__new__(cls, near)
        obj.diverged = diverged
        return obj


def compare(gpu, ora, params, u, kcap):
    """gpu / ora: dicts with tok, keep, cand_ids, cand_probs ([B, kcap]) and ora ncand. Returns a Parity: the rows
    near a boundary and, of those, the ones that differ; asserts everything else."""
    B = len(ora["tok"])
    nb = 0
    nd = 0
    for b in range(B):
        p = params[b]
        m = min(int(ora["ncand"][b]), kcap)
        np.testing.assert_array_equal(gpu["cand_ids"][b, :m], ora["cand_ids"][b, :m], err_msg=f"row {b} top-k ids")
        np.testing.assert_allclose(gpu["cand_probs"][b, :m], ora["cand_probs"][b, :m], rtol=PROB_RTOL, atol=0,
                                   err_msg=f"row {b} probs")
        greedy = p["temperature"] <= 0 or p["top_k"] == 1
        if greedy:
            assert gpu["tok"][b] == ora["tok"][b], f"row {b} greedy token"
            continue
        full = int(ora["ncand"][b]) <= kcap
        at_edge = full and boundary_row(ora["cand_probs"][b, :int(ora["ncand"][b])], int(ora["keep"][b]), u[b],
                                        float(p["top_p"]), float(p["min_p"]))
        if gpu["tok"][b] != ora["tok"][b] or gpu["keep"][b] != ora["keep"][b]:
            assert at_edge, f"row {b}: tok {gpu['tok'][b]} vs {ora['tok'][b]}, keep {gpu['keep'][b]} vs " \
                            f"{ora['keep'][b]} away from any boundary"
            nd += 1
        nb += int(at_edge)
    return Parity(nb, nd)


def oracle_decode_loop(rows_per_step, params, seeds, hist0):
    """Each step samples every stream's row with the stream's current history (oracle sampler, the stream's own
    mt19937_64 draws; greedy rows draw nothing, sampler.cpp:19-23), then appends the tokens with O.hist_append."""
    S = len(seeds)
    engines = [O.MT64(int(sd)) for sd in seeds]
    hist = np.concatenate([np.asarray(h, np.int32) for h in hist0]) if S else np.zeros(0, np.int32)
    off = np.concatenate([[0], np.cumsum([len(h) for h in hist0])]).astype(np.int64)
    toks = []
    for x in rows_per_step:
        t = np.zeros(S, np.int32)
        for s in range(S):
            p = params[s]
            greedy = p["temperature"] <= 0 or p["top_k"] == 1
            u = 0.0 if greedy else O.canonical(engines[s].next())
            t[s] = O.sample(x[s], hist[off[s]:off[s + 1]], p, u)[0]
        hist, off = O.hist_append(hist, off, t)
        toks.append(t)
    return np.stack(toks), hist, off
