"""Comparison helpers for the GPU parity tests: GPU outputs vs the CPU oracle on identical inputs.

Bar (per the sampler's contract): integer outputs (argmax, top-k ids and order, accepted prefix) bit-exact;
probabilities within 1e-5 relative; sampled ids and kept-prefix lengths identical except where the oracle's
sequential sums put u*tot, top_p or the min-p threshold within 1e-6 of a boundary - such rows are counted.
"""
import numpy as np

PROB_RTOL = 1e-5
BOUNDARY = 1e-6


def boundary_row(probs, keep, u, top_p, min_p):
    """True if a sequential-vs-parallel summation difference could flip keep or the drawn index of this row."""
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


def compare(gpu, ora, params, u, kcap):
    """gpu / ora: dicts with tok, keep, cand_ids, cand_probs ([B, kcap]) and ora ncand. Returns #boundary rows;
    asserts everything else."""
    B = len(ora["tok"])
    nb = 0
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
        nb += int(at_edge)
    return nb
