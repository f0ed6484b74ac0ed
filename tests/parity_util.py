"""Comparison of GPU sampler results with the CPU oracle (test helper)."""
from __future__ import annotations

import numpy as np

from oracle import oracle

# ids bit-exact except rows whose truncation
# boundary or draw falls within 1e-6 of a cumulative-probability edge;
# post-truncation probabilities within 1e-5 relative (fp32).
TIE_MARGIN = 1e-6
PROB_RTOL = 1e-5


def compare(gpu, orc, label: str, probs: bool = True) -> dict:
    """Assert GPU == oracle under the tolerance rules; return a summary."""
    B = gpu.ids.size
    mism = np.nonzero(gpu.ids != orc.ids)[0]
    unexplained = [int(b) for b in mism if not (orc.margin[b] < TIE_MARGIN)]
    assert not unexplained, (
        f"{label}: {len(unexplained)} id mismatches not explained by a <1e-6 tie, "
        f"rows {unexplained[:10]} gpu={gpu.ids[unexplained[:10]]} oracle={orc.ids[unexplained[:10]]} "
        f"kept gpu={gpu.kept[unexplained[:10]] if gpu.kept is not None else None} "
        f"oracle={orc.kept[unexplained[:10]]}")
    ok_rows = np.ones(B, dtype=bool)
    ok_rows[mism] = False
    # RNG advance: exactly one step per drawn row, identical to the oracle.
    assert np.array_equal(gpu.rng_state[ok_rows], orc.rng_state[ok_rows]), f"{label}: rng state differs"
    if gpu.kept is not None:
        bad = np.nonzero((gpu.kept != orc.kept) & ok_rows)[0]
        assert bad.size == 0, f"{label}: kept differs at rows {bad[:10]} gpu={gpu.kept[bad[:10]]} oracle={orc.kept[bad[:10]]}"
    max_rel = 0.0
    if probs and gpu.probs is not None and orc.probs is not None:
        g, o = gpu.probs[ok_rows], orc.probs[ok_rows]
        assert np.array_equal(g != 0, o != 0), f"{label}: kept sets differ"
        nz = o != 0
        if nz.any():
            rel = np.abs(g[nz] - o[nz]) / np.abs(o[nz])
            max_rel = float(rel.max())
            assert max_rel <= PROB_RTOL, f"{label}: prob rel err {max_rel}"
    return {"rows": B, "mismatches": int(mism.size), "ties": int(mism.size), "max_prob_rel": max_rel}


def run_both(sampler, w, want_probs=True, threads=8, params=None, allowed=None):
    params = w.params if params is None else params
    g = sampler.sample_host(w.logits, params, w.rng_seeds, w.hist, w.hist_offsets, allowed=allowed,
                            V=w.V, want_probs=want_probs)
    o = oracle.sample_batch(w.logits, params, w.rng_seeds, w.hist, w.hist_offsets, allowed=allowed,
                            V=w.V, want_probs=want_probs, threads=threads)
    return g, o
