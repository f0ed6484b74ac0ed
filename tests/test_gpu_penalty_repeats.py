"""GPU parity for histories that repeat a row's own top candidates many times.

generate.rs:343-352 applies the repetition penalty once per occurrence, each
step rounded. The register path stops a candidate's penalty loop as soon as
the value falls below the selection threshold (or, for greedy rows, below the
largest value no penalty touches), which is exact for rp >= 1 because every
step can only lower the value. These rows exercise both sides of that: at
rp = 1.2 the loop stops after a few steps, at rp = 1.0001 a candidate repeated
5000 times stays above the threshold and the loop runs to the end. Ids, kept
counts and RNG states must equal the oracle's.
"""
import numpy as np
import pytest

from parity_util import compare, run_both
from scriptonait_amd.workloads import make_params, make_workload

pytestmark = pytest.mark.gpu


def _history_of_top_ids(logits: np.ndarray, reps: int, seed: int):
    """Per row: its largest logit's id `reps` times, its next three ids 3 times
    each, and 200 uniform ids, shuffled (the penalty does not depend on the
    order)."""
    rs = np.random.default_rng(seed)
    B, V = logits.shape
    rows = []
    for b in range(B):
        order = np.argsort(-logits[b], kind="stable")
        h = np.concatenate([np.full(reps, order[0]), np.repeat(order[1:4], 3),
                            rs.integers(0, V, size=200)]).astype(np.uint32)
        rs.shuffle(h)
        rows.append(h)
    offs = np.zeros(B + 1, dtype=np.uint32)
    offs[1:] = np.cumsum([len(h) for h in rows])
    return np.concatenate(rows), offs


@pytest.mark.parametrize("reps", [48, 5000])
@pytest.mark.parametrize("rp", [1.2, 1.0001])
@pytest.mark.parametrize("temperature", [1.0, 0.0])
def test_history_repeating_the_top_candidate(sampler, reps, rp, temperature):
    w = make_workload(2, B=16)  # V = 8192: the register path
    w.hist, w.hist_offsets = _history_of_top_ids(w.logits, reps, seed=reps)
    prm = make_params(temperature, 50, 0.9, 0.1, rp)
    g, o = run_both(sampler, w, params=prm)
    s = compare(g, o, f"reps={reps} rp={rp} T={temperature}")
    assert s["mismatches"] == 0, s
    if temperature == 0.0:
        assert np.array_equal(g.rng_state, w.rng_seeds), "greedy rows must not advance the RNG"


def test_repeated_top_ids_at_the_headline_shape(sampler):
    """Config 3's shape and filters, every row's history holding its own top
    id 48 times: the candidates the penalty pushes below the threshold stop
    early, the others are exact."""
    w = make_workload(3, B=64)
    w.hist, w.hist_offsets = _history_of_top_ids(w.logits, 48, seed=3)
    g, o = run_both(sampler, w)
    s = compare(g, o, "config3 shape, top id x48")
    assert s["mismatches"] == 0, s
