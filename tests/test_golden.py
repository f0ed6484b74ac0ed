"""Committed golden cases (tests/golden/sampler_cases.npz, written by
tests/golden/make_golden.py): the CPU oracle must keep reproducing them, and
the GPU library must reproduce them bit for bit (ids, RNG state, kept count,
post-truncation probabilities)."""
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle

FIX = Path(__file__).resolve().parent / "golden" / "sampler_cases.npz"
_data = np.load(FIX, allow_pickle=False)
N = int(_data["count"][0])


def case(i):
    p = f"c{i}_"
    allowed = _data[p + "allowed"] if bool(_data[p + "has_allowed"][0]) else None
    h = _data[p + "hist"]
    offs = np.array([0, h.size], dtype=np.uint32)
    return dict(logits=_data[p + "logits"][None, :], params=_data[p + "params"],
                seed=_data[p + "seed"], hist=h if h.size else None, offs=offs if h.size else None,
                allowed=allowed, id=int(_data[p + "id"][0]), state=int(_data[p + "state"][0]),
                kept=int(_data[p + "kept"][0]), probs=_data[p + "probs"])


@pytest.mark.parametrize("i", range(N))
def test_oracle_reproduces_golden(i):
    c = case(i)
    r = oracle.sample_batch(c["logits"], c["params"], c["seed"], c["hist"], c["offs"],
                            allowed=c["allowed"], want_probs=True)
    assert int(r.ids[0]) == c["id"]
    assert int(r.rng_state[0]) == c["state"]
    assert int(r.kept[0]) == c["kept"]
    assert np.array_equal(r.probs[0], c["probs"])


@pytest.mark.gpu
def test_gpu_reproduces_golden(sampler):
    for i in range(N):
        c = case(i)
        g = sampler.sample_host(c["logits"], c["params"], c["seed"], c["hist"], c["offs"],
                                allowed=c["allowed"], want_probs=True)
        assert int(g.ids[0]) == c["id"], f"case {i}"
        assert int(g.rng_state[0]) == c["state"], f"case {i}"
        assert int(g.kept[0]) == c["kept"], f"case {i}"
        nz = c["probs"] != 0
        assert np.array_equal(g.probs[0] != 0, nz), f"case {i}"
        assert np.array_equal(g.probs[0][nz], c["probs"][nz]), f"case {i}"
