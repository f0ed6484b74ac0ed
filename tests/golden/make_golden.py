"""Writes tests/golden/sampler_cases.npz: small sampler cases with their
expected outputs.

Expected outputs come from the C++ oracle and are checked, case by case,
against the independent pure-Python restatement (tests/pyref.py) before
being written; a case where the two disagree aborts the script. The cases
cover the reference's own sampler tests
(crates/llm-core/src/generate.rs:550-692) plus edge cases: ties, masks,
penalties with repeats and out-of-range ids, greedy rows, top_k >= V,
min_p > 1, top_p <= 0, all-masked rows and empty histories.

Run from the repository root: python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))

from oracle import oracle  # noqa: E402
from pyref import PyRng, sample_with as py_sample_with  # noqa: E402
from scriptonait_amd.workloads import make_params  # noqa: E402

OUT = Path(__file__).resolve().parent / "sampler_cases.npz"


def cases():
    yield dict(x=[0.0, 5.0, 0.0, 9.0, 0.0], T=5.0, k=2, p=1.0, mp=0.0, rp=1.0, h=[], seed=3)
    yield dict(x=[20.0, 0.0, 0.0, 0.0], T=1.0, k=0, p=0.9, mp=0.0, rp=1.0, h=[], seed=11)
    yield dict(x=[2.0, 1.9, 0.0], T=0.0, k=40, p=0.95, mp=0.0, rp=1.5, h=[0], seed=1)
    yield dict(x=[6.0] + [0.0] * 7, T=1.0, k=0, p=1.0, mp=0.1, rp=1.0, h=[], seed=1)
    yield dict(x=[0.10, 0.05, 0.0, -0.05, -0.10], T=1.0, k=0, p=1.0, mp=0.1, rp=1.0, h=[], seed=2)
    yield dict(x=[1.0, 0.9, 0.8], T=1.0, k=0, p=1.0, mp=5.0, rp=1.0, h=[], seed=3)
    yield dict(x=[1.0, 0.9, 0.8], T=1.0, k=0, p=0.0, mp=0.0, rp=1.0, h=[], seed=4)
    yield dict(x=[-np.inf] * 6, T=1.0, k=3, p=0.9, mp=0.0, rp=1.1, h=[1], seed=5)
    yield dict(x=[0.0] * 37, T=1.0, k=5, p=1.0, mp=0.0, rp=1.0, h=[], seed=6)
    yield dict(x=[-0.0, 0.0, -0.0, 0.0], T=1.0, k=3, p=1.0, mp=0.0, rp=1.0, h=[], seed=7)
    rs = np.random.default_rng(20240601)
    for i in range(48):
        V = int(rs.choice([3, 17, 64, 100, 257, 511]))
        x = (rs.normal(size=V) * rs.choice([0.5, 2.0, 5.0])).astype(np.float32)
        if i % 4 == 0:
            x = np.round(x * 4) / 4
        T = float(rs.choice([0.0, 0.25, 0.7, 1.0, 1.7]))
        k = int(rs.choice([0, 1, 5, 40, 64, V, V + 3]))
        p = float(rs.choice([1.0, 0.95, 0.9, 0.3]))
        mp = float(rs.choice([0.0, 0.02, 0.05, 0.2]))
        rp = float(rs.choice([1.0, 1.1, 1.3, 0.9]))
        h = rs.integers(0, V + 2, size=int(rs.integers(0, 3 * V))).tolist()
        allowed = None
        if i % 6 == 1:
            allowed = (rs.random(max(1, V - 2)) > 0.4).astype(np.uint8).tolist()
        yield dict(x=x.tolist(), T=T, k=k, p=p, mp=mp, rp=rp, h=h, seed=int(rs.integers(0, 1 << 63)),
                   allowed=allowed)


def main():
    arrays = {}
    n = 0
    for i, c in enumerate(cases()):
        x = np.asarray(c["x"], dtype=np.float32)
        h = np.asarray(c["h"], dtype=np.uint32)
        allowed = None if c.get("allowed") is None else np.asarray(c["allowed"], dtype=np.uint8)
        prm = make_params(c["T"], c["k"], c["p"], c["mp"], c["rp"])
        offs = np.array([0, h.size], dtype=np.uint32)
        r = oracle.sample_batch(x[None, :], prm, np.array([c["seed"]], dtype=np.uint64),
                                h if h.size else None, offs if h.size else None, allowed=allowed,
                                want_probs=True)
        want, kept = py_sample_with(x, c["T"], c["k"], c["p"], c["mp"], c["rp"], c["h"],
                                    PyRng(c["seed"]), allowed=allowed)
        assert int(r.ids[0]) == want, (i, int(r.ids[0]), want)
        for kid, pv in kept.items():
            assert r.probs[0, kid] == np.float32(pv), (i, kid)
        p = f"c{i}_"
        arrays[p + "logits"] = x
        arrays[p + "params"] = prm
        arrays[p + "hist"] = h
        arrays[p + "allowed"] = allowed if allowed is not None else np.zeros(0, dtype=np.uint8)
        arrays[p + "has_allowed"] = np.array([allowed is not None])
        arrays[p + "seed"] = np.array([c["seed"]], dtype=np.uint64)
        arrays[p + "id"] = r.ids.copy()
        arrays[p + "state"] = r.rng_state.copy()
        arrays[p + "kept"] = r.kept.copy()
        arrays[p + "probs"] = r.probs[0].copy()
        n += 1
    arrays["count"] = np.array([n])
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {n} cases to {OUT}")


if __name__ == "__main__":
    main()
