"""Independent pure-Python restatement of the reference sampler (test helper).

A second, separately written implementation of
crates/llm-core/src/generate.rs:325-420 and crates/llm-core/src/rng.rs:6-34,
used only to cross-check the C++ oracle on small rows: both must agree bit
for bit, so a slip in either (a dropped term, a wrong comparison, an
off-by-one in a truncation) shows up as a disagreement. Every f32 operation
is done on numpy.float32 scalars (IEEE binary32, round to nearest); exp is
the C library's expf, called through ctypes, which is what Rust's f32::exp
links to on x86_64 Linux.
"""
from __future__ import annotations

import ctypes
import ctypes.util
import math

import numpy as np

f32 = np.float32
_libm = ctypes.CDLL(ctypes.util.find_library("m") or "libm.so.6")
_libm.expf.restype = ctypes.c_float
_libm.expf.argtypes = [ctypes.c_float]
MASK64 = (1 << 64) - 1


def expf(x: np.float32) -> np.float32:
    return f32(_libm.expf(float(x)))


class PyRng:
    """rng.rs:6-34."""

    def __init__(self, seed: int):
        self.state = seed & MASK64

    def next_u64(self) -> int:
        self.state = (self.state + 0x9E3779B97F4A7C15) & MASK64
        z = self.state
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK64
        return z ^ (z >> 31)

    def next_f32(self) -> np.float32:
        return f32(self.next_u64() >> 40) / f32(1 << 24)


def argmax(row) -> int:
    """ops/loss.rs:6-16."""
    best, best_val = 0, f32(-np.inf)
    for i, v in enumerate(row):
        if v > best_val:
            best_val, best = v, i
    return best


def sample_with(logits, temperature, top_k, top_p, min_p, rep, recent, rng: PyRng,
                allowed=None, eos=258):
    """generate.rs:325-420. Returns (id, kept probabilities as {id: p})."""
    with np.errstate(all="ignore"):
        work = [f32(v) for v in logits]
        if allowed is not None:
            for i in range(len(work)):
                if i != eos and i < len(allowed) and not allowed[i]:
                    work[i] = f32(-np.inf)
        rp = f32(rep)
        if rp != f32(1.0):
            for i in recent:
                if i < len(work):
                    work[i] = work[i] / rp if work[i] > f32(0) else work[i] * rp
        T = f32(temperature)
        if T <= f32(0):
            return argmax(work), {}
        work = [w / T for w in work]
        order = sorted(range(len(work)), key=lambda i: (-float(work[i]), i))
        if top_k > 0:
            order = order[:top_k]
        mx = f32(-np.inf)
        for i in order:
            mx = max(mx, work[i])
        probs = [expf(work[i] - mx) for i in order]
        s = f32(0)
        for p in probs:
            s = s + p
        if not (s > f32(0)) or not math.isfinite(float(s)):
            return (order[0] if order else 0), {}
        probs = [p / s for p in probs]
        if f32(min_p) > f32(0):
            thr = f32(min_p) * (probs[0] if probs else f32(0))
            keep = 0
            while keep < len(probs) and probs[keep] >= thr:
                keep += 1
            keep = max(keep, 1)
            probs, order = probs[:keep], order[:keep]
        if f32(top_p) < f32(1):
            c, keep = f32(0), len(probs)
            for i, p in enumerate(probs):
                c = c + p
                if c >= f32(top_p):
                    keep = i + 1
                    break
            probs, order = probs[:keep], order[:keep]
        total = f32(0)
        for p in probs:
            total = total + p
        r = rng.next_f32() * total
        kept = {order[i]: probs[i] for i in range(len(order))}
        for i, p in enumerate(probs):
            if r < p:
                return order[i], kept
            r = r - p
        return (order[-1] if order else 0), kept
