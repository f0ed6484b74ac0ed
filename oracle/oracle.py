"""ctypes loader of the CPU oracle (liboracle_sampler.so).

TEST INFRASTRUCTURE ONLY. Imported by tests/, by __graft_entry__.smoke() and
by bench.py's cpu_baseline leg, always as the checker or the timed CPU
baseline, never as the product path. The oracle restates
crates/llm-core/src/generate.rs:325-420, rng.rs:11-34 and
ops/linear.rs:19-32, 110-125 in C++ (sampler_oracle.cpp).
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path
from typing import Optional

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle_sampler.so"
_lib: Optional[ctypes.CDLL] = None

PARAMS_DTYPE = np.dtype(
    [
        ("temperature", "<f4"),
        ("top_k", "<u4"),
        ("top_p", "<f4"),
        ("min_p", "<f4"),
        ("repetition_penalty", "<f4"),
    ]
)


def build() -> Path:
    subprocess.run(["make", "-s", "-B", "-C", str(HERE)], check=True)
    return LIB_PATH


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        build()
    lib = ctypes.CDLL(str(LIB_PATH))
    vp, sz, u32 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint32
    lib.oracle_splitmix64_next.restype = ctypes.c_uint64
    lib.oracle_splitmix64_next.argtypes = [vp]
    lib.oracle_next_f32.restype = ctypes.c_float
    lib.oracle_next_f32.argtypes = [vp]
    lib.oracle_argmax.restype = u32
    lib.oracle_argmax.argtypes = [vp, sz]
    lib.oracle_linear_fwd.restype = None
    lib.oracle_linear_fwd.argtypes = [vp, vp, sz, sz, sz, vp, ctypes.c_int]
    lib.oracle_sample_batch.restype = ctypes.c_int
    lib.oracle_sample_batch.argtypes = [vp, sz, sz, sz, vp, sz, vp, vp, vp, sz, u32, vp, vp, vp, vp,
                                        vp, ctypes.c_int]
    _lib = lib
    return lib


def _ptr(a):
    return None if a is None else a.ctypes.data


def linear_fwd(x: np.ndarray, w: np.ndarray, threads: int = 1) -> np.ndarray:
    """crates/llm-core/src/ops/linear.rs:110-125: y = x @ w^T in the
    reference's dot order (x [rows, in_dim], w [out_dim, in_dim], f32)."""
    lib = load()
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    if x.ndim == 1:
        x = x[None, :]
    rows, in_dim = x.shape
    out_dim = w.shape[0]
    assert w.shape[1] == in_dim
    y = np.zeros((rows, out_dim), dtype=np.float32)
    lib.oracle_linear_fwd(x.ctypes.data, w.ctypes.data, rows, in_dim, out_dim, y.ctypes.data, threads)
    return y


class OracleResult:
    def __init__(self, ids, rng_state, kept, probs, margin):
        self.ids, self.rng_state, self.kept, self.probs, self.margin = ids, rng_state, kept, probs, margin


def sample_batch(logits: np.ndarray, params: np.ndarray, rng_state: np.ndarray,
                 hist: Optional[np.ndarray] = None, hist_offsets: Optional[np.ndarray] = None,
                 allowed: Optional[np.ndarray] = None, eos_id: int = 258, V: Optional[int] = None,
                 want_probs: bool = False, threads: int = 1, rows: Optional[slice] = None) -> OracleResult:
    """Batched sample_with on the CPU, same argument meaning as the C ABI."""
    lib = load()
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    if logits.ndim == 1:
        logits = logits[None, :]
    B, ld = logits.shape
    V = ld if V is None else V
    params = np.ascontiguousarray(params, dtype=PARAMS_DTYPE)
    stride = 0 if params.shape[0] == 1 else 1
    st = np.ascontiguousarray(rng_state, dtype=np.uint64).copy()
    ids = np.zeros(B, dtype=np.uint32)
    kept = np.zeros(B, dtype=np.uint32)
    margin = np.zeros(B, dtype=np.float32)
    probs = np.zeros((B, V), dtype=np.float32) if want_probs else None
    if hist is not None:
        hist = np.ascontiguousarray(hist, dtype=np.uint32)
        hist_offsets = np.ascontiguousarray(hist_offsets, dtype=np.uint32)
    if allowed is not None:
        allowed = np.ascontiguousarray(allowed, dtype=np.uint8)
    rc = lib.oracle_sample_batch(_ptr(logits), B, V, ld, _ptr(params), stride, _ptr(hist),
                                 _ptr(hist_offsets), _ptr(allowed),
                                 0 if allowed is None else allowed.size, eos_id, _ptr(st),
                                 _ptr(ids), _ptr(probs), _ptr(kept), _ptr(margin), threads)
    if rc != 0:
        raise ValueError(f"oracle_sample_batch failed: {rc}")
    return OracleResult(ids, st, kept, probs, margin)


def splitmix64_next(state: int) -> tuple[int, int]:
    """One rng.rs next_u64 step: returns (output, new_state)."""
    s = np.array([state], dtype=np.uint64)
    out = load().oracle_splitmix64_next(_ptr(s))
    return int(out), int(s[0])


def next_f32(state: int) -> tuple[float, int]:
    s = np.array([state], dtype=np.uint64)
    out = load().oracle_next_f32(_ptr(s))
    return float(out), int(s[0])


def seen_tokens(tokens, V: int) -> np.ndarray:
    """crates/llm-core/src/corpus.rs:236-247 (Corpus::seen_tokens): one flag per
    id < V, set when some token equals it; ids >= V are skipped, as
    seen.get_mut(id) returns None for them. `tokens` is the concatenation of
    the corpus's token lists (the order does not matter)."""
    seen = np.zeros(V, dtype=bool)
    t = np.asarray(tokens, dtype=np.uint64).ravel()
    seen[t[t < V].astype(np.int64)] = True
    return seen


def pack_bits(mask) -> np.ndarray:
    """A bool mask as the C ABI's bit mask: bit i % 32 of u32 word i / 32."""
    m = np.asarray(mask, dtype=bool).ravel()
    words = (m.size + 31) // 32
    padded = np.zeros(words * 32, dtype=bool)
    padded[: m.size] = m
    return np.packbits(padded, bitorder="little").view("<u4").astype(np.uint32)


def unpack_bits(words, n: int) -> np.ndarray:
    """Inverse of pack_bits for the first n ids."""
    w = np.ascontiguousarray(words, dtype="<u4")
    return np.unpackbits(w.view(np.uint8), bitorder="little")[:n].astype(bool)
