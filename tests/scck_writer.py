"""Test fixture writer for scriptonait checkpoint files.

Restates crates/llm-core/src/checkpoint.rs:130-168 (write_checkpoint),
tokenizer.rs:348-358 (Tokenizer::to_bytes) and bf16.rs:10-20 (to_bf16),
so the tests can build files of any version and dtype; the reader under
test is the library's (scriptonait_amd.checkpoint).
"""
import struct

import numpy as np

BASE_VOCAB_SIZE = 264


def ffn_dim(h):  # config.rs:149-153
    return -(-(h * 8 // 3) // 32) * 32


def param_count(num_layers, hidden_dim, num_heads, num_kv_heads, vocab_size, use_ple=False):  # config.rs:245-264
    h, v, f = hidden_dim, vocab_size, ffn_dim(hidden_dim)
    kv = num_kv_heads * (hidden_dim // num_heads)
    per_layer = (v * h if use_ple else 0) + (h + 2 * h * h + 2 * kv * h) + (h + 3 * h * f)
    return v * h + num_layers * per_layer + h


def tokenizer_bytes(num_merges, seed=0):
    rs = np.random.default_rng(seed)
    out = bytearray(b"SCTK") + struct.pack("<II", 1, num_merges)
    for i in range(num_merges):
        limit = BASE_VOCAB_SIZE + i
        out += struct.pack("<II", int(rs.integers(0, limit)), int(rs.integers(0, limit)))
    return bytes(out)


def to_bf16(x: np.ndarray) -> np.ndarray:
    bits = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    lsb = (bits >> 16) & 1
    r = ((bits + 0x7FFF + lsb) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    r[nan] = ((bits[nan] >> 16) | 0x0040).astype(np.uint16)
    return r


def write(weights: np.ndarray, num_layers=2, hidden_dim=16, num_heads=4, num_kv_heads=2, context_len=32,
          local_window=16, vocab_size=300, rope_theta=50000.0, use_ple=False, step=4242, tokens_seen=9_000_000,
          planned_steps=23_000, plateau_scale=0.5, bf16=False, version=4, tokenizer=None) -> bytes:
    """A version-`version` file (the reference writes version 4; 2 and 3 drop
    the fields those versions lacked, as the reference's own tests do)."""
    tok = tokenizer if tokenizer is not None else tokenizer_bytes(vocab_size - BASE_VOCAB_SIZE)
    w = np.ascontiguousarray(weights, dtype=np.float32)
    blob = to_bf16(w).tobytes() if bf16 else w.tobytes()
    out = bytearray(b"SCCK") + struct.pack("<I", version)
    out += struct.pack("<7I", num_layers, hidden_dim, num_heads, num_kv_heads, context_len, local_window, vocab_size)
    out += struct.pack("<fI", rope_theta, int(use_ple))
    out += struct.pack("<Q", step)
    if version >= 3:
        out += struct.pack("<Q", tokens_seen)
    if version >= 4:
        out += struct.pack("<If", planned_steps, plateau_scale)
    out += struct.pack("<I", 1 if bf16 else 0)
    out += struct.pack("<I", len(tok)) + tok
    out += struct.pack("<I", len(blob)) + blob
    return bytes(out)


def sample_weights(vocab_size=300, hidden_dim=16, num_layers=2, num_heads=4, num_kv_heads=2, seed=5):
    n = param_count(num_layers, hidden_dim, num_heads, num_kv_heads, vocab_size)
    rs = np.random.default_rng(seed)
    return (0.02 * rs.standard_normal(n)).astype(np.float32)
