"""Python mirror of scriptonait's checkpoint reader over the library's
llmhip_scck_* entry points (host code, no GPU needed).

Mirrors crates/llm-core/src/checkpoint.rs: `Checkpoint.from_bytes` accepts
exactly the files `Checkpoint::from_bytes` (checkpoint.rs:192-262) accepts
and raises ValueError with the reason otherwise. The weights are not built
into a model (the forward pass is not part of this library); parameters are
widened to f32 on request, so the tied head's embedding table (`embed()`,
the first vocab_size * hidden_dim parameters, model.rs:75-82) can feed
llmhip_sample_tied_head_device.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from .sampler import load_library

BASE_VOCAB_SIZE = 264  # crates/llm-core/src/tokenizer.rs:49-52


class LlmhipScckInfo(ctypes.Structure):
    _fields_ = [
        ("version", ctypes.c_uint32),
        ("num_layers", ctypes.c_uint32),
        ("hidden_dim", ctypes.c_uint32),
        ("num_heads", ctypes.c_uint32),
        ("num_kv_heads", ctypes.c_uint32),
        ("context_len", ctypes.c_uint32),
        ("local_window", ctypes.c_uint32),
        ("vocab_size", ctypes.c_uint32),
        ("rope_theta", ctypes.c_float),
        ("use_ple", ctypes.c_uint32),
        ("step", ctypes.c_uint64),
        ("tokens_seen", ctypes.c_uint64),
        ("planned_steps", ctypes.c_uint32),
        ("plateau_scale", ctypes.c_float),
        ("weight_dtype", ctypes.c_uint32),
        ("num_merges", ctypes.c_uint32),
        ("tokenizer_offset", ctypes.c_uint64),
        ("tokenizer_bytes", ctypes.c_uint64),
        ("weights_offset", ctypes.c_uint64),
        ("weights_bytes", ctypes.c_uint64),
        ("param_count", ctypes.c_uint64),
    ]


def _lib():
    lib = load_library()
    if not getattr(lib, "_scck_bound", False):
        vp, sz, u64 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint64
        lib.llmhip_scck_parse.restype = ctypes.c_int
        lib.llmhip_scck_parse.argtypes = [vp, sz, ctypes.POINTER(LlmhipScckInfo)]
        lib.llmhip_scck_read_params.restype = ctypes.c_int
        lib.llmhip_scck_read_params.argtypes = [vp, sz, ctypes.POINTER(LlmhipScckInfo), u64, u64, vp]
        lib._scck_bound = True
    return lib


@dataclass
class ModelConfig:
    """The shape fields of crates/llm-core/src/config.rs's ModelConfig."""

    num_layers: int
    hidden_dim: int
    num_heads: int
    num_kv_heads: int
    context_len: int
    local_window: int
    vocab_size: int
    rope_theta: float
    use_ple: bool


class Checkpoint:
    """checkpoint.rs:86-117: config, step, tokens_seen, planned_steps,
    plateau_scale; the tokenizer's merge count; the weights on request."""

    def __init__(self, data: bytes, info: LlmhipScckInfo):
        self._data = data
        self._buf = np.frombuffer(data, dtype=np.uint8)
        self.info = info
        self.config = ModelConfig(info.num_layers, info.hidden_dim, info.num_heads, info.num_kv_heads,
                                  info.context_len, info.local_window, info.vocab_size, float(info.rope_theta),
                                  bool(info.use_ple))
        self.version = info.version
        self.step = info.step
        self.tokens_seen = info.tokens_seen
        self.planned_steps = info.planned_steps
        self.plateau_scale = float(info.plateau_scale)
        self.weight_dtype = "bf16" if info.weight_dtype == 1 else "f32"
        self.num_merges = info.num_merges
        self.param_count = info.param_count

    @classmethod
    def from_bytes(cls, data: bytes) -> "Checkpoint":
        lib = _lib()
        data = bytes(data)
        info = LlmhipScckInfo()
        buf = np.frombuffer(data, dtype=np.uint8) if data else np.zeros(1, dtype=np.uint8)
        rc = lib.llmhip_scck_parse(buf.ctypes.data, len(data), ctypes.byref(info))
        if rc != 0:
            raise ValueError(lib.llmhip_last_error().decode(errors="replace"))
        return cls(data, info)

    @classmethod
    def load(cls, path) -> "Checkpoint":
        with open(path, "rb") as f:
            return cls.from_bytes(f.read())

    def params(self, first: int, count: int) -> np.ndarray:
        """Parameters first .. first+count in ModelWeights::tensors() order, as f32."""
        out = np.empty(count, dtype=np.float32)
        rc = _lib().llmhip_scck_read_params(self._buf.ctypes.data, len(self._data), ctypes.byref(self.info), first,
                                            count, out.ctypes.data if count else None)
        if rc != 0:
            raise ValueError(_lib().llmhip_last_error().decode(errors="replace"))
        return out

    def embed(self) -> np.ndarray:
        """The embedding table, tied with the output head: [vocab_size, hidden_dim]."""
        v, h = self.config.vocab_size, self.config.hidden_dim
        return self.params(0, v * h).reshape(v, h)

    def final_norm_gain(self) -> np.ndarray:
        h = self.config.hidden_dim
        return self.params(self.param_count - h, h)
