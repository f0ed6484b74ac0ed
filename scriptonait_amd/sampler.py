"""Python host mirror of llm-core's sampler API over the gfx950 C ABI.

Mirrors crates/llm-core/src/generate.rs (SamplingConfig 25-95, sample_with
325-420, sample 423-433) and crates/llm-core/src/rng.rs (Rng 6-34) with the
same names, argument meaning and defaults, but every sample is computed by
libllmhip_sampler.so on the GPU. There is no CPU fallback here: when the
library or a GPU is missing the calls raise, so a test that passes has run
the HIP kernels.

Batched entry points:
  Sampler.sample_host(...)    host numpy arrays in and out (llmhip_sample_host)
  Sampler.sample_device(...)  torch CUDA tensors, stream-ordered (llmhip_sample_device)
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from pathlib import Path
from typing import Optional, Sequence

import numpy as np

from .workloads import PARAMS_DTYPE

LIB_PATH = Path(__file__).resolve().parent / "libllmhip_sampler.so"
BOS = 257  # crates/llm-core/src/tokenizer.rs:36
EOS = 258  # crates/llm-core/src/tokenizer.rs:38

LLMHIP_OK = 0
STATUS_NAMES = {
    0: "LLMHIP_OK",
    -1: "LLMHIP_ERR_INVALID_ARGUMENT",
    -2: "LLMHIP_ERR_NO_DEVICE",
    -3: "LLMHIP_ERR_HIP",
    -4: "LLMHIP_ERR_OUT_OF_MEMORY",
    -5: "LLMHIP_ERR_UNSUPPORTED",
}
EXPORTED_SYMBOLS = (
    "llmhip_abi_version",
    "llmhip_status_string",
    "llmhip_last_error",
    "llmhip_ctx_create",
    "llmhip_ctx_destroy",
    "llmhip_sample_host",
    "llmhip_sample_device",
    "llmhip_sample_device_noalloc",
    "llmhip_sample_tied_head_device",
    "llmhip_decode_step",
    "llmhip_decode_step_counts",
    "llmhip_seen_tokens",
    "llmhip_sample_device_bits",
    "llmhip_decode_step_bits",
    "llmhip_ctx_status",
    "llmhip_ctx_debug",
    "llmhip_scck_parse",
    "llmhip_scck_read_params",
    "llmhip_bench_floor",
)
KSTATUS_SYNC_TIMEOUT = 1
DEBUG_SPIN_LIMIT = 1
DEBUG_SET_FLAGS = 2


class SamplerError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")
        self.status = status


class LlmhipStatus(ctypes.Structure):
    _fields_ = [("flags", ctypes.c_uint32), ("handovers", ctypes.c_uint32)]


class LlmhipParams(ctypes.Structure):
    _fields_ = [
        ("temperature", ctypes.c_float),
        ("top_k", ctypes.c_uint32),
        ("top_p", ctypes.c_float),
        ("min_p", ctypes.c_float),
        ("repetition_penalty", ctypes.c_float),
    ]


_lib: Optional[ctypes.CDLL] = None


def load_library(path: Path = LIB_PATH) -> ctypes.CDLL:
    """Load libllmhip_sampler.so (built by scriptonait_amd.build). Raises if absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not path.exists():
        raise FileNotFoundError(
            f"{path} is not built; run `python -m scriptonait_amd.build` (or __graft_entry__.build())"
        )
    lib = ctypes.CDLL(str(path))
    vp, sz, u32, u64 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint32, ctypes.c_uint64
    lib.llmhip_abi_version.restype = ctypes.c_int
    lib.llmhip_status_string.restype = ctypes.c_char_p
    lib.llmhip_status_string.argtypes = [ctypes.c_int]
    lib.llmhip_last_error.restype = ctypes.c_char_p
    lib.llmhip_ctx_create.restype = ctypes.c_int
    lib.llmhip_ctx_create.argtypes = [ctypes.c_int, ctypes.POINTER(vp)]
    lib.llmhip_ctx_destroy.restype = ctypes.c_int
    lib.llmhip_ctx_destroy.argtypes = [vp]
    common = [vp, vp, sz, sz, sz, vp, sz, vp, vp, vp, sz, u32, vp, vp, vp, vp]
    lib.llmhip_sample_host.restype = ctypes.c_int
    lib.llmhip_sample_host.argtypes = common
    lib.llmhip_sample_device.restype = ctypes.c_int
    lib.llmhip_sample_device.argtypes = common + [vp]
    lib.llmhip_sample_device_noalloc.restype = ctypes.c_int
    lib.llmhip_sample_device_noalloc.argtypes = common + [vp]
    lib.llmhip_sample_tied_head_device.restype = ctypes.c_int
    lib.llmhip_sample_tied_head_device.argtypes = [vp, vp, sz, sz, sz, vp, sz, sz, vp, sz, vp, vp, vp, sz, u32, vp, vp,
                                                   vp, vp, vp, vp]
    lib.llmhip_decode_step.restype = ctypes.c_int
    decode = [vp, vp, sz, sz, sz, vp, sz, vp, sz, vp, vp, vp, sz, vp, sz, u32, vp, vp, vp]
    lib.llmhip_decode_step.argtypes = decode
    lib.llmhip_decode_step_counts.restype = ctypes.c_int
    lib.llmhip_decode_step_counts.argtypes = [vp, vp, sz, sz, sz, vp, sz, vp, sz, vp, vp, vp, sz, vp, sz, vp, vp, sz,
                                              u32, vp, vp, vp]
    lib.llmhip_sample_device_bits.restype = ctypes.c_int
    lib.llmhip_sample_device_bits.argtypes = common + [vp]
    lib.llmhip_decode_step_bits.restype = ctypes.c_int
    lib.llmhip_decode_step_bits.argtypes = decode
    lib.llmhip_ctx_status.restype = ctypes.c_int
    lib.llmhip_ctx_status.argtypes = [vp, vp, ctypes.POINTER(LlmhipStatus)]
    lib.llmhip_ctx_debug.restype = ctypes.c_int
    lib.llmhip_ctx_debug.argtypes = [vp, ctypes.c_int, u32]
    lib.llmhip_seen_tokens.restype = ctypes.c_int
    lib.llmhip_seen_tokens.argtypes = [vp, vp, sz, sz, vp, vp]
    lib.llmhip_bench_floor.restype = ctypes.c_int
    lib.llmhip_bench_floor.argtypes = [vp, vp, sz, sz, sz, ctypes.c_int, vp, vp]
    _lib = lib
    return lib


def _check(lib: ctypes.CDLL, status: int) -> None:
    if status != LLMHIP_OK:
        raise SamplerError(status, lib.llmhip_last_error().decode(errors="replace"))


def _ptr(a: Optional[np.ndarray]) -> Optional[int]:
    return None if a is None else a.ctypes.data


# ---------------------------------------------------------------------------
# Mirror of the reference types
# ---------------------------------------------------------------------------
@dataclass
class SamplingConfig:
    """generate.rs:25-95 (same fields and defaults)."""

    temperature: float = 0.9
    top_k: int = 40
    top_p: float = 0.95
    min_p: float = 0.0
    repetition_penalty: float = 1.1
    repetition_window: int = 128
    seed: int = 0
    allowed: Optional[Sequence[bool]] = None

    def to_params(self) -> np.ndarray:
        p = np.zeros(1, dtype=PARAMS_DTYPE)
        p["temperature"] = self.temperature
        p["top_k"] = self.top_k
        p["top_p"] = self.top_p
        p["min_p"] = self.min_p
        p["repetition_penalty"] = self.repetition_penalty
        return p

    def allowed_mask(self) -> Optional[np.ndarray]:
        if self.allowed is None:
            return None
        return np.asarray(self.allowed, dtype=np.uint8)


@dataclass
class Rng:
    """rng.rs:6-34 — SplitMix64; `state` is what the C ABI carries per row."""

    state: int = 0

    @classmethod
    def seed_from_u64(cls, seed: int) -> "Rng":
        return cls(state=seed & 0xFFFFFFFFFFFFFFFF)

    def next_u64(self) -> int:
        self.state = (self.state + 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF
        z = self.state
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & 0xFFFFFFFFFFFFFFFF
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & 0xFFFFFFFFFFFFFFFF
        return z ^ (z >> 31)

    def next_f32(self) -> float:
        return float(np.float32(self.next_u64() >> 40) / np.float32(1 << 24))


# ---------------------------------------------------------------------------
# Batched sampler over the C ABI
# ---------------------------------------------------------------------------
@dataclass
class SampleResult:
    ids: np.ndarray
    rng_state: np.ndarray
    kept: Optional[np.ndarray] = None
    probs: Optional[np.ndarray] = None
    extra: dict = field(default_factory=dict)


class Sampler:
    """Owns one llmhip_ctx (device scratch reused across calls)."""

    def __init__(self, device: int = 0):
        self.lib = load_library()
        ctx = ctypes.c_void_p()
        _check(self.lib, self.lib.llmhip_ctx_create(device, ctypes.byref(ctx)))
        self.ctx = ctx

    def close(self) -> None:
        if self.ctx:
            self.lib.llmhip_ctx_destroy(self.ctx)
            self.ctx = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def sample_host(self, logits: np.ndarray, params: np.ndarray, rng_state: np.ndarray,
                    hist: Optional[np.ndarray] = None, hist_offsets: Optional[np.ndarray] = None,
                    allowed: Optional[np.ndarray] = None, eos_id: int = EOS, V: Optional[int] = None,
                    want_probs: bool = False, want_kept: bool = True) -> SampleResult:
        """llmhip_sample_host on numpy arrays. logits is [B, ld]; params is a
        PARAMS_DTYPE array of length 1 (shared) or B (per row). rng_state is
        copied, not modified in place; the advanced state is returned."""
        logits = np.ascontiguousarray(logits, dtype=np.float32)
        if logits.ndim == 1:
            logits = logits[None, :]
        B, ld = logits.shape
        V = ld if V is None else V
        params = np.ascontiguousarray(params, dtype=PARAMS_DTYPE)
        stride = 0 if params.shape[0] == 1 else 1
        if stride and params.shape[0] != B:
            raise ValueError("params must have 1 or B entries")
        st = np.ascontiguousarray(rng_state, dtype=np.uint64).copy()
        ids = np.zeros(B, dtype=np.uint32)
        kept = np.zeros(B, dtype=np.uint32) if want_kept else None
        probs = np.zeros((B, V), dtype=np.float32) if want_probs else None
        if hist is not None:
            hist = np.ascontiguousarray(hist, dtype=np.uint32)
            hist_offsets = np.ascontiguousarray(hist_offsets, dtype=np.uint32)
            if hist.size == 0:
                hist = np.zeros(1, dtype=np.uint32)
        if allowed is not None:
            allowed = np.ascontiguousarray(allowed, dtype=np.uint8)
        status = self.lib.llmhip_sample_host(
            self.ctx, _ptr(logits), B, V, ld, _ptr(params), stride,
            _ptr(hist), _ptr(hist_offsets), _ptr(allowed),
            0 if allowed is None else allowed.size, eos_id,
            _ptr(st), _ptr(ids), _ptr(probs), _ptr(kept))
        _check(self.lib, status)
        return SampleResult(ids=ids, rng_state=st, kept=kept, probs=probs)

    def sample_device(self, logits, params: np.ndarray, rng_state, out_ids, V: Optional[int] = None,
                      hist=None, hist_offsets=None, allowed=None, eos_id: int = EOS,
                      out_probs=None, out_kept=None, stream=None, allowed_bits=None,
                      allowed_len: Optional[int] = None, noalloc: bool = False) -> None:
        """llmhip_sample_device on torch CUDA tensors (logits [B, ld] f32,
        rng_state [B] int64 viewed as u64, out_ids [B] int32). Enqueued on
        `stream` (default: torch's current stream); does not synchronize.
        With allowed_bits (int32 words, as seen_tokens writes them; covering
        allowed_len ids, default V) it calls llmhip_sample_device_bits; with
        noalloc, llmhip_sample_device_noalloc (the entry that allocates no
        device memory)."""
        import torch

        B, ld = logits.shape
        V = ld if V is None else V
        params = np.ascontiguousarray(params, dtype=PARAMS_DTYPE)
        stride = 0 if params.shape[0] == 1 else 1
        if stream is None:
            stream = torch.cuda.current_stream(logits.device)
        dp = lambda t: None if t is None else t.data_ptr()  # noqa: E731
        if allowed_bits is not None:
            if allowed is not None or noalloc:
                raise ValueError("allowed_bits goes with neither allowed nor noalloc")
            status = self.lib.llmhip_sample_device_bits(
                self.ctx, dp(logits), B, V, ld, _ptr(params), stride,
                dp(hist), dp(hist_offsets), dp(allowed_bits), V if allowed_len is None else allowed_len,
                eos_id, dp(rng_state), dp(out_ids), dp(out_probs), dp(out_kept), stream.cuda_stream)
        else:
            entry = self.lib.llmhip_sample_device_noalloc if noalloc else self.lib.llmhip_sample_device
            status = entry(
                self.ctx, dp(logits), B, V, ld, _ptr(params), stride,
                dp(hist), dp(hist_offsets), dp(allowed),
                0 if allowed is None else allowed.numel(), eos_id,
                dp(rng_state), dp(out_ids), dp(out_probs), dp(out_kept), stream.cuda_stream)
        _check(self.lib, status)

    def sample_tied_head_device(self, hidden, embed, params: np.ndarray, rng_state, out_ids, hist=None,
                                hist_offsets=None, allowed=None, eos_id: int = EOS, out_probs=None, out_kept=None,
                                out_logits=None, stream=None) -> None:
        """llmhip_sample_tied_head_device on torch CUDA tensors: logits =
        hidden [B, h] @ embed [V, h]^T in the reference's dot order, then the
        sampler on them. out_logits ([B, V] float32) receives the logits if
        given. Enqueued on `stream` (default: torch's current stream)."""
        import torch

        B, h = hidden.shape
        V = embed.shape[0]
        if embed.shape[1] != h:
            raise ValueError("embed must be [V, h]")
        params = np.ascontiguousarray(params, dtype=PARAMS_DTYPE)
        stride = 0 if params.shape[0] == 1 else 1
        if stream is None:
            stream = torch.cuda.current_stream(hidden.device)
        dp = lambda t: None if t is None else t.data_ptr()  # noqa: E731
        status = self.lib.llmhip_sample_tied_head_device(
            self.ctx, dp(hidden), B, h, hidden.stride(0), dp(embed), V, embed.stride(0), _ptr(params), stride,
            dp(hist), dp(hist_offsets), dp(allowed), 0 if allowed is None else allowed.numel(), eos_id,
            dp(rng_state), dp(out_ids), dp(out_probs), dp(out_kept), dp(out_logits), stream.cuda_stream)
        _check(self.lib, status)

    def seen_tokens(self, tokens, V: int, out_bits=None, stream=None):
        """llmhip_seen_tokens: the allowed mask as bits (an int32 CUDA tensor
        of ceil(V / 32) words) from a CUDA tensor of token ids (int32 viewed
        as u32). Enqueued on `stream` (default: torch's current stream)."""
        import torch

        words = (V + 31) // 32
        if out_bits is None:
            out_bits = torch.empty(max(words, 1), dtype=torch.int32, device=tokens.device)
        if stream is None:
            stream = torch.cuda.current_stream(tokens.device)
        status = self.lib.llmhip_seen_tokens(self.ctx, tokens.data_ptr() if tokens.numel() else None,
                                             tokens.numel(), V, out_bits.data_ptr(), stream.cuda_stream)
        _check(self.lib, status)
        return out_bits


    def decode_step(self, logits, params: np.ndarray, ring, ring_len, done, window: int, rng_state, out_ids,
                    V: Optional[int] = None, allowed=None, eos_id: int = EOS, stream=None, allowed_bits=None,
                    allowed_len: Optional[int] = None, hist_start=None, counts=None, counted=None) -> None:
        """llmhip_decode_step on torch CUDA tensors: one Generator::step
        (generate.rs:157-165) for B generations whose history ring
        ([B, ring_cap] int32), lengths and done flags ([B] int32) and RNG
        states ([B] int64 viewed as u64) live on the device; hist_start
        ([B] int32, optional) is the first ring token still in each row's
        model cache. With counts ([B, >= (V+1)//2] int32, the u16 count
        table) and counted ([B, 2] int32) it calls llmhip_decode_step_counts
        (incremental history counts). Enqueued on `stream` (default: torch's
        current stream); does not synchronize."""
        import torch

        B, ld = logits.shape
        V = ld if V is None else V
        params = np.ascontiguousarray(params, dtype=PARAMS_DTYPE)
        stride = 0 if params.shape[0] == 1 else 1
        if stream is None:
            stream = torch.cuda.current_stream(logits.device)
        dp = lambda t: None if t is None else t.data_ptr()  # noqa: E731
        if counts is not None:
            if allowed_bits is not None:
                raise ValueError("counts go with the byte mask (allowed), not allowed_bits")
            status = self.lib.llmhip_decode_step_counts(
                self.ctx, dp(logits), B, V, ld, _ptr(params), stride, dp(ring), ring.shape[1], dp(ring_len),
                dp(done), dp(hist_start), window, dp(counts), counts.shape[1], dp(counted), dp(allowed),
                0 if allowed is None else allowed.numel(), eos_id, dp(rng_state), dp(out_ids), stream.cuda_stream)
        elif allowed_bits is not None:
            if allowed is not None:
                raise ValueError("pass allowed or allowed_bits, not both")
            status = self.lib.llmhip_decode_step_bits(
                self.ctx, dp(logits), B, V, ld, _ptr(params), stride, dp(ring), ring.shape[1], dp(ring_len),
                dp(done), dp(hist_start), window, dp(allowed_bits), V if allowed_len is None else allowed_len, eos_id,
                dp(rng_state), dp(out_ids), stream.cuda_stream)
        else:
            status = self.lib.llmhip_decode_step(
                self.ctx, dp(logits), B, V, ld, _ptr(params), stride, dp(ring), ring.shape[1], dp(ring_len),
                dp(done), dp(hist_start), window, dp(allowed), 0 if allowed is None else allowed.numel(), eos_id,
                dp(rng_state), dp(out_ids), stream.cuda_stream)
        _check(self.lib, status)


    def bench_floor(self, logits, read: bool, out, V: Optional[int] = None, stream=None) -> None:
        """llmhip_bench_floor on a [B, ld] float32 CUDA tensor: one launch of
        the register path's grid that only streams the rows in (read) or
        loads nothing; `out` is a [B] float32 CUDA tensor."""
        import torch

        B, ld = logits.shape
        if stream is None:
            stream = torch.cuda.current_stream(logits.device)
        _check(self.lib, self.lib.llmhip_bench_floor(self.ctx, logits.data_ptr(), B, ld if V is None else V, ld,
                                                     1 if read else 0, out.data_ptr(), stream.cuda_stream))

    def status(self, stream=None) -> LlmhipStatus:
        """llmhip_ctx_status: waits for `stream` (default: the null stream),
        returns and clears the device-entry flags and the hand-over count."""
        out = LlmhipStatus()
        _check(self.lib, self.lib.llmhip_ctx_status(self.ctx, None if stream is None else stream.cuda_stream,
                                                     ctypes.byref(out)))
        return out

    def debug(self, what: int, value: int) -> None:
        """llmhip_ctx_debug (test hooks: DEBUG_SPIN_LIMIT, DEBUG_SET_FLAGS)."""
        _check(self.lib, self.lib.llmhip_ctx_debug(self.ctx, what, value))


_default: Optional[Sampler] = None


def prompt_ring_tokens(prompt: Sequence[int], context_len: int) -> np.ndarray:
    """The tokens a decode-step ring starts with for `prompt`: what
    Generator::new prefills (crates/llm-core/src/generate.rs:131-139). An
    empty prompt becomes [BOS]; a prompt longer than context_len keeps only
    its last context_len tokens. The ring's owner fills row b with these and
    sets ring_len[b] to their count before the first llmhip_decode_step, so
    that step 1's `recent` is the reference's."""
    if context_len < 1:
        raise ValueError("context_len must be at least 1")
    tokens = np.asarray(prompt, dtype=np.uint32).reshape(-1)
    if tokens.size == 0:
        tokens = np.array([BOS], dtype=np.uint32)
    if tokens.size > context_len:
        tokens = tokens[tokens.size - context_len:]
    return tokens.copy()


def _default_sampler() -> Sampler:
    global _default
    if _default is None:
        _default = Sampler(0)
    return _default


def sample_with(logits: Sequence[float], sampling: SamplingConfig, recent: Sequence[int],
                rng: Rng) -> int:
    """generate.rs:325-420 — one row, computed on the GPU; advances `rng`."""
    x = np.asarray(logits, dtype=np.float32)[None, :]
    h = np.asarray(recent, dtype=np.uint32)
    offs = np.array([0, h.size], dtype=np.uint32)
    res = _default_sampler().sample_host(
        x, sampling.to_params(), np.array([rng.state], dtype=np.uint64),
        hist=h, hist_offsets=offs, allowed=sampling.allowed_mask())
    rng.state = int(res.rng_state[0])
    return int(res.ids[0])


def sample(logits: Sequence[float], temperature: float, rng: Rng) -> int:
    """generate.rs:423-433 — temperature only, no truncation or penalty."""
    cfg = SamplingConfig(temperature=temperature, top_k=0, top_p=1.0, min_p=0.0,
                         repetition_penalty=1.0)
    return sample_with(logits, cfg, [], rng)
