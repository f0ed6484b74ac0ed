"""MI355X (gfx950) decode-time sampler for scriptonait.

A drop-in for llm-core's `sample_with` (crates/llm-core/src/generate.rs:325-420),
batched over rows and computed by hand-written HIP kernels. The C ABI is in
include/llmhip_sampler.h; `scriptonait_amd.sampler` is the Python host mirror.
"""
from .workloads import CONFIGS, PARAMS_DTYPE, make_workload  # noqa: F401

__all__ = ["CONFIGS", "PARAMS_DTYPE", "make_workload"]
