"""The kernel's exp (scriptonait_amd/csrc/glibc_expf.h) is bit-identical to
the host glibc expf that Rust's f32::exp links to (the reference computes
`(work[i] - max).exp()`, crates/llm-core/src/generate.rs:373).

The header is compiled for the host with g++ (same double-precision
operations, explicit fused multiply-adds) and compared with libm's expf over
every binary32 input. The device build of the same header is compared with
the host oracle on the GPU by the parity tests. A control variant without the
fused steps must differ: the comparison can tell the two apart.
"""
import subprocess
import textwrap
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HDR = ROOT / "scriptonait_amd" / "csrc" / "glibc_expf.h"

SRC = textwrap.dedent(r"""
    #include "glibc_expf.h"
    #include <math.h>
    #include <stdio.h>
    #include <stdlib.h>
    #include <thread>
    #include <vector>
    #include <atomic>
    int main(int argc, char** argv) {
      const uint64_t lo = strtoull(argv[1], 0, 0), hi = strtoull(argv[2], 0, 0);
      std::atomic<unsigned long long> bad{0};
      const int nt = 8;
      std::vector<std::thread> th;
      for (int t = 0; t < nt; ++t) th.emplace_back([&, t] {
        unsigned long long b = 0;
        for (uint64_t u = lo + t; u < hi; u += nt) {
          const float x = llmhip::f32_from_bits((uint32_t)u);
          const float a = expf(x), c = llmhip::glibc_expf(x);
          if (llmhip::f32_bits(a) != llmhip::f32_bits(c) && !(isnan(a) && isnan(c))) ++b;
        }
        bad += b;
      });
      for (auto& x : th) x.join();
      printf("%llu\n", (unsigned long long)bad);
      return 0;
    }
""")


def _build(tmp_path, fused: int) -> Path:
    src = tmp_path / "expf_check.cpp"
    src.write_text(SRC)
    exe = tmp_path / f"expf_check_{fused}"
    flags = ["-mfma"] if fused else []
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", *flags,
                    f"-DLLMHIP_EXPF_FUSED={fused}", f"-I{HDR.parent}", str(src), "-o", str(exe),
                    "-lm", "-lpthread"], check=True)
    return exe


def _mismatches(exe, lo, hi) -> int:
    out = subprocess.run([str(exe), hex(lo), hex(hi)], check=True, capture_output=True, text=True)
    return int(out.stdout.strip())


def test_expf_bit_exact_over_every_binary32(tmp_path):
    exe = _build(tmp_path, 1)
    assert _mismatches(exe, 0, 1 << 32) == 0


def test_unfused_control_variant_differs(tmp_path):
    # The plain-multiply-add form differs from glibc on a few inputs, so the
    # exhaustive comparison is sharp enough to see the contraction choice.
    exe = _build(tmp_path, 0)
    assert _mismatches(exe, 0, 1 << 32) > 0
