"""Build step for the gfx950 sampler library (libllmhip_sampler.so).

Compiles the HIP sources under csrc/ with hipcc for gfx950 only, in-tree,
so the built library travels with the source tree. Flags that matter for
parity with the reference's f32 arithmetic:

* ``-ffp-contract=off``: no fused multiply-adds in f32 code (the reference's
  Rust code rounds every operation); the exp routine asks for its fused
  double-precision steps explicitly with __builtin_fma.
* ``-fhip-fp32-correctly-rounded-divide-sqrt``: IEEE division, as Rust's
  ``/`` on f32.
* no fast-math.
* ``-Xclang -target-feature -Xclang -packed-fp32-ops``: no packed f32
  instructions are generated.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
LIB_NAME = "libllmhip_sampler.so"
LIB_PATH = PKG_DIR / LIB_NAME
SOURCES = ["sampler_kernels.hip", "vocab_full.hip", "vocab_plain.hip", "fast_nch8.hip", "fast_nch_small.hip", "fast_counts.hip", "fast_counts8.hip",
           "fast_counts_small.hip", "tied_head.hip", "bench_floor.hip", "stream_topk.hip", "stream_topk_bigk.hip", "sampler_api.hip", "scck_reader.cpp"]
ARCH = "gfx950"


def source_hash() -> str:
    """SHA-256 (first 16 hex digits) over the library's sources and the
    header: the identity of a build, which measured profile figures name so
    that bench.py can tell whether they belong to the library it runs."""
    import hashlib

    h = hashlib.sha256()
    files = (sorted(CSRC.glob("*.h")) + sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
             + [PKG_DIR.parent / "include" / "llmhip_sampler.h"])
    for f in files:
        h.update(f.name.encode())
        h.update(f.read_bytes())
    return h.hexdigest()[:16]


def hipcc_path() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build the sampler)")


def compile_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-ffp-contract=off",
        "-fno-fast-math",
        "-fhip-fp32-correctly-rounded-divide-sqrt",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall",
        "-Wno-unused-result",
    ]


def build_library(verbose: bool = False) -> Path:
    """Compile every HIP source and link the shared library. Always rebuilds."""
    from concurrent.futures import ThreadPoolExecutor

    hipcc = hipcc_path()
    cmds, objs = [], []
    for src in SOURCES:
        obj = CSRC / (Path(src).stem + ".o")
        cmds.append([hipcc, *compile_flags(), "-c", str(CSRC / src), "-o", str(obj)])
        objs.append(str(obj))
    if verbose:
        for cmd in cmds:
            print(" ".join(cmd), flush=True)
    # The sources compile independently; the kernel files dominate.
    workers = max(1, min(len(cmds), os.cpu_count() or 1, 8))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        for r in list(pool.map(lambda c: subprocess.run(c, check=True), cmds)):
            pass
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *objs]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB_PATH)
    for o in objs:
        Path(o).unlink(missing_ok=True)
    return LIB_PATH


if __name__ == "__main__":
    build_library(verbose="-v" in sys.argv)
    print(LIB_PATH)
