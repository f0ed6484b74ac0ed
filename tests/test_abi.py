"""The C-ABI library loads and exports every entry point that
include/llmhip_sampler.h declares; argument errors come back as status codes
(no GPU is touched: every call here fails validation or finds no device)."""
import ctypes
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

from scriptonait_amd import sampler as smp

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "llmhip_sampler.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(llmhip_[a-z_]+)\s*\(", text)))


def test_header_declares_the_expected_entry_points():
    assert declared_functions() == sorted(smp.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol():
    lib = smp.load_library()
    out = subprocess.run(["nm", "-D", "--defined-only", str(smp.LIB_PATH)], check=True,
                         capture_output=True, text=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    for name in declared_functions():
        assert name in exported, name
        assert hasattr(lib, name)


def test_params_struct_layout_matches_header():
    assert ctypes.sizeof(smp.LlmhipParams) == 20
    assert smp.PARAMS_DTYPE.itemsize == 20
    names = [f[0] for f in smp.LlmhipParams._fields_]
    assert names == list(smp.PARAMS_DTYPE.names)


def test_version_and_status_strings():
    lib = smp.load_library()
    assert lib.llmhip_abi_version() == 7
    assert lib.llmhip_status_string(0) == b"ok"
    assert lib.llmhip_status_string(-1) == b"invalid argument"
    assert lib.llmhip_status_string(-2) == b"no HIP device"
    assert lib.llmhip_status_string(12345) == b"unknown status"


def test_argument_validation_without_a_device():
    lib = smp.load_library()
    vp = ctypes.c_void_p
    # null context
    ids = np.zeros(1, dtype=np.uint32)
    st = np.zeros(1, dtype=np.uint64)
    prm = np.zeros(1, dtype=smp.PARAMS_DTYPE)
    x = np.zeros((1, 8), dtype=np.float32)
    rc = lib.llmhip_sample_host(None, x.ctypes.data, 1, 8, 8, prm.ctypes.data, 0, None, None, None,
                                0, 258, st.ctypes.data, ids.ctypes.data, None, None)
    assert rc == -1
    assert b"ctx" in lib.llmhip_last_error()
    rc = lib.llmhip_ctx_create(0, None)
    assert rc == -1
    assert lib.llmhip_ctx_destroy(None) == 0
    out = smp.LlmhipStatus()
    assert lib.llmhip_ctx_status(None, None, ctypes.byref(out)) == -1
    assert lib.llmhip_ctx_debug(None, smp.DEBUG_SPIN_LIMIT, 1) == -1


def test_status_struct_layout_matches_header():
    assert ctypes.sizeof(smp.LlmhipStatus) == 8
    text = HEADER.read_text()
    assert "uint32_t flags;" in text and "uint32_t handovers;" in text
    assert re.search(r"#define LLMHIP_KSTATUS_SYNC_TIMEOUT 1u", text)
    assert re.search(rf"#define LLMHIP_DEBUG_SPIN_LIMIT {smp.DEBUG_SPIN_LIMIT}\b", text)
    assert re.search(rf"#define LLMHIP_DEBUG_SET_FLAGS {smp.DEBUG_SET_FLAGS}\b", text)


def test_context_creation_reports_missing_device_or_succeeds():
    lib = smp.load_library()
    ctx = ctypes.c_void_p()
    rc = lib.llmhip_ctx_create(0, ctypes.byref(ctx))
    assert rc in (0, -2)
    if rc == 0:
        assert lib.llmhip_ctx_destroy(ctx) == 0
    else:
        with pytest.raises(smp.SamplerError):
            smp.Sampler(0)


def test_rust_shim_in_integration_notes_names_every_symbol():
    text = (ROOT / "INTEGRATION.md").read_text()
    for name in declared_functions():
        assert name in text, name
