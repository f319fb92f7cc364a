"""The C ABI library loads and exports every entry point include/leafhip.h declares."""
from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    text = (ROOT / "include" / "leafhip.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:lh_status|const char\*)\s+(lh_\w+)\s*\(", text, re.M)))


def test_header_declares_the_boundary():
    names = declared_symbols()
    for required in ("lh_context_create", "lh_model_load_file", "lh_session_create", "lh_forward", "lh_reset",
                     "lh_generate", "lh_gemv_w8a8", "lh_gemm_w8a8", "lh_attention", "lh_rmsnorm", "lh_last_error"):
        assert required in names


def test_library_exports_every_declared_symbol():
    from leaf_amd.runtime import LIBRARY, library
    assert LIBRARY.exists(), "libleafhip.so is not built (python -m leaf_amd.build)"
    lib = library()
    for name in declared_symbols():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", str(LIBRARY)], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (lh_\w+)", out))
    assert set(declared_symbols()) <= exported
    assert lib.lh_version().decode().startswith("leafhip")


def test_errors_are_status_codes_not_exceptions():
    from leaf_amd.runtime import library
    lib = library()
    out = ctypes.c_void_p()
    status = lib.lh_model_load_file(None, b"/nonexistent", 8, 0, ctypes.byref(out))
    assert status == 1 and b"required" in lib.lh_last_error()
