"""The C ABI library loads and exports exactly what include/rt_hip.h declares.
No compute is run here (no GPU needed)."""
import ctypes
import os
import subprocess

import pytest

from conftest import load_package

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_library_exports_every_declared_function():
    pkg = load_package()
    lib = pkg.rt_hip.library()
    declared = pkg.rt_hip.header_functions()
    assert len(declared) >= 14
    missing = [f for f in declared if not hasattr(lib.lib, f)]
    assert not missing, missing


def test_exported_symbols_match_header():
    pkg = load_package()
    out = subprocess.run(["nm", "-D", "--defined-only", pkg.rt_hip.LIB_PATH],
                         capture_output=True, text=True, check=True).stdout
    exported = sorted({ln.split()[-1] for ln in out.splitlines() if " T rt_hip_" in ln})
    assert exported == pkg.rt_hip.header_functions()


def test_version_and_last_error_without_gpu():
    pkg = load_package()
    lib = pkg.rt_hip.library()
    assert "gfx950" in lib.version()
    assert isinstance(lib.lib.rt_hip_last_error(), bytes)


def test_argument_errors_are_reported_not_crashed():
    """Host-side validation runs before any device call: null pointers, bad
    M, K % 256 != 0 (the reference's unchecked Q4_K precondition) and
    misaligned pointers come back as status codes with a message."""
    pkg = load_package()
    lib = pkg.rt_hip.library()
    buf = ctypes.create_string_buffer(4096 + 16)
    base = (ctypes.addressof(buf) + 15) & ~15
    assert lib.status("rt_hip_gemv_q4k", None, base, base, 4, 256, 1, None) == 1      # null
    assert lib.status("rt_hip_gemv_q4k", base, base, base, 4, 256, 9, None) == 2      # m > 8
    assert lib.status("rt_hip_gemv_q4k", base, base, base, 4, 0, 1, None) == 1        # k = 0
    assert lib.status("rt_hip_gemv_q4k", base, base, base, 4, 1152, 1, None) == 3     # K % 256
    assert b"multiple of 256" in lib.lib.rt_hip_last_error()
    assert lib.status("rt_hip_gemv_q4k", base + 4, base, base, 4, 256, 1, None) == 3  # align
    assert lib.status("rt_hip_gemv_bf16", base, base, base, 4, 12, 1, None) == 3      # K % 8
    assert lib.status("rt_hip_gemm_q4k", base, 7, base, None, base, 4, 4, 256, None) == 1
    assert lib.status("rt_hip_gemm_bf16", base, 0, base, None, base, 4, 4, 96, None) == 3
    assert lib.status("rt_hip_argmax", base, 0, 4, base, None, None) == 1
    assert lib.status("rt_hip_quantize_q4k", base, base, 2, 300, None) == 3
    assert lib.status("rt_hip_linear_forward", 9, base, None, base, base, 1, 4, 256, None) == 6


def test_python_binding_fails_loudly_without_library(tmp_path):
    pkg = load_package()
    with pytest.raises(FileNotFoundError):
        pkg.rt_hip.Library(str(tmp_path / "missing.so"))
