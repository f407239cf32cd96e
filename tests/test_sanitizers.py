"""The host code under AddressSanitizer and UndefinedBehaviorSanitizer.

`make -C rich-triplet-cpp_amd asan` builds the library's host sources (the
GGUF reader, the ABI's validation and workspace bookkeeping, the host
drop-ins) with both sanitizers on the host side only, linked with the
ordinary device objects.  The GGUF reader tests (corrupt and truncated files
included) and the ABI tests then run against that build in a child process
with the sanitizer runtime preloaded; any report fails the run.  No GPU."""
import glob
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "rich-triplet-cpp_amd")


def _asan_runtime():
    hits = sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    return hits[-1] if hits else None


@pytest.mark.skipif(_asan_runtime() is None, reason="clang ASan runtime not found")
def test_host_code_under_sanitizers():
    subprocess.run(["make", "-C", PKG, "asan", "-j8"], check=True, capture_output=True)
    lib = os.path.join(PKG, "lib_asan", "librt_hip.so")
    env = dict(os.environ)
    env["LD_PRELOAD"] = _asan_runtime()
    env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=1"
    env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1"
    env["RT_HIP_LIB_PATH"] = lib
    out = subprocess.run([sys.executable, "-m", "pytest", "-q", "-m", "not gpu", "-p", "no:cacheprovider",
                          os.path.join(ROOT, "tests", "test_gguf.py"), os.path.join(ROOT, "tests", "test_abi.py")],
                         env=env, capture_output=True, text=True, cwd=ROOT)
    report = out.stdout[-3000:] + out.stderr[-3000:]
    assert out.returncode == 0, report
    assert "ERROR: AddressSanitizer" not in report and "runtime error:" not in report, report
    assert " passed" in out.stdout
