"""A compiled C caller of include/rt_hip.h (tests/cpp/test_c_abi.c, built by
tests/cpp/Makefile against lib/librt_hip.so): the header compiles as C and
the library links and runs from C, without Python or torch.

CPU: argument checking and size queries.  GPU: the host drop-in
rt_hip_host_matmul (Q4_K and Q4Mat, with its weight cache), a weight handle
on device activations, and a captured graph replayed three times, each
against the oracle."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "cpp", "test_c_abi")


def test_c_caller_cpu_checks():
    subprocess.run(["make", "-C", os.path.join(ROOT, "tests", "cpp")], check=True, capture_output=True)
    out = subprocess.run([EXE, "cpu"], capture_output=True, text=True)
    assert out.returncode == 0, out.stderr
    assert "all checks passed" in out.stdout


@pytest.mark.gpu
def test_c_caller_gpu_checks():
    assert os.path.exists(EXE), "tests/cpp/test_c_abi is built by __graft_entry__.build()"
    print("[c abi] running the C caller on the GPU", flush=True)
    out = subprocess.run([EXE, "gpu"], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    assert "all checks passed" in out.stdout
