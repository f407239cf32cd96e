"""The workspace growth rules (csrc/workspace_pool.hpp) on the CPU: a host-only
C++ check built with g++ under the address and undefined-behaviour
sanitizers and run here (no GPU)."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not installed")
def test_workspace_pool_rules(tmp_path):
    exe = tmp_path / "test_workspace_pool"
    subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
                    "-I", os.path.join(ROOT, "rich-triplet-cpp_amd", "csrc"),
                    os.path.join(ROOT, "tests", "cpp", "test_workspace_pool.cpp"), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0, out.stderr
    assert "all checks passed" in out.stdout
