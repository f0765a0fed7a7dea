"""Runs the C++17 boundary test (tests/cpp/test_linear_hip.cpp), which drives
include/infer/linear_hip.hpp and include/infer/linear_dispatch.hpp the way
the reference's gtest suite drives include/infer/cuda_ops.hpp."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BINARY = os.path.join(ROOT, "tests", "cpp", "test_linear_hip")


def test_cpp_boundary(dev):
    assert os.path.exists(BINARY), "build() compiles tests/cpp/test_linear_hip"
    out = subprocess.run([BINARY], capture_output=True, text=True, timeout=120)
    print(out.stdout)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "PASSED" in out.stdout
