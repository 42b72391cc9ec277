"""Runs the C++ op test (tests/cpp/test_ops_hip.cpp): the reference's
GPU-vs-CPU op checks (test_ops.cpp:356-477) through the C++17 tensor.h-style
host API (libsdh_tensor.so) on the GPU, plus the fused ops and the error
behaviour. Exit status 0 means every check passed."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_cpp_op_test_on_gpu():
    exe = os.path.join(ROOT, "tests", "cpp", "test_ops_hip")
    assert os.path.exists(exe), "tests/cpp/test_ops_hip not built"
    r = subprocess.run([exe], capture_output=True, text=True, timeout=240)
    print(r.stdout)
    assert "GPU comparisons skipped" not in r.stdout, "no device visible to the C++ test"
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all ok" in r.stdout
