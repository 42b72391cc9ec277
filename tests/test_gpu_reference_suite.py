"""The reference's own op tests on the MI355X.

tests/test_ops.cpp of the reference and its src/tensor.cpp, compiled unchanged
where they lie and linked against backend_hip through
tests/cpp/reference_backend_binding.cpp (the reference's GPU backend interface,
src/backend_cuda.h, on this library's C ABI; oracle/Makefile, target suite).
Its test_cuda section (test_ops.cpp:356-477) then compares every device op
with the reference's CPU path at the reference's own tolerances: host/device
round trip, linear with fp32 and bf16 weights, conv2d, group/layer/RMS norms,
per-head RMS norm, both rotary conventions, swiglu, geglu, the activations,
add/scale/affine, attention (MHA, GQA, causal), the row helpers and the shape
ops. A drop-in must pass this suite; the one check that the reference's own
device path fails by construction is named below with its reason.
"""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "oracle", "_ref", "test_ops_sdh")


# The one check the reference's own device path cannot meet either: its
# gemm_nt_bf16 rounds x to bf16 before the product (backend_cuda.cu:466-467,
# as this backend does: the bf16 x bf16 MFMA / library GEMM), its CPU path
# keeps x in fp32 (tensor.cpp:496-497). With unit-variance x and W over
# K = 300 that difference alone is about 0.1 max-abs, above the suite's 3e-2;
# the reference's GPU backend has never run on hardware (README.md:330-333).
# tests/test_gpu_gemm.py::test_linear_bf16_at_reference_suite_shape pins this
# check's value: the exact sum of the rounded operands within the fp32 bound,
# and 0.05-0.2 from the fp32-x product.
KNOWN_GAP = "cuda linear bf16 +bias"


def test_reference_op_suite_on_device():
    if not os.path.exists(EXE):
        pytest.skip("oracle/_ref/test_ops_sdh not built (the reference tree was absent when build() ran)")
    r = subprocess.run([EXE], capture_output=True, text=True, timeout=600)
    lines = r.stdout.splitlines()
    print("\n".join(l for l in lines if l.startswith("cuda")))
    assert not any("GPU comparisons skipped" in l for l in lines), "the device section did not run"
    checks = [l for l in lines if "max|err|" in l]
    device = [l for l in checks if l.startswith("cuda ")]
    assert len(device) >= 40, "\n".join(device)
    failed = [l for l in checks if not l.rstrip().endswith("ok")]
    assert all(l.startswith(KNOWN_GAP) for l in failed), "\n".join(failed)
    if failed:  # the known gap, and nothing else: exit status 1, "1 FAILED"
        err = float(failed[0].split("=")[1].split()[0])
        assert err <= 0.25, failed[0]
        assert r.returncode == 1 and "1 FAILED" in r.stdout, r.stdout[-2000:] + r.stderr[-2000:]
    else:
        assert r.returncode == 0 and "all ok" in r.stdout, r.stdout[-2000:] + r.stderr[-2000:]
