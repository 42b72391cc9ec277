"""The C ABI boundary without a GPU: every entry point declared in
include/*.h is exported by both libsdh.so (the HIP build) and libsdh_stub.so
(the CPU-only stub), the bindings declare exactly that set, and the stub and
the device-less HIP build fail loudly with typed statuses instead of
computing anything (the role of backend_cuda_stub.cpp, :14-56).
"""
import ctypes as C
import glob
import os
import re
import subprocess

import pytest

import sdhip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(sdh_\w+)\s*\(", text, flags=re.M))
    return names


def exported(path):
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line and line.split()[-1].startswith("sdh_")}


def test_header_declares_the_boundary():
    names = declared_symbols()
    # the backend_cuda.h non-GEMM surface (backend_cuda.h:23-36, :48-73) plus the fused ops
    for n in ("sdh_available", "sdh_device_name", "sdh_device_memory", "sdh_malloc", "sdh_free", "sdh_upload",
              "sdh_download", "sdh_copy", "sdh_zero", "sdh_synchronize", "sdh_group_norm", "sdh_layer_norm",
              "sdh_rms_norm", "sdh_rms_norm_heads", "sdh_rope", "sdh_softmax_rows", "sdh_geglu", "sdh_swiglu",
              "sdh_silu", "sdh_tanh", "sdh_gelu", "sdh_quick_gelu", "sdh_add", "sdh_scale", "sdh_affine",
              "sdh_mul_rows", "sdh_add_rows_scaled", "sdh_add_channel_bias", "sdh_add_rms_norm",
              "sdh_group_norm_silu", "sdh_ln_modulate_gate", "sdh_rope_qk"):
        assert n in names, n
    assert len(names) >= 40


@pytest.mark.parametrize("lib", [sdhip.LIB_PATH, sdhip.STUB_PATH])
def test_library_exports_every_declared_symbol(lib):
    assert os.path.exists(lib), f"{lib} not built"
    missing = declared_symbols() - exported(lib)
    assert not missing, f"{os.path.basename(lib)} lacks {sorted(missing)}"
    C.CDLL(lib)  # loads


def test_bindings_cover_the_header():
    assert set(sdhip.SIGNATURES) == declared_symbols()


def test_stub_fails_loudly():
    lib = sdhip.load_library(sdhip.STUB_PATH)
    assert lib.sdh_available() == 0
    assert lib.sdh_swiglu(None, None, None, 16) == sdhip.SDH_ERR_UNAVAILABLE
    assert b"stub" in lib.sdh_last_error()
    p = C.c_void_p()
    assert lib.sdh_malloc(64, C.byref(p)) == sdhip.SDH_ERR_UNAVAILABLE


def test_hip_build_without_device_is_unavailable():
    lib = sdhip.load_library(sdhip.LIB_PATH)
    if lib.sdh_available():
        pytest.skip("a HIP device is visible here")
    p = C.c_void_p()
    assert lib.sdh_malloc(64, C.byref(p)) == sdhip.SDH_ERR_UNAVAILABLE
    assert b"no HIP device" in lib.sdh_last_error()
    with pytest.raises(sdhip.SdhError) as e:
        sdhip.Backend()
    assert e.value.status == sdhip.SDH_ERR_UNAVAILABLE


def test_cpp_host_test_skips_without_device():
    """The C++ op test (mirror of the reference's test_ops GPU section) runs
    and reports the skip on a host without a GPU, like test_ops.cpp:357-360."""
    exe = os.path.join(ROOT, "tests", "cpp", "test_ops_hip")
    assert os.path.exists(exe), "tests/cpp/test_ops_hip not built (run __graft_entry__.build())"
    lib = sdhip.load_library(sdhip.LIB_PATH)
    if lib.sdh_available():
        pytest.skip("a HIP device is visible here; the GPU test runs it")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and "GPU comparisons skipped" in r.stdout
