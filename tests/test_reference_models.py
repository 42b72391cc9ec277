"""The reference's own model tests, compiled unchanged, on this backend.

tests/test_zimage.cpp and tests/test_vae.cpp of the reference load a model
directory and a dump (input, expected output), run the reference's
ZImageTransformer::forward / VAEDecoder::decode and compare
(test_zimage.cpp:74-77: relative RMS < 2e-2; test_vae.cpp:71-73: < 1e-3).
oracle/Makefile (target suite) compiles each with the reference's model code,
weights loader and tensor library where they lie, linked against backend_hip
through tests/cpp/reference_backend_binding.cpp. With SD_TEST_DEVICE=cuda
the reference's own model code then runs on the MI355X, every tensor op
going through this library's C ABI: the drop-in as a user of the reference
would run it.

The reference's dumps come from PyTorch with the released checkpoints (absent
offline). Here the model is a random checkpoint of the real layout (Z-Image at
its full width, 30 heads of 128, with one block of each kind and a small FFN;
a small and a wide VAE decoder, tests/vae_model.py), and the expected output
is the reference's own CPU forward of the same file (oracle/_ref/libsdref.so).
On the CPU the compiled test must then reproduce it exactly, which pins the
harness (dump format, weight loading); on the GPU it must pass the
reference's own bar.
"""
import json
import os
import re
import subprocess

import numpy as np
import pytest

import vae_model as vm
import zimage_model as zm

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_DIR = os.path.join(ROOT, "oracle", "_ref")
ZIMAGE_EXE = os.path.join(REF_DIR, "test_zimage_sdh")
VAE_EXE = os.path.join(REF_DIR, "test_vae_sdh")
TIMING_EXE = os.path.join(REF_DIR, "zimage_reference_timing")

# test_zimage.cpp builds ZImageTransformer with the default Config: 30 heads
# and rotary axes 32 + 48 + 48, so the head size is 128 and dim 3840.
ZFULL = dict(dim=3840, heads=30, ffn=512, in_channels=16, cap_dim=64, t_freq=256, t_hidden=64, adaln_dim=64,
             noise_refiners=1, context_refiners=1, layers=1, patch=2)
Z_T = 0.7


def _dump(prefix, a, **meta):
    """The dumps' format (test_zimage.cpp:17-31): <prefix>.json with "shape" and
    metadata, <prefix>.bin with the float32 values."""
    a = np.ascontiguousarray(a, np.float32)
    with open(prefix + ".json", "w") as f:
        json.dump(dict(shape=list(a.shape), **meta), f)
    a.tofile(prefix + ".bin")


def _run(exe, model_dir, prefix, device):
    env = dict(os.environ)
    env.pop("SD_TEST_DEVICE", None)
    if device:
        env["SD_TEST_DEVICE"] = device
    print(f"running {os.path.basename(exe)} on {device or 'cpu'}", flush=True)
    r = subprocess.run([exe, model_dir, prefix], capture_output=True, text=True, timeout=600, env=env)
    print(r.stdout[-3000:], r.stderr[-2000:])
    m = re.search(r"relative rms error = ([0-9.eE+-]+)\s+(ok|FAIL)", r.stdout)
    assert m, r.stdout[-2000:] + r.stderr[-2000:]
    return r.returncode, float(m.group(1)), m.group(2)


def _need(exe):
    if not os.path.exists(exe):
        pytest.skip(f"{os.path.relpath(exe, ROOT)} not built (the reference tree was absent when build() ran)")


@pytest.fixture(scope="module")
def zimage_case(ref, orc, tmp_path_factory):
    """Model dir + dump prefix for test_zimage.cpp, expected output from the
    reference's CPU forward (weights loaded as test_zimage.cpp:48 loads them:
    keep_bf16, tensors of 2^20 elements or more in BF16)."""
    _need(ZIMAGE_EXE)
    root = tmp_path_factory.mktemp("zimage_ref")
    os.makedirs(root / "transformer")
    path = str(root / "transformer" / "diffusion_pytorch_model.safetensors")
    zm.write_safetensors(path, zm.make_weights(seed=3, s=ZFULL))
    x, cap = zm.inputs(orc, seed=3, H=16, W=16, L=8, s=ZFULL)
    want = ref.zimage_forward(path, x, Z_T, cap, ZFULL["heads"], keep_bf16=True, bf16_min_numel=1 << 20)
    assert np.all(np.isfinite(want))
    prefix = str(root / "ref_transformer")
    _dump(prefix + "_x", x[0], t=Z_T)
    _dump(prefix + "_cap", cap[0])
    _dump(prefix, want)
    return str(root), prefix


@pytest.fixture(scope="module", params=["small", "wide"])
def vae_case(request, ref, orc, tmp_path_factory):
    """Model dir + dump prefix for test_vae.cpp, expected image from the
    reference's CPU decode (F32 weights, as test_vae.cpp:51 loads them)."""
    _need(VAE_EXE)
    shape, hw = (vm.SMALL, 8) if request.param == "small" else (vm.WIDE, 32)
    root = tmp_path_factory.mktemp("vae_ref_" + request.param)
    os.makedirs(root / "vae")
    path = str(root / "vae" / "diffusion_pytorch_model.safetensors")
    vm.write_safetensors_f32(path, vm.make_weights(seed=5, s=shape))
    z = orc.randn((1, shape["latent"], hw, hw), 950)
    scaling, shift = 0.3611, 0.1159  # the FLUX VAE's latent scaling and shift
    want = ref.vae_decode(path, z, scaling, shift)
    assert np.all(np.isfinite(want)) and want.shape[1] == shape["out"]
    prefix = str(root / "ref_vae")
    _dump(prefix + "_in", z, scaling_factor=scaling, shift_factor=shift)
    _dump(prefix, want)
    return str(root), prefix, request.param


def test_reference_zimage_test_on_cpu(zimage_case):
    """The compiled test on the CPU reproduces the dump bit for bit."""
    rc, rel, verdict = _run(ZIMAGE_EXE, *zimage_case, None)
    assert rc == 0 and verdict == "ok" and rel == 0.0, (rc, rel)


def test_reference_vae_test_on_cpu(vae_case):
    rc, rel, verdict = _run(VAE_EXE, vae_case[0], vae_case[1], None)
    assert rc == 0 and verdict == "ok" and rel == 0.0, (rc, rel)


@pytest.mark.gpu
def test_reference_zimage_test_on_device(zimage_case):
    """The reference's zimage.cpp forward on the MI355X through backend_hip
    (linears on bf16 weights, attention, norms, rotary, the adaLN chain)
    within the reference's own bar against its CPU forward."""
    rc, rel, verdict = _run(ZIMAGE_EXE, *zimage_case, "cuda")
    assert rc == 0 and verdict == "ok" and rel < 2e-2, (rc, rel)


@pytest.mark.gpu
def test_reference_vae_test_on_device(vae_case):
    """The reference's vae.cpp decode on the MI355X through backend_hip
    (GroupNorm + SiLU, conv2d, nearest upsampling, the one-head attention)
    within the reference's own bar against its CPU decode."""
    rc, rel, verdict = _run(VAE_EXE, vae_case[0], vae_case[1], "cuda")
    assert rc == 0 and verdict == "ok" and rel < 1e-3, (rc, rel)


@pytest.mark.gpu
def test_reference_zimage_forward_at_step_shapes_on_device():
    """The reference's Z-Image forward through backend_hip at the 1024x1024
    step's token counts and the checkpoint's widths
    (tests/cpp/zimage_reference_timing.cpp; two main blocks and one refiner
    of each kind here, to keep the test short): it runs, op by op, and its
    output is finite and of the input's scale."""
    _need(TIMING_EXE)
    print("running zimage_reference_timing cuda 128 128 128 2 1 2", flush=True)
    r = subprocess.run([TIMING_EXE, "cuda", "128", "128", "128", "2", "1", "2"], capture_output=True, text=True,
                       timeout=300)
    print(r.stdout[-2000:], r.stderr[-2000:])
    assert r.returncode == 0 and "finite" in r.stdout and "NOT FINITE" not in r.stdout, r.stdout + r.stderr
    m = re.search(r"mean \|y\| ([0-9.eE+-]+)", r.stdout)
    assert m and 0.05 < float(m.group(1)) < 20.0, r.stdout
