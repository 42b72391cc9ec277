"""Pins of the Z-Image transformer oracle (oracle/oracle.py:
Oracle.zimage_forward), without a GPU.

The oracle restates ZImageTransformer::forward (zimage.cpp:71-228) in float64.
It is pinned against the reference's own forward, compiled from its sources
(zimage.cpp, modules.cpp, safetensors.cpp, json.cpp, tensor.cpp in oracle/_ref)
and run on a small model of the checkpoint's names and layout
(tests/zimage_model.py) loaded from a .safetensors file by the reference's own
loader, with BF16 and with F32 weights, two latent sizes (one with image pad
tokens) and two timesteps. Bar: relative RMS 2e-5 (the reference computes in
fp32; measured 2.3e-6). Planted mistakes: the rotary h and w axes of the image
positions swapped, the attention scale and gate of the modulation swapped.
"""
import numpy as np
import pytest

import zimage_model as zm


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    W = zm.make_weights(0)
    path = tmp_path_factory.mktemp("zimage") / "model.safetensors"
    zm.write_safetensors(path, W)
    return W, path


CASES = [(16, 16, 20, 0.3), (24, 20, 40, 0.9)]  # H, W, text tokens, t (24x20: 120 image tokens + 8 pad)


@pytest.mark.parametrize("H,W,L,t", CASES)
@pytest.mark.parametrize("keep_bf16", [True, False])
def test_zimage_oracle_vs_reference_forward(orc, ref, model, H, W, L, t, keep_bf16):
    Wt, path = model
    x, cap = zm.inputs(orc, H=H, W=W, L=L)
    want = ref.zimage_forward(path, x, t, cap, zm.SHAPES["heads"], keep_bf16, zm.BF16_MIN)
    got = orc.zimage_forward(Wt, x, t, cap, zm.SHAPES["heads"])
    assert zm.rel_rms(got, want) <= 2e-5


def _pin(orc, ref, model):
    Wt, path = model
    x, cap = zm.inputs(orc)
    want = ref.zimage_forward(path, x, 0.3, cap, zm.SHAPES["heads"], True, zm.BF16_MIN)
    assert zm.rel_rms(orc.zimage_forward(Wt, x, 0.3, cap, zm.SHAPES["heads"]), want) <= 2e-5


@pytest.mark.parametrize("which", [13, 14])
def test_zimage_pin_catches_planted_mistakes(orc, ref, model, which):
    _pin(orc, ref, model)
    orc.plant(which)
    try:
        with pytest.raises(AssertionError):
            _pin(orc, ref, model)
    finally:
        orc.plant(0)


def test_zimage_bf16_inputs_switch(orc, model):
    """Rounding the inputs of BF16-weight linears (the device numerics) moves the
    output by about the rounding's size, not more: the two oracle modes differ
    at relative RMS between 1e-4 and 1e-2."""
    Wt, _ = model
    x, cap = zm.inputs(orc)
    a = orc.zimage_forward(Wt, x, 0.3, cap, 2)
    b = orc.zimage_forward(Wt, x, 0.3, cap, 2, zm.bf16_names(Wt), act_bf16=True)
    assert 1e-4 <= zm.rel_rms(b, a) <= 1e-2
