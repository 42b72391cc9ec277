"""Pins of the conv2d oracle (oracle/oracle.py: Oracle.conv2d), without a GPU.

The oracle restates tensor.cpp:520-560 in float64. It is pinned by:
  * the reference's own CPU conv2d (compiled, oracle/_ref) on the shapes of
    the reference's GPU-vs-CPU checks (test_ops.cpp:383-388: k3 s1, k3 s2, k1)
    and a few more (k4 s2 p1, non-square kernels, no bias);
  * closed forms: a 1x1 convolution is a matrix product over channels; a
    centred delta kernel (3x3, pad 1) copies the input; a corner delta shifts
    it by one pixel with zeros entering (the padding);
  * planted mistakes: kernel taps transposed, bias dropped.
"""
import numpy as np
import pytest

from tolerances import assert_gemm

SHAPES = [  # N, Cin, H, W, Cout, kh, kw, stride, pad, bias
    (2, 5, 9, 11, 6, 3, 3, 1, 1, True), (2, 5, 9, 11, 6, 3, 3, 2, 1, True), (2, 5, 9, 11, 4, 1, 1, 1, 0, True),
    (1, 3, 16, 12, 8, 4, 4, 2, 1, True), (1, 4, 7, 9, 3, 3, 1, 1, 0, False), (1, 6, 10, 10, 5, 2, 5, 3, 2, True),
]


def _case(orc, N, Cin, H, W, Cout, kh, kw, bias, seed):
    x = orc.randn((N, Cin, H, W), seed)
    w = orc.randn((Cout, Cin, kh, kw), seed + 1, 0.0, 0.3)
    b = orc.randn((Cout,), seed + 2) if bias else None
    return x, w, b


@pytest.mark.parametrize("N,Cin,H,W,Cout,kh,kw,stride,pad,bias", SHAPES)
def test_conv2d_oracle_vs_reference(orc, ref, N, Cin, H, W, Cout, kh, kw, stride, pad, bias):
    x, w, b = _case(orc, N, Cin, H, W, Cout, kh, kw, bias, 1100 + H + kh)
    want, S = orc.conv2d(x, w, b, stride, pad)
    got = ref.conv2d(x, w, b, stride, pad)
    assert_gemm(got, want, S, Cin * kh * kw + 1, f"reference conv2d {x.shape} k{kh}x{kw} s{stride} p{pad}")


def _pin_1x1_is_matmul(orc):
    x = orc.randn((2, 7, 5, 6), 1201)
    w = orc.randn((3, 7, 1, 1), 1202)
    out, _ = orc.conv2d(x, w)
    want = np.einsum("ck,nkp->ncp", w[:, :, 0, 0].astype(np.float64), x.reshape(2, 7, 30).astype(np.float64))
    np.testing.assert_allclose(out.reshape(2, 3, 30), want, rtol=1e-6, atol=1e-6)


def _pin_delta_copies(orc):
    x = orc.randn((1, 4, 6, 5), 1203)
    w = np.zeros((4, 4, 3, 3), np.float32)
    w[np.arange(4), np.arange(4), 1, 1] = 1.0
    out, _ = orc.conv2d(x, w, None, 1, 1)
    assert np.array_equal(out, x)


def _pin_corner_delta_shifts(orc):
    x = orc.randn((1, 2, 6, 5), 1204)
    w = np.zeros((2, 2, 3, 3), np.float32)
    w[0, 0, 0, 0] = 1.0  # out[0, oy, ox] = x[0, oy - 1, ox - 1]
    w[1, 1, 0, 2] = 1.0  # out[1, oy, ox] = x[1, oy - 1, ox + 1]
    out, _ = orc.conv2d(x, w, None, 1, 1)
    want = np.zeros_like(x)
    want[0, 0, 1:, 1:] = x[0, 0, :-1, :-1]
    want[0, 1, 1:, :-1] = x[0, 1, :-1, 1:]
    assert np.array_equal(out, want)


def _pin_bias(orc):
    x = np.zeros((1, 3, 4, 4), np.float32)
    w = orc.randn((2, 3, 3, 3), 1205)
    b = np.array([1.5, -2.0], np.float32)
    out, _ = orc.conv2d(x, w, b, 1, 1)
    assert np.array_equal(out, np.broadcast_to(b[None, :, None, None], out.shape))


def test_conv2d_closed_forms(orc):
    _pin_1x1_is_matmul(orc)
    _pin_delta_copies(orc)
    _pin_corner_delta_shifts(orc)
    _pin_bias(orc)


@pytest.mark.parametrize("which,pin", [(15, _pin_corner_delta_shifts), (16, _pin_bias)])
def test_conv2d_pins_catch_planted_mistakes(orc, which, pin):
    pin(orc)
    orc.plant(which)
    try:
        with pytest.raises(AssertionError):
            pin(orc)
    finally:
        orc.plant(0)
