"""GPU tests of sdh_conv2d (backend_cuda.h:45-47; tensor.cpp:520-560) against
the float64 oracle within the fp32 accumulation bound, and against the
reference's CPU conv2d at the bar of its own GPU check (test_ops.cpp:383-388,
max-abs 1e-3). Shapes: the reference's checks, VAE-like 3x3 convolutions
(one with more gathered floats than one chunk holds, so pixels run in two
chunks), a 1x1 projection, a stride-2 downsample, K not a multiple of 4
(the hand-written fp32 GEMM), no bias."""
import numpy as np
import pytest

from tolerances import assert_gemm

pytestmark = pytest.mark.gpu

SHAPES = [  # N, Cin, H, W, Cout, kh, kw, stride, pad, bias
    (2, 5, 9, 11, 6, 3, 3, 1, 1, True), (2, 5, 9, 11, 6, 3, 3, 2, 1, True), (2, 5, 9, 11, 4, 1, 1, 1, 0, True),
    (1, 128, 64, 64, 128, 3, 3, 1, 1, True), (1, 64, 256, 256, 32, 3, 3, 1, 1, True),
    (1, 512, 32, 32, 256, 1, 1, 1, 0, True), (1, 128, 64, 64, 128, 3, 3, 2, 0, False),
    (2, 3, 17, 13, 7, 3, 3, 1, 1, True),
]


@pytest.mark.parametrize("N,Cin,H,W,Cout,kh,kw,stride,pad,bias", SHAPES)
def test_conv2d(be, orc, N, Cin, H, W, Cout, kh, kw, stride, pad, bias):
    x = orc.randn((N, Cin, H, W), 1300 + Cin + H)
    w = orc.randn((Cout, Cin, kh, kw), 1301 + Cout, 0.0, 1.0 / np.sqrt(Cin * kh * kw))
    b = orc.randn((Cout,), 1302) if bias else None
    Ho, Wo = (H + 2 * pad - kh) // stride + 1, (W + 2 * pad - kw) // stride + 1
    out = be.empty((N, Cout, Ho, Wo))
    be.conv2d(be.array(x), N, Cin, H, W, be.array(w), Cout, kh, kw, be.array(b) if bias else None, stride, pad, out,
              Ho, Wo)
    want, S = orc.conv2d(x, w, b, stride, pad)
    assert_gemm(out.download(), want, S, Cin * kh * kw + 2, f"conv2d {x.shape} k{kh} s{stride} p{pad}")


def test_conv2d_vs_reference(be, orc, ref):
    """test_ops.cpp:383-388 on the device: k3 s1, k3 s2, k1 against the
    reference's CPU conv2d, max-abs 1e-3."""
    x = orc.randn((2, 5, 9, 11), 1310)
    w, b = orc.randn((6, 5, 3, 3), 1311), orc.randn((6,), 1312)
    w1, b1 = orc.randn((4, 5, 1, 1), 1313), orc.randn((4,), 1314)
    for ww, bb, s, p in ((w, b, 1, 1), (w, b, 2, 1), (w1, b1, 1, 0)):
        Cout, _, kh, kw = ww.shape
        Ho, Wo = (9 + 2 * p - kh) // s + 1, (11 + 2 * p - kw) // s + 1
        out = be.empty((2, Cout, Ho, Wo))
        be.conv2d(be.array(x), 2, 5, 9, 11, be.array(ww), Cout, kh, kw, be.array(bb), s, p, out, Ho, Wo)
        assert float(np.max(np.abs(out.download() - ref.conv2d(x, ww, bb, s, p)))) <= 1e-3


def test_conv2d_rejects_bad_output_size(be):
    import sdhip

    x, w, out = be.empty((1, 2, 5, 5)), be.empty((3, 2, 3, 3)), be.empty((1, 3, 5, 5))
    with pytest.raises(sdhip.SdhError) as e:
        be.conv2d(x, 1, 2, 5, 5, w, 3, 3, 3, None, 1, 0, out, 5, 5)  # pad 0 gives 3 x 3
    assert e.value.status == sdhip.SDH_ERR_INVALID
