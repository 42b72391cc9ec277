"""The reductions' relative 1e-4 read elementwise, at the BASELINE config
sizes, against the oracle (bit-exact with the reference's tensor.cpp).

For each norm, GroupNorm and adaLN config the test reports the true
elementwise relative error |got - want| / max(|want|, 1e-6 max|want|) and
the elements beyond 1e-4. Those must be cancellation cases: elements formed
from terms much larger than themselves, whose error is within a few units
of 2^-24 of the terms' magnitude (tolerances.assert_true_relative). The
terms' magnitude is computed here in float64 from the inputs:
  * rms_norm / add_rms_norm, y = x rstd w: one product, no cancellation;
    the scale is |y| itself, so every element must meet 1e-4;
  * layer_norm, y = (x - mean) rstd g + b: (|x - mean| + |mean|) rstd |g| +
    |b| (the float mean's rounding enters through x - mean);
  * group_norm(+silu), o = x a + (b - mean a), a = rstd g: |x a| + |mean a| +
    |b|, times 1.1 after SiLU (|silu'| <= 1.1);
  * ln_modulate_gate, res += tanh(gate) (LN(x)(1 + scale) + shift): |res| +
    |tanh(gate)| (LN scale |1 + scale| + |shift|).
"""
import numpy as np
import pytest

from tolerances import assert_true_relative

pytestmark = pytest.mark.gpu

T, D = 4096, 3840


def _row_stats(x):
    x = x.astype(np.float64)
    mean = x.mean(axis=-1, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=-1, keepdims=True)
    return mean, var


@pytest.mark.parametrize("affine", [True, False])
def test_rms_norm_and_add_rms_norm_config_1(be, orc, affine):
    x = orc.randn((T, D), 7001)
    r = orc.randn((T, D), 7002)
    w = orc.randn((D,), 7003, 1.0, 0.1) if affine else None
    dw = be.array(w) if affine else None
    dx, dy = be.array(x), be.empty((T, D))
    be.rms_norm(dx, dy, T, D, dw, 1e-6)
    want = orc.rms_norm(x, w, 1e-6)
    assert_true_relative(dy.download(), want, np.abs(want), f"rms_norm [4096,3840] affine={affine}")
    dr = be.array(r)
    be.add_rms_norm(dx, dr, dy, T, D, dw, 1e-6)
    _, want = orc.add_rms_norm(x, r, w, 1e-6)
    assert_true_relative(dy.download(), want, np.abs(want), f"add_rms_norm (config 1) affine={affine}")


@pytest.mark.parametrize("gb", ["both", "none"])
def test_layer_norm_full_size(be, orc, gb):
    x = orc.randn((T, D), 7011)
    g = orc.randn((D,), 7012, 1.0, 0.1) if gb == "both" else None
    b = orc.randn((D,), 7013, 0.0, 0.1) if gb == "both" else None
    dx, dy = be.array(x), be.empty((T, D))
    be.layer_norm(dx, dy, T, D, be.array(g) if g is not None else None, be.array(b) if b is not None else None, 1e-6)
    want = orc.layer_norm(x, g, b, 1e-6)
    mean, var = _row_stats(x)
    rstd = 1.0 / np.sqrt(var + 1e-6)
    gg = np.abs(g.astype(np.float64)) if g is not None else 1.0
    bb = np.abs(b.astype(np.float64)) if b is not None else 0.0
    scale = (np.abs(x - mean) + np.abs(mean)) * rstd * gg + bb
    assert_true_relative(dy.download(), want, scale, f"layer_norm [4096,3840] {gb}")


GN = [((1, 512, 128, 128), 1e-6, True), ((1, 512, 128, 128), 1e-6, False), ((1, 128, 1024, 1024), 1e-6, True),
      ((2, 320, 64, 64), 1e-5, True), ((2, 1280, 8, 8), 1e-5, True)]


@pytest.mark.parametrize("shape,eps,silu", GN)
def test_group_norm_configs_4(be, orc, shape, eps, silu):
    groups = 32
    N, C = shape[0], shape[1]
    HW = shape[2] * shape[3]
    x = orc.randn(shape, 7021 + C, 0.0, 2.0)
    g = orc.randn((C,), 7022, 1.0, 0.1)
    b = orc.randn((C,), 7023, 0.0, 0.1)
    dx, dy = be.array(x), be.empty(shape)
    be.group_norm(dx, dy, N, C, HW, groups, be.array(g), be.array(b), eps, silu=silu)
    got = dy.download()
    want = orc.group_norm(x, groups, g, b, eps, silu=silu)
    seg = x.reshape(N, groups, -1).astype(np.float64)
    mean = seg.mean(axis=-1, keepdims=True)
    rstd = 1.0 / np.sqrt(((seg - mean) ** 2).mean(axis=-1, keepdims=True) + eps)
    a = (rstd.reshape(N, groups, 1) * g.astype(np.float64).reshape(1, groups, C // groups)).reshape(N, C, 1)
    mean_c = np.repeat(mean.reshape(N, groups), C // groups, axis=1).reshape(N, C, 1)
    scale = np.abs(x.reshape(N, C, HW) * a) + np.abs(mean_c * a) + np.abs(b.astype(np.float64)).reshape(1, C, 1)
    if silu:
        scale = 1.1 * scale
    del seg
    assert_true_relative(got.reshape(N, C, HW), want.reshape(N, C, HW), scale,
                         f"group_norm{'+silu' if silu else ''} {shape}")


@pytest.mark.parametrize("store_y", [True, False])
def test_ln_modulate_gate_config_5a(be, orc, store_y):
    x = orc.randn((T, D), 7031)
    res = orc.randn((T, D), 7032)
    sc = orc.randn((D,), 7033, 0.0, 0.2)
    sh = orc.randn((D,), 7034, 0.0, 0.2)
    gt = orc.randn((D,), 7035, 0.0, 0.2)
    dx, dres = be.array(x), be.array(res)
    dy = be.empty((T, D)) if store_y else None
    be.ln_modulate_gate(dx, dres, be.array(sc), be.array(sh), be.array(gt), dy, T, D, 1e-6)
    want_res, want_y = orc.ln_modulate_gate(x, res, sc, sh, gt, 1e-6)
    mean, var = _row_stats(x)
    rstd = 1.0 / np.sqrt(var + 1e-6)
    y_scale = (np.abs(x - mean) + np.abs(mean)) * rstd * np.abs(1.0 + sc.astype(np.float64)) + np.abs(sh)
    res_scale = np.abs(res.astype(np.float64)) + np.abs(np.tanh(gt.astype(np.float64))) * y_scale
    assert_true_relative(dres.download(), want_res, res_scale, "ln_modulate_gate (config 5a) res")
    if store_y:
        assert_true_relative(dy.download(), want_y, y_scale, "ln_modulate_gate (config 5a) y")


def test_rms_norm_heads_full_size(be, orc):
    """QK-norm at the Z-Image shape: 4096 tokens x 30 heads of 128, in place."""
    x = orc.randn((T * 30, 128), 7041)
    g = orc.randn((128,), 7042, 1.0, 0.1)
    dx = be.array(x)
    be.rms_norm_heads(dx, T * 30, 128, be.array(g), 1e-5)
    want = orc.rms_norm_heads(x, 128, g, 1e-5)
    assert_true_relative(dx.download(), want, np.abs(want), "rms_norm_heads [4096*30,128]")
