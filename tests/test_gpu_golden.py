"""backend_hip against the reference's own outputs (golden fixtures written by
tests/golden/make_golden.py from the compiled reference tensor.cpp):

  * every op at small shapes, element by element;
  * every BASELINE config at FULL size, through size-independent summaries of
    the output: float64 checksums (sum, sum of squares, sum of |y|) and a
    strided sample of elements compared one by one.

Tolerances as tolerances.py (elementwise max-abs 1e-5; reductions and softmax
relative 1e-4).
"""
import math
import os

import numpy as np
import pytest

from test_golden import inputs
from tolerances import assert_elementwise, assert_reduction, assert_softmax

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
T, D, F = 4096, 3840, 10240
STRIDE = 9973


@pytest.fixture(scope="module")
def small():
    return dict(np.load(os.path.join(GOLDEN, "ops_small.npz"), allow_pickle=False))


@pytest.fixture(scope="module")
def cfg():
    return dict(np.load(os.path.join(GOLDEN, "configs.npz"), allow_pickle=False))


def test_small_ops_vs_reference(be, orc, small):
    i = inputs(orc, small)
    A = be.array
    n = lambda a: a.size

    def run_new(fn, shape):
        y = be.empty(shape)
        fn(y)
        return y.download()

    got = {}
    got["rms_norm"] = run_new(lambda y: be.rms_norm(A(i["x"]), y, 5, 24, A(i["g"]), 1e-6), (5, 24))
    got["layer_norm"] = run_new(lambda y: be.layer_norm(A(i["z"]), y, 21, 64, A(i["g64"]), A(i["b64"]), 1e-5), (3, 7, 64))
    got["layer_norm_noaffine"] = run_new(lambda y: be.layer_norm(A(i["z"]), y, 21, 64, None, None, 1e-5), (3, 7, 64))
    got["group_norm"] = run_new(lambda y: be.group_norm(A(i["img"]), y, 2, 64, 35, 32, A(i["g64"]), A(i["b64"]), 1e-6),
                                (2, 64, 5, 7))
    got["group_norm_silu"] = run_new(
        lambda y: be.group_norm(A(i["img"]), y, 2, 64, 35, 32, A(i["g64"]), A(i["b64"]), 1e-6, silu=True), (2, 64, 5, 7))
    h = A(i["x"])
    be.rms_norm_heads(h, 15, 8, A(i["gd"]), 1e-6)
    got["rms_norm_heads"] = h.download().reshape(15, 8)
    cs, sn = A(small["rope_cos"]), A(small["rope_sin"])
    for key, inter in (("rope_half", False), ("rope_inter", True)):
        r = A(i["xr"])
        be.rope(r, 1, 5, 24, 8, cs, sn, inter)
        got[key] = r.download()
    got["swiglu"] = run_new(lambda y: be.swiglu(A(i["xr"]), A(i["u"]), y, 120), (1, 5, 24))
    got["geglu"] = run_new(lambda y: be.geglu(A(i["gg"]), y, 6, 20), (6, 20))
    for op in ("silu", "tanh", "gelu", "quick_gelu"):
        a = A(i["a"])
        getattr(be, op)(a, 1000)
        got[op] = a.download()
    a = A(i["a"])
    be.add(a, A(i["b"]), 1000)
    got["add"] = a.download()
    a = A(i["a"])
    be.scale(a, 0.37, 1000)
    got["scale"] = a.download()
    a = A(i["a"])
    be.affine(a, 1.5, -0.25, 1000)
    got["affine"] = a.download()
    m = A(i["m"])
    be.mul_rows(m, A(i["v"]), 4, 6)
    got["mul_rows"] = m.download()
    m = A(i["m"])
    be.add_rows_scaled(m, A(i["my"]), A(i["v"]), 4, 6)
    got["add_rows_scaled"] = m.download()
    c = A(i["cimg"])
    be.add_channel_bias(c, A(i["cb"]), 2, 3, 20)
    got["add_channel_bias"] = c.download()
    s = A(i["sm"])
    be.softmax_rows(s, 54, 9, 0.35, True)
    got["softmax_causal"] = s.download()
    s = A(i["sm2"])
    be.softmax_rows(s, 33, 100, 0.125, False)
    got["softmax"] = s.download()
    res, y = A(i["lr"]), be.empty((7, 64))
    be.ln_modulate_gate(A(i["lx"]), res, A(i["lsc"]), A(i["lsh"]), A(i["lgt"]), y, 7, 64, 1e-6)
    got["ln_modulate_gate_res"], got["ln_modulate_gate_y"] = res.download(), y.download()
    xs, y = A(i["lx"]), be.empty((7, 64))
    be.add_rms_norm(xs, A(i["lr"]), y, 7, 64, A(i["g64"]), 1e-6)
    got["add_rms_norm_sum"], got["add_rms_norm_y"] = xs.download(), y.download()

    img, img2 = A(i["cimg"]), A(i["img2"])
    got["upsample_nearest2x"] = run_new(lambda y: be.upsample_nearest2x(img, y, 6, 4, 5), (2, 3, 8, 10))
    got["concat_channels"] = run_new(lambda y: be.concat_channels(img, img2, y, 2, 3, 2, 20), (2, 5, 4, 5))
    nlc = be.empty((2, 20, 3))
    be.nchw_to_nlc(img, nlc, 2, 3, 20)
    got["nchw_to_nlc"] = nlc.download()
    got["nlc_to_nchw"] = run_new(lambda y: be.nlc_to_nchw(nlc, y, 2, 3, 20), (2, 3, 4, 5))
    tok = be.empty((12, 64))
    be.patchify(A(i["lat"]), tok, 16, 6, 8, 2)
    got["patchify2d"] = tok.download()
    got["unpatchify2d"] = run_new(lambda y: be.unpatchify(tok, y, 16, 6, 8, 2), (1, 16, 6, 8))
    exact = {"upsample_nearest2x", "concat_channels", "nchw_to_nlc", "nlc_to_nchw", "patchify2d", "unpatchify2d"}

    reductions = {"rms_norm", "layer_norm", "layer_norm_noaffine", "group_norm", "group_norm_silu", "rms_norm_heads",
                  "ln_modulate_gate_res", "ln_modulate_gate_y", "add_rms_norm_y"}
    for k, v in got.items():
        want = small[k]
        if k in exact:
            assert v.shape == want.shape and np.array_equal(v, want), k
        elif k.startswith("softmax"):
            assert_softmax(v, want, k)
        elif k in reductions:
            assert_reduction(v, want, k)
        else:
            assert_elementwise(v, want, k)
    assert n(got["add"]) == 1000


def _compare_summary(cfg, name, y, kind):
    """Checksums within relative 1e-5 and the strided sample element-wise."""
    want = cfg[f"{name}/sum"]
    y64 = y.astype(np.float64).reshape(-1)
    got = np.array([y64.sum(), (y64 * y64).sum(), np.abs(y64).sum(), y64.size])
    assert got[3] == want[3]
    assert abs(got[1] - want[1]) <= 1e-5 * abs(want[1]), f"{name} sum of squares {got[1]} vs {want[1]}"
    assert abs(got[2] - want[2]) <= 1e-5 * abs(want[2]), f"{name} sum |y| {got[2]} vs {want[2]}"
    assert abs(got[0] - want[0]) <= 1e-5 * want[2], f"{name} sum {got[0]} vs {want[0]}"
    sample = y.reshape(-1)[::STRIDE]
    {"elementwise": assert_elementwise, "reduction": assert_reduction, "softmax": assert_softmax}[kind](
        sample, cfg[f"{name}/sample"], name)


def test_config1_add_rms_norm(be, orc, cfg):
    x, r = orc.randn((T, D), 101), orc.randn((T, D), 102)
    w = orc.randn((D,), 103, 1.0, 0.1)
    dx, dy = be.array(x), be.empty((T, D))
    be.add_rms_norm(dx, be.array(r), dy, T, D, be.array(w), 1e-6)
    _compare_summary(cfg, "c1_sum", dx.download(), "elementwise")
    _compare_summary(cfg, "c1_norm", dy.download(), "reduction")


def test_config2_swiglu(be, orc, cfg):
    g, u = orc.randn((T, F), 104, 0.0, 1.5), orc.randn((T, F), 105, 0.0, 1.5)
    dy = be.empty((T, F))
    be.swiglu(be.array(g), be.array(u), dy, T * F)
    _compare_summary(cfg, "c2_swiglu", dy.download(), "elementwise")


def test_config3_rope(be, orc, cfg):
    pos = np.array([[0, h, w] for h in range(64) for w in range(64)], np.int32)
    cs, sn = orc.rope_tables_3axis(pos, [32, 48, 48], 128, 256.0)
    q = be.array(orc.randn((1, T, D), 106))
    be.rope(q, 1, T, D, 128, be.array(cs), be.array(sn), True)
    _compare_summary(cfg, "c3_rope_q", q.download(), "elementwise")


@pytest.mark.parametrize("tag,shape,eps,seed", [("c4a", (1, 512, 128, 128), 1e-6, 107),
                                                ("c4b", (1, 128, 1024, 1024), 1e-6, 108),
                                                ("c4c", (2, 320, 64, 64), 1e-5, 109),
                                                ("c4d", (2, 1280, 8, 8), 1e-5, 110)])
def test_config4_group_norm_silu(be, orc, cfg, tag, shape, eps, seed):
    x = orc.randn(shape, seed, 0.0, 2.0)
    gm = orc.randn((shape[1],), seed + 1000, 1.0, 0.1)
    bt = orc.randn((shape[1],), seed + 2000, 0.0, 0.1)
    dy = be.empty(shape)
    N, C = shape[0], shape[1]
    be.group_norm(be.array(x), dy, N, C, x.size // (N * C), 32, be.array(gm), be.array(bt), eps, silu=True)
    _compare_summary(cfg, f"{tag}_gn_silu", dy.download(), "reduction")


def test_config5a_ln_modulate_gate(be, orc, cfg):
    x, res = orc.randn((T, D), 111), orc.randn((T, D), 112)
    sc, sh, gt = (orc.randn((D,), 113 + i, 0.0, 0.2) for i in range(3))
    dres = be.array(res)
    be.ln_modulate_gate(be.array(x), dres, be.array(sc), be.array(sh), be.array(gt), None, T, D, 1e-6)
    _compare_summary(cfg, "c5a_res", dres.download(), "reduction")


def test_config5b_softmax(be, orc, cfg):
    sm = orc.randn((30 * T, T), 116, 0.0, 3.0)
    d = be.array(sm)
    del sm
    be.softmax_rows(d, 30 * T, T, 1.0 / math.sqrt(128.0), False)
    _compare_summary(cfg, "c5b_softmax", d.download(), "softmax")
