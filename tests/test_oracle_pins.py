"""Pins of the CPU oracle (oracle/sd_oracle.c) that do not depend on the
oracle's own formulas:

  * the reference's own known-answer checks, restated: closed forms in double
    for rms_norm / rms_norm_heads_ / rope_ (both conventions) / swiglu, and the
    mean-0 / var-1 invariants of group_norm / layer_norm
    (tests/test_ops.cpp:119-153, :181-257);
  * brute force in float64 (numpy) on small inputs for every other op;
  * invariants: softmax rows sum to 1, are shift-invariant and keep exact
    zeros in the causal tail; RoPE is the identity at position 0 and keeps
    pair norms; add_rows_scaled_ with g = 1 equals add_;
  * an independent library routine (torch.nn.functional in float64) for
    group_norm / layer_norm / rms_norm / softmax / silu;
  * planted mistakes: each pin must FAIL when a plausible bug (dropped eps,
    flipped sign, wrong channel index, exp(+g), missing max subtraction,
    swapped patch axes, a missing transpose) is planted in the oracle.
"""
import math

import numpy as np
import pytest

from tolerances import max_abs


def _x(orc, shape, seed, mean=0.0, std=1.0):
    return orc.randn(shape, seed, mean, std)


# ---------------------------------------------------------------- test_ops.cpp restated
def test_rms_norm_closed_form(orc):  # test_ops.cpp:184-193
    S, H, Dh = 5, 3, 8
    x = _x(orc, (S, H * Dh), 1)
    g = _x(orc, (H * Dh,), 2)
    y = orc.rms_norm(x, g, 1e-6)
    xd = x.astype(np.float64)
    rstd = 1.0 / np.sqrt((xd * xd).sum(1, keepdims=True) / (H * Dh) + 1e-6)
    assert max_abs(y, xd * rstd * g) <= 1e-5


def test_rms_norm_heads_closed_form(orc):  # test_ops.cpp:195-204
    S, H, Dh = 5, 3, 8
    x = _x(orc, (S, H * Dh), 3)
    gd = _x(orc, (Dh,), 4)
    y = orc.rms_norm_heads(x, Dh, gd, 1e-6)
    xd = x.astype(np.float64).reshape(S * H, Dh)
    rstd = 1.0 / np.sqrt((xd * xd).sum(1, keepdims=True) / Dh + 1e-6)
    assert max_abs(y.reshape(S * H, Dh), xd * rstd * gd) <= 1e-5


def _angles(S, Dh):
    return np.array([[s * 10000.0 ** (-2.0 * i / Dh) for i in range(Dh // 2)] for s in range(S)])


def test_rope_rotate_half_closed_form(orc):  # test_ops.cpp:206-226
    S, H, Dh = 5, 3, 8
    x = _x(orc, (S, H * Dh), 5)
    ang = _angles(S, Dh)
    cs = np.concatenate([np.cos(ang), np.cos(ang)], 1).astype(np.float32)
    sn = np.concatenate([np.sin(ang), np.sin(ang)], 1).astype(np.float32)
    y = orc.rope(x, Dh, cs, sn, False).reshape(S, H, Dh)
    xd = x.astype(np.float64).reshape(S, H, Dh)
    a, b = xd[..., : Dh // 2], xd[..., Dh // 2:]
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    assert max_abs(y[..., : Dh // 2], a * c - b * s) <= 1e-5
    assert max_abs(y[..., Dh // 2:], b * c + a * s) <= 1e-5


def test_rope_interleaved_closed_form(orc):  # test_ops.cpp:228-246
    S, H, Dh = 5, 3, 8
    x = _x(orc, (S, H * Dh), 6)
    ang = _angles(S, Dh)
    cs = np.repeat(np.cos(ang), 2, axis=1).astype(np.float32)
    sn = np.repeat(np.sin(ang), 2, axis=1).astype(np.float32)
    y = orc.rope(x, Dh, cs, sn, True).reshape(S, H, Dh)
    xd = x.astype(np.float64).reshape(S, H, Dh)
    a, b = xd[..., 0::2], xd[..., 1::2]
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    assert max_abs(y[..., 0::2], a * c - b * s) <= 1e-5
    assert max_abs(y[..., 1::2], b * c + a * s) <= 1e-5


def test_swiglu_closed_form(orc):  # test_ops.cpp:248-256
    x = _x(orc, (5, 24), 7)
    u = _x(orc, (5, 24), 8)
    gd = x.astype(np.float64)
    assert max_abs(orc.swiglu(x, u), gd / (1 + np.exp(-gd)) * u) <= 1e-5


def test_norm_invariants(orc):  # test_ops.cpp:119-153
    x = _x(orc, (2, 64, 5, 7), 9) * 3.0 + 2.0
    g, b = np.ones(64, np.float32), np.zeros(64, np.float32)
    y = orc.group_norm(x, 32, g, b, 1e-6).astype(np.float64).reshape(2, 32, -1)
    assert np.max(np.abs(y.mean(-1))) <= 1e-3 and np.max(np.abs(y.var(-1) - 1)) <= 1e-3
    z = _x(orc, (3, 7, 64), 10)
    ln = orc.layer_norm(z, g, b, 1e-5).astype(np.float64).reshape(21, 64)
    assert np.max(np.abs(ln.mean(-1))) <= 1e-3 and np.max(np.abs(ln.var(-1) - 1)) <= 1e-3


# ---------------------------------------------------------------- brute force in float64
def test_group_norm_brute_force(orc):
    x = _x(orc, (2, 12, 3, 5), 11, 1.0, 2.0)
    g = _x(orc, (12,), 12, 1.0, 0.3)
    b = _x(orc, (12,), 13, 0.0, 0.3)
    xd = x.astype(np.float64).reshape(2, 4, 3, 15)
    mean = xd.mean(axis=(2, 3), keepdims=True)
    var = ((xd - mean) ** 2).mean(axis=(2, 3), keepdims=True)
    want = ((xd - mean) / np.sqrt(var + 1e-6)).reshape(2, 12, 15) * g[None, :, None] + b[None, :, None]
    got = orc.group_norm(x, 4, g, b, 1e-6).reshape(2, 12, 15)
    assert max_abs(got, want) <= 1e-5
    silu = want / (1 + np.exp(-want))
    assert max_abs(orc.group_norm(x, 4, g, b, 1e-6, silu=True).reshape(2, 12, 15), silu) <= 1e-5


def test_layer_norm_brute_force(orc):
    x = _x(orc, (6, 70), 14, 2.0, 3.0)
    g = _x(orc, (70,), 15, 1.0, 0.3)
    b = _x(orc, (70,), 16)
    xd = x.astype(np.float64)
    m = xd.mean(1, keepdims=True)
    v = ((xd - m) ** 2).mean(1, keepdims=True)
    want = (xd - m) / np.sqrt(v + 1e-5) * g + b
    assert max_abs(orc.layer_norm(x, g, b, 1e-5), want) <= 1e-5


def test_softmax_brute_force_and_invariants(orc):
    x = _x(orc, (17, 33), 17, 0.0, 3.0)
    xd = x.astype(np.float64) * 0.3
    e = np.exp(xd - xd.max(1, keepdims=True))
    want = e / e.sum(1, keepdims=True)
    got = orc.softmax_rows(x, 0.3)
    assert np.max(np.abs(got - want) / want) <= 1e-5
    assert np.max(np.abs(got.sum(1, dtype=np.float64) - 1)) <= 1e-5
    # shift invariance: adding a constant to a row does not change it
    got2 = orc.softmax_rows(x + np.float32(4.0), 0.3)
    assert np.max(np.abs(got2 - want) / want) <= 1e-5
    # causal: row r keeps columns 0..r, the rest are exact zeros
    c = orc.softmax_rows(x, 0.3, causal=True)
    for r in range(17):
        assert np.all(c[r, r + 1:] == 0.0)
        er = np.exp(xd[r, : r + 1] - xd[r, : r + 1].max())
        assert np.max(np.abs(c[r, : r + 1] - er / er.sum())) <= 1e-6
    # large logits do not overflow (max subtraction)
    big = orc.softmax_rows(np.full((2, 8), 200.0, np.float32), 1.0)
    assert np.allclose(big, 1.0 / 8)


def test_broadcasts_brute_force(orc):
    x = _x(orc, (9, 40), 18)
    y = _x(orc, (9, 40), 19)
    v = _x(orc, (40,), 20)
    assert max_abs(orc.mul_rows(x, v), x.astype(np.float64) * v) <= 1e-6
    assert max_abs(orc.add_rows_scaled(x, y, v), x + v.astype(np.float64) * y) <= 1e-6
    assert np.array_equal(orc.add_rows_scaled(x, y, np.ones(40, np.float32)), orc.add(x, y))
    img = _x(orc, (2, 3, 4, 5), 21)
    b = _x(orc, (2, 3), 22)
    assert max_abs(orc.add_channel_bias(img, b), img + b[:, :, None, None].astype(np.float64)) <= 1e-6
    assert max_abs(orc.affine(x, 1.5, -0.25), x.astype(np.float64) * 1.5 - 0.25) <= 1e-6
    assert max_abs(orc.scale(x, 0.37), x.astype(np.float64) * np.float32(0.37)) <= 1e-6


def test_activations_brute_force(orc):
    x = _x(orc, (1000,), 23, 0.0, 3.0)
    xd = x.astype(np.float64)
    from math import erf

    assert max_abs(orc.silu(x), xd / (1 + np.exp(-xd))) <= 1e-5
    assert max_abs(orc.tanh(x), np.tanh(xd)) <= 1e-6
    assert max_abs(orc.gelu(x), 0.5 * xd * (1 + np.vectorize(erf)(xd / math.sqrt(2)))) <= 1e-5
    assert max_abs(orc.quick_gelu(x), xd / (1 + np.exp(-1.702 * xd))) <= 1e-5
    gg = _x(orc, (6, 40), 24)
    a, g = gg[:, :20].astype(np.float64), gg[:, 20:].astype(np.float64)
    assert max_abs(orc.geglu(gg), a * 0.5 * g * (1 + np.vectorize(erf)(g / math.sqrt(2)))) <= 1e-5


def test_fused_compositions_brute_force(orc):
    x = _x(orc, (7, 64), 25)
    r = _x(orc, (7, 64), 26)
    w = _x(orc, (64,), 27, 1.0, 0.1)
    s, y = orc.add_rms_norm(x, r, w, 1e-6)
    sd = x.astype(np.float64) + r
    assert max_abs(s, sd) <= 1e-6
    assert max_abs(y, sd / np.sqrt((sd * sd).mean(1, keepdims=True) + 1e-6) * w) <= 1e-5
    sc, sh, gt = _x(orc, (64,), 28, 0, 0.2), _x(orc, (64,), 29, 0, 0.2), _x(orc, (64,), 30, 0, 0.2)
    res, yy = orc.ln_modulate_gate(x, r, sc, sh, gt, 1e-6)
    xd = x.astype(np.float64)
    ln = (xd - xd.mean(1, keepdims=True)) / np.sqrt(xd.var(1, keepdims=True) + 1e-6)
    yw = ln * (1 + sc.astype(np.float64)) + sh
    assert max_abs(yy, yw) <= 1e-5
    assert max_abs(res, r + np.tanh(gt.astype(np.float64)) * yw) <= 1e-5


def test_rope_tables_and_invariants(orc):
    pos = np.array([[0, h, w] for h in range(8) for w in range(8)], np.int32)
    cs, sn = orc.rope_tables_3axis(pos, [32, 48, 48], 128, 256.0)
    # closed form of zimage.cpp:71-88: angle_k = (float)(pos * theta^(-2k/da)),
    # each angle stored at (2k, 2k+1) of its axis block
    off = 0
    for a, da in enumerate([32, 48, 48]):
        freq = 1.0 / 256.0 ** (np.arange(da // 2) * 2.0 / da)
        ang = (pos[:, a:a + 1].astype(np.float64) * freq).astype(np.float32).astype(np.float64)
        assert max_abs(cs[:, off:off + da:2], np.cos(ang)) <= 1e-6
        assert max_abs(cs[:, off + 1:off + da:2], np.cos(ang)) <= 1e-6
        assert max_abs(sn[:, off:off + da:2], np.sin(ang)) <= 1e-6
        off += da
    x = _x(orc, (1, 64, 2 * 128), 31)
    y = orc.rope(x, 128, cs, sn, True)
    assert np.array_equal(y[0, 0], x[0, 0])  # position (0, 0, 0): identity
    pn = lambda t: np.hypot(t[..., 0::2].astype(np.float64), t[..., 1::2])
    assert max_abs(pn(y), pn(x)) <= 1e-5  # rotations keep pair norms
    c2, s2 = orc.rope_tables_half(16, 64, 1e6)
    i = np.arange(32)
    a2 = np.arange(16)[:, None] * 1e6 ** (-2.0 * i / 64)
    assert max_abs(c2[:, :32], np.cos(a2)) <= 1e-7 and np.array_equal(c2[:, :32], c2[:, 32:])


def test_torch_library_cross_check(orc):
    """Independent library routines (not the reference) in float64."""
    torch = pytest.importorskip("torch")
    F = torch.nn.functional
    x = _x(orc, (2, 64, 6, 6), 32, 0.5, 2.0)
    g = _x(orc, (64,), 33, 1.0, 0.1)
    b = _x(orc, (64,), 34, 0.0, 0.1)
    t = lambda a: torch.from_numpy(a.astype(np.float64))
    want = F.group_norm(t(x), 32, t(g), t(b), 1e-6).numpy()
    assert max_abs(orc.group_norm(x, 32, g, b, 1e-6), want) <= 1e-5
    z = _x(orc, (5, 64), 35)
    assert max_abs(orc.layer_norm(z, g, b, 1e-5), F.layer_norm(t(z), (64,), t(g), t(b), 1e-5).numpy()) <= 1e-5
    assert max_abs(orc.rms_norm(z, g, 1e-6), F.rms_norm(t(z), (64,), t(g), 1e-6).numpy()) <= 1e-5
    assert max_abs(orc.softmax_rows(z, 0.7), F.softmax(t(z) * 0.7, -1).numpy()) <= 1e-6
    assert max_abs(orc.silu(z), F.silu(t(z)).numpy()) <= 1e-6


# ---------------------------------------------------------------- layout ops
# Each layout op is a permutation/duplication of its input. The pins state it
# independently as a numpy reshape/transpose/repeat (library routines, not the
# reference's loops), plus the round trips the reference relies on.
def test_patchify_matches_reshape_transpose(orc):
    for Cc, H, W, p in ((16, 6, 8, 2), (3, 9, 12, 3), (5, 4, 4, 4), (2, 5, 7, 1)):
        x = _x(orc, (1, Cc, H, W), 70 + Cc + p)
        want = x.reshape(Cc, H // p, p, W // p, p).transpose(1, 3, 2, 4, 0).reshape((H // p) * (W // p), p * p * Cc)
        tok = orc.patchify(x, p)
        assert np.array_equal(tok, want), (Cc, H, W, p)
        assert np.array_equal(orc.unpatchify(tok, Cc, H, W, p), x), "unpatchify(patchify(x)) != x"


def test_nchw_nlc_match_transpose(orc):
    for N, Cc, H, W in ((2, 3, 4, 5), (1, 64, 16, 24), (3, 7, 1, 9)):
        x = _x(orc, (N, Cc, H, W), 80 + Cc)
        nlc = orc.nchw_to_nlc(x)
        assert np.array_equal(nlc, x.reshape(N, Cc, H * W).transpose(0, 2, 1))
        back = orc.nlc_to_nchw(nlc, H, W)
        assert np.array_equal(back, x), "nlc_to_nchw(nchw_to_nlc(x)) != x"


def test_upsample_and_concat_match_numpy(orc):
    x = _x(orc, (2, 3, 4, 5), 90)
    assert np.array_equal(orc.upsample_nearest2x(x), np.repeat(np.repeat(x, 2, axis=2), 2, axis=3))
    b = _x(orc, (2, 2, 4, 5), 91)
    assert np.array_equal(orc.concat_channels(x, b), np.concatenate([x, b], axis=1))
    e = np.zeros((2, 0, 4, 5), np.float32)
    assert np.array_equal(orc.concat_channels(e, b), b)


# ---------------------------------------------------------------- planted mistakes
PLANTS = {
    1: ("rope interleaved sign", test_rope_interleaved_closed_form),
    2: ("rms_norm drops eps", None),
    3: ("softmax without max subtraction", test_softmax_brute_force_and_invariants),
    4: ("group_norm wrong gamma channel", test_group_norm_brute_force),
    5: ("swiglu exp(+g)", test_swiglu_closed_form),
    6: ("patchify with ph and pw swapped", test_patchify_matches_reshape_transpose),
    7: ("nlc_to_nchw without the transpose", test_nchw_nlc_match_transpose),
}


def _eps_sensitive_rms(orc):
    # eps matters when a row is (nearly) zero: rms_norm of zeros with eps
    # must give 0, and of tiny values must follow the closed form.
    x = np.full((2, 8), 1e-4, np.float32)
    y = orc.rms_norm(x, None, 1e-6)
    want = x.astype(np.float64) / np.sqrt(1e-8 + 1e-6)
    assert max_abs(y, want) <= 1e-5


@pytest.mark.parametrize("which", sorted(PLANTS))
def test_pins_catch_planted_mistakes(orc, which):
    name, pin = PLANTS[which]
    if pin is None:
        pin = _eps_sensitive_rms
    pin(orc)  # passes on the clean oracle
    orc.plant(which)
    try:
        with pytest.raises(AssertionError):
            pin(orc)
    finally:
        orc.plant(0)
