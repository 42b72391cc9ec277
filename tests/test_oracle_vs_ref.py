"""The oracle (C restatement) against the compiled reference tensor library
(oracle/_ref, the reference's own src/tensor.cpp): bit-for-bit equality on
seeded random inputs, for every op on the path, at tiny, odd and mid-size
shapes. Skipped where oracle/_ref was not built.
"""
import os

import numpy as np
import pytest


def _eq(a, b, what):
    assert a.shape == b.shape, what
    assert np.array_equal(a, b), f"{what}: max diff {np.max(np.abs(a - b)):.3e}"


@pytest.mark.parametrize("rows,C", [(21, 64), (3, 70), (37, 3840), (1, 1)])
def test_norms_bitexact(orc, ref, rows, C):
    x = orc.randn((rows, C), 100 + C, 1.0, 2.0)
    g = orc.randn((C,), 200 + C, 1.0, 0.1)
    b = orc.randn((C,), 300 + C, 0.0, 0.1)
    _eq(orc.rms_norm(x, g, 1e-6), ref.rms_norm(x, g, 1e-6), "rms_norm")
    _eq(orc.rms_norm(x, None, 1e-5), ref.rms_norm(x, None, 1e-5), "rms_norm no gamma")
    for gg, bb in ((g, b), (None, None), (g, None), (None, b)):
        _eq(orc.layer_norm(x, gg, bb, 1e-5), ref.layer_norm(x, gg, bb, 1e-5), "layer_norm")
    s1, y1 = orc.add_rms_norm(x, x[::-1].copy(), g, 1e-6)
    s2, y2 = ref.add_rms_norm(x, x[::-1].copy(), g, 1e-6)
    _eq(s1, s2, "add_rms_norm sum")
    _eq(y1, y2, "add_rms_norm norm")


@pytest.mark.parametrize("groups,dim", [(15, 8), (64, 128), (9, 30)])
def test_rms_norm_heads_bitexact(orc, ref, groups, dim):
    x = orc.randn((groups, dim), 7 + dim)
    g = orc.randn((dim,), 8 + dim, 1.0, 0.1)
    _eq(orc.rms_norm_heads(x, dim, g, 1e-5), ref.rms_norm_heads(x, dim, g, 1e-5), "rms_norm_heads")


@pytest.mark.parametrize("shape,groups", [((2, 64, 5, 7), 32), ((1, 128, 32, 32), 32), ((2, 96, 7, 3), 8)])
def test_group_norm_bitexact(orc, ref, shape, groups):
    x = orc.randn(shape, 11, 0.0, 2.0)
    g = orc.randn((shape[1],), 12, 1.0, 0.1)
    b = orc.randn((shape[1],), 13, 0.0, 0.1)
    _eq(orc.group_norm(x, groups, g, b, 1e-6), ref.group_norm(x, groups, g, b, 1e-6), "group_norm")
    _eq(orc.group_norm(x, groups, g, b, 1e-5, silu=True), ref.group_norm(x, groups, g, b, 1e-5, silu=True),
        "group_norm+silu")


@pytest.mark.parametrize("rows,cols", [(9, 9), (40, 37), (16, 4096)])
@pytest.mark.parametrize("causal", [False, True])
def test_softmax_bitexact(orc, ref, rows, cols, causal):
    x = orc.randn((rows, cols), 21 + cols, 0.0, 3.0)
    _eq(orc.softmax_rows(x, 0.0883883, causal), ref.softmax_rows(x, 0.0883883, causal), "softmax")


@pytest.mark.parametrize("blocks,p,cols", [(3, 37, 37), (4, 9, 9), (2, 16, 40), (5, 1, 7), (3, 13, 4096)])
@pytest.mark.parametrize("causal", [False, True])
def test_softmax_period_bitexact(orc, ref, blocks, p, cols, causal):
    """The batched form (rows in blocks of `period`, the causal mask restarting
    at each block: backend_cuda.cu:351-367, one block per attention head) is
    the reference's softmax_rows_ (tensor.cpp:752-769) applied to each block
    of p rows on its own, bit for bit."""
    x = orc.randn((blocks * p, cols), 31 + p + cols, 0.0, 3.0)
    want = np.concatenate([ref.softmax_rows(x[i * p:(i + 1) * p], 0.0883883, causal) for i in range(blocks)])
    _eq(orc.softmax_rows(x, 0.0883883, causal, period=p), want, f"softmax period {p}")


@pytest.mark.parametrize("interleaved", [True, False])
def test_rope_bitexact(orc, ref, interleaved):
    S = 64
    pos = np.array([[0, h, w] for h in range(8) for w in range(8)], np.int32)
    if interleaved:
        cs, sn = orc.rope_tables_3axis(pos, [32, 48, 48], 128, 256.0)
    else:
        cs, sn = orc.rope_tables_half(S, 128, 1e6)
    x = orc.randn((2, S, 3 * 128), 31)
    _eq(orc.rope(x, 128, cs, sn, interleaved), ref.rope(x, 128, cs, sn, interleaved), "rope")


def test_elementwise_bitexact(orc, ref):
    x = orc.randn((33, 100), 41, 0.0, 3.0)
    u = orc.randn((33, 100), 42, 0.0, 1.5)
    v = orc.randn((100,), 43, 0.0, 0.2)
    _eq(orc.swiglu(x, u), ref.swiglu(x, u), "swiglu")
    _eq(orc.geglu(x), ref.geglu(x), "geglu")
    for op in ("silu", "tanh", "gelu", "quick_gelu"):
        _eq(getattr(orc, op)(x), getattr(ref, op)(x), op)
    _eq(orc.add(x, u), ref.add(x, u), "add")
    _eq(orc.scale(x, 0.37), ref.scale(x, 0.37), "scale")
    _eq(orc.affine(x, 1.5, -0.25), ref.affine(x, 1.5, -0.25), "affine")
    _eq(orc.mul_rows(x, v), ref.mul_rows(x, v), "mul_rows")
    _eq(orc.add_rows_scaled(x, u, v), ref.add_rows_scaled(x, u, v), "add_rows_scaled")
    img = orc.randn((2, 3, 4, 5), 44)
    b = orc.randn((2, 3), 45)
    _eq(orc.add_channel_bias(img, b), ref.add_channel_bias(img, b), "add_channel_bias")


@pytest.mark.parametrize("shift", [True, False])
def test_ln_modulate_gate_bitexact(orc, ref, shift):
    x = orc.randn((12, 3840), 51)
    r = orc.randn((12, 3840), 52)
    sc = orc.randn((3840,), 53, 0.0, 0.2)
    sh = orc.randn((3840,), 54, 0.0, 0.2) if shift else None
    gt = orc.randn((3840,), 55, 0.0, 0.2)
    a = orc.ln_modulate_gate(x, r, sc, sh, gt, 1e-6)
    b = ref.ln_modulate_gate(x, r, sc, sh, gt, 1e-6)
    _eq(a[0], b[0], "res")
    _eq(a[1], b[1], "y")


@pytest.mark.parametrize("N,Cc,H,W", [(2, 3, 4, 5), (1, 64, 16, 24), (3, 5, 7, 1), (1, 16, 6, 8)])
def test_layout_bitexact(orc, ref, N, Cc, H, W):
    x = orc.randn((N, Cc, H, W), 61 + Cc)
    x2 = orc.randn((N, Cc + 1, H, W), 62 + Cc)
    _eq(orc.upsample_nearest2x(x), ref.upsample_nearest2x(x), "upsample_nearest2x")
    _eq(orc.concat_channels(x, x2), ref.concat_channels(x, x2), "concat_channels")
    nlc = orc.nchw_to_nlc(x)
    _eq(nlc, ref.nchw_to_nlc(x), "nchw_to_nlc")
    _eq(orc.nlc_to_nchw(nlc, H, W), ref.nlc_to_nchw(nlc, H, W), "nlc_to_nchw")
    for p in (1, 2, 3):
        if H % p == 0 and W % p == 0 and N == 1:
            tok = orc.patchify(x, p)
            _eq(tok, ref.patchify(x, p), f"patchify p={p}")
            _eq(orc.unpatchify(tok, Cc, H, W, p), ref.unpatchify(tok, Cc, H, W, p), f"unpatchify p={p}")


@pytest.mark.parametrize("interleaved", [True, False])
def test_qknorm_rope_bitexact(orc, ref, interleaved):
    """The fused QK-norm + RoPE oracle equals the reference's op sequence
    (zimage.cpp:117-120, qwen3.cpp:59-62) run through its own tensor.cpp."""
    S, dim = 16, 64
    q = orc.randn((2, S, 4 * dim), 71, 0.5, 2.0)
    k = orc.randn((2, S, 2 * dim), 72, 0.5, 2.0)
    gq = orc.randn((dim,), 73, 1.0, 0.1)
    gk = orc.randn((dim,), 74, 1.0, 0.1)
    ang = orc.randn((S, dim), 75, 0.0, 1.0)
    cs, sn = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    q2, k2 = orc.qknorm_rope(q, k, dim, gq, gk, 1e-5, cs, sn, interleaved)
    rq = ref.rope(ref.rms_norm_heads(q, dim, gq, 1e-5).reshape(q.shape), dim, cs, sn, interleaved)
    rk = ref.rope(ref.rms_norm_heads(k, dim, gk, 1e-5).reshape(k.shape), dim, cs, sn, interleaved)
    _eq(q2, rq, "qknorm_rope q")
    _eq(k2, rk, "qknorm_rope k")


REF_V4 = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle", "_ref", "libsdref_v4.so")


def _avx512():
    try:
        flags = next(l for l in open("/proc/cpuinfo") if l.startswith("flags")).split()
    except Exception:
        return False
    return all(f in flags for f in ("avx512f", "avx512bw", "avx512cd", "avx512dq", "avx512vl"))


@pytest.mark.skipif(not (os.path.exists(REF_V4) and _avx512()), reason="no AVX-512 build of the reference or host")
def test_reference_v4_build_equals_v3(orc, ref):
    """The AVX-512 build of the reference (bench.py's CPU baseline on AVX-512
    hosts) computes the same bits as the x86-64-v3 build the parity tests
    pin, on every op the benchmark times."""
    from oracle import Reference

    r4 = Reference(REF_V4)
    x = orc.randn((64, 3840), 91)
    w = orc.randn((3840,), 92, 1.0, 0.1)
    g, u = orc.randn((64, 3840), 93, 0.0, 1.5), orc.randn((64, 3840), 94, 0.0, 1.5)
    _eq(r4.rms_norm(x, w, 1e-6), ref.rms_norm(x, w, 1e-6), "rms_norm v4")
    _eq(r4.layer_norm(x, None, None, 1e-6), ref.layer_norm(x, None, None, 1e-6), "layer_norm v4")
    _eq(r4.swiglu(g, u), ref.swiglu(g, u), "swiglu v4")
    _eq(r4.softmax_rows(x, 0.0883883), ref.softmax_rows(x, 0.0883883), "softmax v4")
    xg = orc.randn((1, 64, 32, 32), 95, 0.0, 2.0)
    gg, bb = orc.randn((64,), 96, 1.0, 0.1), orc.randn((64,), 97, 0.0, 0.1)
    _eq(r4.group_norm(xg, 32, gg, bb, 1e-6, silu=True), ref.group_norm(xg, 32, gg, bb, 1e-6, silu=True), "gn v4")
