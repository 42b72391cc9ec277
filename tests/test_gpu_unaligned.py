"""GPU tests of every op on operands that start 4 bytes past a 16-byte
boundary, through the C ABI.

The launchers take their float4 kernels only for 16-byte aligned operands;
a pointer into the middle of a tensor (a row slice, an offset view) sends the
same shapes to the scalar or generic kernels. Shapes here are ones whose
aligned form takes the vector kernels, so each case checks the dispatch on
alignment as well as the fallback kernel, against the oracle with the usual
tolerances.
"""
import math

import numpy as np
import pytest

import sdhip
from oracle import bf16_to_f32, f32_to_bf16
from tolerances import assert_elementwise, assert_gemm, assert_reduction, assert_softmax

pytestmark = pytest.mark.gpu
ATTN_TOL = 1e-4  # max-abs, as tests/test_gpu_attention.py (unit-variance inputs)


class Off:
    """A device copy of `a` that starts one float past an aligned block."""

    def __init__(self, be, a):
        a = np.ascontiguousarray(a, np.float32)
        self.shape = a.shape
        self.base = be.empty((a.size + 1,))
        self.view = sdhip.DArray(be, (a.size,), ptr=self.base.ptr + 4, owned=False)
        self.view.keep = self.base  # the block lives as long as the view (Off(...).view as an argument)
        self.view.upload(a.reshape(-1))

    def get(self):
        return self.view.download().reshape(self.shape)


def test_streaming_unaligned(be, orc):
    n = 4096 + 3
    g, u = orc.randn((n,), 3001, 0.0, 1.5), orc.randn((n,), 3002, 0.0, 1.5)
    dg, du, dy = Off(be, g), Off(be, u), Off(be, np.zeros(n))
    be.swiglu(dg.view, du.view, dy.view, n)
    assert_elementwise(dy.get(), orc.swiglu(g, u), "swiglu unaligned")
    for op in ("silu", "tanh", "gelu", "quick_gelu"):
        d = Off(be, g)
        getattr(be, op)(d.view, n)
        assert_elementwise(d.get(), getattr(orc, op)(g), f"{op} unaligned")
    d = Off(be, g)
    be.add(d.view, du.view, n)
    assert_elementwise(d.get(), orc.add(g, u), "add unaligned")
    d = Off(be, g)
    be.affine(d.view, 1.5, -0.25, n)
    assert_elementwise(d.get(), orc.affine(g, 1.5, -0.25), "affine unaligned")
    x = orc.randn((12, 512), 3003)
    dx, dy = Off(be, x), Off(be, np.zeros((12, 256)))
    be.geglu(dx.view, dy.view, 12, 256)
    assert_elementwise(dy.get(), orc.geglu(x), "geglu unaligned")


def test_row_norms_unaligned(be, orc):
    rows, C = 37, 3840
    x, r = orc.randn((rows, C), 3011), orc.randn((rows, C), 3012)
    g, b = orc.randn((C,), 3013, 1.0, 0.1), orc.randn((C,), 3014, 0.0, 0.1)
    dg, db = Off(be, g), Off(be, b)
    dx, dy = Off(be, x), Off(be, np.zeros((rows, C)))
    be.rms_norm(dx.view, dy.view, rows, C, dg.view, 1e-6)
    assert_reduction(dy.get(), orc.rms_norm(x, g, 1e-6), "rms_norm unaligned")
    be.layer_norm(dx.view, dy.view, rows, C, dg.view, db.view, 1e-6)
    assert_reduction(dy.get(), orc.layer_norm(x, g, b, 1e-6), "layer_norm unaligned")
    dr = Off(be, r)
    be.add_rms_norm(dx.view, dr.view, dy.view, rows, C, dg.view, 1e-6)
    s_want, y_want = orc.add_rms_norm(x, r, g, 1e-6)
    assert_elementwise(dx.get(), s_want, "add_rms_norm sum unaligned")
    assert_reduction(dy.get(), y_want, "add_rms_norm unaligned")
    sc, sh, gt = (orc.randn((C,), 3015 + i, 0.0, 0.2) for i in range(3))
    dx, dres, dyo = Off(be, x), Off(be, r), Off(be, np.zeros((rows, C)))
    be.ln_modulate_gate(dx.view, dres.view, Off(be, sc).view, Off(be, sh).view, Off(be, gt).view, dyo.view, rows, C,
                        1e-6)
    res_want, y_want = orc.ln_modulate_gate(x, r, sc, sh, gt, 1e-6)
    assert_reduction(dyo.get(), y_want, "ln_modulate_gate y unaligned")
    assert_reduction(dres.get(), res_want, "ln_modulate_gate res unaligned")
    h = orc.randn((300, 128), 3018)
    gh = orc.randn((128,), 3019, 1.0, 0.1)
    dh = Off(be, h)
    be.rms_norm_heads(dh.view, 300, 128, Off(be, gh).view, 1e-5)
    assert_reduction(dh.get(), orc.rms_norm_heads(h, 128, gh, 1e-5), "rms_norm_heads unaligned")


def test_fused_block_ops_unaligned(be, orc):
    rows, C = 21, 3840
    x, a = orc.randn((rows, C), 3021), orc.randn((rows, C), 3022, 0.0, 3.0)
    g, s = orc.randn((C,), 3023, 1.0, 0.1), orc.randn((C,), 3024, 1.0, 0.3)
    dx, dg, ds = Off(be, x), Off(be, g), Off(be, s)
    y16 = be.array(np.zeros(rows * C, np.uint16))
    be.rms_norm_modulate_bf16(dx.view, y16, rows, C, dg.view, ds.view, 1e-5)
    want = orc.mul_rows(orc.rms_norm(x, g, 1e-5), s)
    got = bf16_to_f32(y16.download()).reshape(rows, C)
    assert np.max(np.abs(got - want) / np.maximum(np.abs(want), 1e-30)) <= 2.0 ** -8
    be.rms_norm_gated_add(dx.view, Off(be, a).view, rows, C, dg.view, ds.view, 1e-5)
    assert_reduction(dx.get(), orc.add_rows_scaled(x, orc.rms_norm(a, g, 1e-5), s), "rms_norm_gated_add unaligned")


def test_softmax_unaligned(be, orc):
    for rows, cols, causal in ((64, 4096, False), (33, 4096, True), (50, 100, True)):
        x = orc.randn((rows, cols), 3031, 0.0, 3.0)
        d = Off(be, x)
        be.softmax_rows(d.view, rows, cols, 1.0 / math.sqrt(128.0), causal)
        assert_softmax(d.get(), orc.softmax_rows(x, 1.0 / math.sqrt(128.0), causal), f"softmax [{rows},{cols}] unaligned")


def test_broadcasts_unaligned(be, orc):
    rows, dim = 33, 3840
    x, y = orc.randn((rows, dim), 3041), orc.randn((rows, dim), 3042)
    v = orc.randn((dim,), 3043, 1.0, 0.2)
    dx, dv = Off(be, x), Off(be, v)
    be.mul_rows(dx.view, dv.view, rows, dim)
    assert_elementwise(dx.get(), orc.mul_rows(x, v), "mul_rows unaligned")
    dx = Off(be, x)
    be.add_rows_scaled(dx.view, Off(be, y).view, dv.view, rows, dim)
    assert_elementwise(dx.get(), orc.add_rows_scaled(x, y, v), "add_rows_scaled unaligned")
    xb = orc.randn((2, 320, 16, 16), 3044)
    b = orc.randn((2, 320), 3045)
    dx = Off(be, xb)
    be.add_channel_bias(dx.view, Off(be, b).view, 2, 320, 256)
    assert_elementwise(dx.get(), orc.add_channel_bias(xb, b), "add_channel_bias unaligned")


def test_group_norm_unaligned(be, orc):
    for shape in ((1, 64, 32, 32), (2, 320, 16, 16)):
        x = orc.randn(shape, 3051, 0.5, 2.0)
        g, b = orc.randn((shape[1],), 3052, 1.0, 0.1), orc.randn((shape[1],), 3053, 0.0, 0.1)
        dx, dy = Off(be, x), Off(be, np.zeros(shape))
        be.group_norm(dx.view, dy.view, shape[0], shape[1], shape[2] * shape[3], 32, Off(be, g).view,
                      Off(be, b).view, 1e-6, silu=True)
        assert_reduction(dy.get(), orc.group_norm(x, 32, g, b, 1e-6, silu=True), f"group_norm {shape} unaligned")


def test_rotary_unaligned(be, orc):
    N, S, heads, dim = 1, 64, 4, 128
    pos = np.array([[0, h, w] for h in range(8) for w in range(8)], np.int32)
    cs, sn = orc.rope_tables_3axis(pos, [32, 48, 48], dim, 256.0)
    q, k = orc.randn((N, S, heads * dim), 3061), orc.randn((N, S, heads * dim), 3062)
    dcs, dsn = Off(be, cs), Off(be, sn)
    dq, dk = Off(be, q), Off(be, k)
    be.rope_qk(dq.view, heads * dim, dk.view, heads * dim, N, S, dim, dcs.view, dsn.view, True)
    assert_elementwise(dq.get(), orc.rope(q, dim, cs, sn, True), "rope q unaligned")
    assert_elementwise(dk.get(), orc.rope(k, dim, cs, sn, True), "rope k unaligned")
    gq, gk = orc.randn((dim,), 3063, 1.0, 0.1), orc.randn((dim,), 3064, 1.0, 0.1)
    dq, dk = Off(be, q), Off(be, k)
    be.qknorm_rope(dq.view, heads * dim, dk.view, heads * dim, N, S, dim, Off(be, gq).view, Off(be, gk).view, 1e-5,
                   dcs.view, dsn.view, True)
    wq, wk = orc.qknorm_rope(q, k, dim, gq, gk, 1e-5, cs, sn, True)
    assert_reduction(dq.get(), wq, "qknorm_rope q unaligned")
    assert_reduction(dk.get(), wk, "qknorm_rope k unaligned")


def test_layout_unaligned(be, orc):
    x = orc.randn((1, 8, 16, 16), 3071)
    dx, dy = Off(be, x), Off(be, np.zeros((1, 8, 32, 32)))
    be.upsample_nearest2x(dx.view, dy.view, 8, 16, 16)
    assert_elementwise(dy.get(), orc.upsample_nearest2x(x), "upsample unaligned")
    dt = Off(be, np.zeros((1, 256, 8)))
    be.nchw_to_nlc(dx.view, dt.view, 1, 8, 256)
    assert_elementwise(dt.get(), orc.nchw_to_nlc(x), "nchw_to_nlc unaligned")
    a, b = orc.randn((2, 4, 8, 8), 3072), orc.randn((2, 8, 8, 8), 3073)
    dc = Off(be, np.zeros((2, 12, 8, 8)))
    be.concat_channels(Off(be, a).view, Off(be, b).view, dc.view, 2, 4, 8, 64)
    assert_elementwise(dc.get(), orc.concat_channels(a, b), "concat unaligned")


def test_attention_and_gemm_unaligned(be, orc):
    N, S, heads, d = 1, 70, 2, 64
    q, k, v = (orc.randn((N, S, heads * d), 3081 + i) for i in range(3))
    dq, dk, dv, do = Off(be, q), Off(be, k), Off(be, v), Off(be, np.zeros((N, S, heads * d)))
    be.attention(dq.view, dk.view, dv.view, do.view, N, S, S, heads, heads, d)
    err = float(np.max(np.abs(do.get() - orc.attention(q, k, v, heads))))
    assert err <= ATTN_TOL, f"attention unaligned: max-abs {err:.3e}"
    M, Nn, K = 33, 40, 64
    A, B = orc.randn((M, K), 3091), orc.randn((Nn, K), 3092, 0.0, 0.1)
    dc = Off(be, np.zeros((M, Nn)))
    be.gemm_nt_f32(M, Nn, K, Off(be, A).view, K, Off(be, B).view, K, dc.view, Nn)
    want, Sb = orc.gemm_nt_f32(A, B)
    assert_gemm(dc.get(), want, Sb, K, "gemm_nt_f32 unaligned")
    W16 = f32_to_bf16(B)
    dc = Off(be, np.zeros((M, Nn)))
    be.gemm_nt_bf16(M, Nn, K, Off(be, A).view, K, be.array(W16), K, dc.view, Nn)
    want, Sb = orc.gemm_nt_bf16(A, W16)
    assert_gemm(dc.get(), want, Sb, K + 1, "gemm_nt_bf16 unaligned")
