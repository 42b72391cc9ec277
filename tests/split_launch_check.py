"""Run by test_gpu_limits.test_split_launches in a child process with
SDH_LAUNCH_ITEMS=4096: the launchers then cover any tensor of more than 4096
work-items in several launches, so ordinary sizes take the path that tensors
past 2^31 elements take in production. Each op is checked against the oracle
on the CPU with the usual tolerances; prints "split ok" at the end.

Pieces exercised: the float4 streaming kernels with a scalar tail in the last
piece, whole rows of the row and broadcast kernels, softmax pieces that start
mid-tensor (causal mask phase, batched period), rotary pieces of whole
sequences and of parts of one sequence (tables offset), GroupNorm pieces of
whole samples.
"""
import math
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
sys.path[:0] = [os.path.join(ROOT, "stablediffusion-cpp_amd"), os.path.join(ROOT, "oracle"), HERE]

import numpy as np  # noqa: E402

import sdhip  # noqa: E402
from oracle import Oracle, bf16_to_f32  # noqa: E402
from tolerances import assert_elementwise, assert_reduction, assert_softmax  # noqa: E402


def main():
    assert os.environ.get("SDH_LAUNCH_ITEMS") == "4096", "run with SDH_LAUNCH_ITEMS=4096"
    be, orc = sdhip.Backend(), Oracle()

    def step(name):
        print(name, flush=True)

    step("streaming")
    for n in (100003, 4 * 4096 + 2, 3):
        g, u = orc.randn((n,), 1, 0.0, 1.5), orc.randn((n,), 2, 0.0, 1.5)
        dg, du, dy = be.array(g), be.array(u), be.empty((n,))
        be.swiglu(dg, du, dy, n)
        assert_elementwise(dy.download(), orc.swiglu(g, u), f"swiglu {n}")
        y16 = be.array(np.zeros(n, np.uint16))
        be.swiglu_bf16(dg, du, y16, n)
        ref16 = be.array(np.zeros(n, np.uint16))
        be.to_bf16(dy, ref16, n)
        assert np.array_equal(y16.download(), ref16.download()), f"swiglu_bf16 {n}"
        be.add(dg, du, n)
        assert_elementwise(dg.download(), orc.add(g, u), f"add {n}")
        be.silu(du, n)
        assert_elementwise(du.download(), orc.silu(u), f"silu {n}")
    x = orc.randn((50, 512), 3)
    dx, dy = be.array(x), be.empty((50, 256))
    be.geglu(dx, dy, 50, 256)
    assert_elementwise(dy.download(), orc.geglu(x), "geglu")

    step("broadcast")
    rows, C = 300, 256
    x, y = orc.randn((rows, C), 4), orc.randn((rows, C), 5)
    v = orc.randn((C,), 6, 1.0, 0.2)
    dx, dv = be.array(x), be.array(v)
    be.mul_rows(dx, dv, rows, C)
    assert_elementwise(dx.download(), orc.mul_rows(x, v), "mul_rows")
    dx = be.array(x)
    be.add_rows_scaled(dx, be.array(y), dv, rows, C)
    assert_elementwise(dx.download(), orc.add_rows_scaled(x, y, v), "add_rows_scaled")

    step("rows")
    gam, bet = orc.randn((C,), 7, 1.0, 0.1), orc.randn((C,), 8, 0.0, 0.1)
    dg, db = be.array(gam), be.array(bet)
    dx, dy = be.array(x), be.empty((rows, C))
    be.rms_norm(dx, dy, rows, C, dg, 1e-6)
    assert_reduction(dy.download(), orc.rms_norm(x, gam, 1e-6), "rms_norm")
    be.layer_norm(dx, dy, rows, C, dg, db, 1e-6)
    assert_reduction(dy.download(), orc.layer_norm(x, gam, bet, 1e-6), "layer_norm")
    dr = be.array(y)
    be.add_rms_norm(dx, dr, dy, rows, C, dg, 1e-6)
    s_want, y_want = orc.add_rms_norm(x, y, gam, 1e-6)
    assert_elementwise(dx.download(), s_want, "add_rms_norm sum")
    assert_reduction(dy.download(), y_want, "add_rms_norm")
    sc, sh, ga = (orc.randn((C,), 9 + i, 0.0, 0.2) for i in range(3))
    dx, dres, dyo = be.array(x), be.array(y), be.empty((rows, C))
    be.ln_modulate_gate(dx, dres, be.array(sc), be.array(sh), be.array(ga), dyo, rows, C, 1e-6)
    res_want, y_want = orc.ln_modulate_gate(x, y, sc, sh, ga, 1e-6)
    assert_reduction(dyo.download(), y_want, "ln_modulate_gate y")
    assert_reduction(dres.download(), res_want, "ln_modulate_gate res")
    y16 = be.array(np.zeros(rows * C, np.uint16))
    be.rms_norm_modulate_bf16(be.array(x), y16, rows, C, dg, dv, 1e-5)
    want = orc.mul_rows(orc.rms_norm(x, gam, 1e-5), v)
    got = bf16_to_f32(y16.download()).reshape(rows, C)
    assert np.max(np.abs(got - want) / np.maximum(np.abs(want), 1e-30)) <= 2.0 ** -8, "rms_norm_modulate_bf16"
    dx = be.array(x)
    be.rms_norm_gated_add(dx, be.array(y), rows, C, dg, dv, 1e-5)
    assert_reduction(dx.download(), orc.add_rows_scaled(x, orc.rms_norm(y, gam, 1e-5), v), "rms_norm_gated_add")
    # rows of 3840 (the gated add runs one workgroup per row: 16 rows per launch here)
    xw, yw = orc.randn((40, 3840), 20), orc.randn((40, 3840), 21, 0.0, 3.0)
    gw, vw = orc.randn((3840,), 22, 1.0, 0.1), orc.randn((3840,), 23, 0.0, 0.5)
    dxw, dyw = be.array(xw), be.empty((40, 3840))
    be.add_rms_norm(dxw, be.array(yw), dyw, 40, 3840, be.array(gw), 1e-6)
    s_want, y_want = orc.add_rms_norm(xw, yw, gw, 1e-6)
    assert_elementwise(dxw.download(), s_want, "add_rms_norm sum, wide rows")
    assert_reduction(dyw.download(), y_want, "add_rms_norm, wide rows")
    dxw = be.array(xw)
    be.rms_norm_gated_add(dxw, be.array(yw), 40, 3840, be.array(gw), be.array(vw), 1e-5)
    assert_reduction(dxw.download(), orc.add_rows_scaled(xw, orc.rms_norm(yw, gw, 1e-5), vw), "gated_add, wide rows")
    # residual add + RMSNorm + modulate, narrow and wide rows, against the two ops in the same pieces
    for xx, yy, gg, vv in ((x, y, dg, dv), (xw, yw, be.array(gw), be.array(vw))):
        r_, c_ = xx.shape
        dxf, dyf = be.array(xx), be.array(yy)
        f16 = be.array(np.zeros(r_ * c_, np.uint16))
        be.rms_norm_gated_add_modulate_bf16(dxf, dyf, f16, r_, c_, gg, vv, gg, vv, 1e-5)
        dxs = be.array(xx)
        be.rms_norm_gated_add(dxs, dyf, r_, c_, gg, vv, 1e-5)
        s16 = be.array(np.zeros(r_ * c_, np.uint16))
        be.rms_norm_modulate_bf16(dxs, s16, r_, c_, gg, vv, 1e-5)
        assert np.array_equal(dxf.download(), dxs.download()), f"gated_add_modulate x, rows of {c_}"
        assert np.array_equal(f16.download(), s16.download()), f"gated_add_modulate y, rows of {c_}"
    h = orc.randn((3000, 128), 12)
    gh = orc.randn((128,), 13, 1.0, 0.1)
    dh = be.array(h)
    be.rms_norm_heads(dh, 3000, 128, be.array(gh), 1e-5)
    assert_reduction(dh.download(), orc.rms_norm_heads(h, 128, gh, 1e-5), "rms_norm_heads")

    step("softmax")
    for r, c, causal, period in ((300, 4096, True, None), (300, 4096, False, None), (300, 100, True, None),
                                 (111 * 12, 37, True, 111)):
        x = orc.randn((r, c), 14, 0.0, 3.0)
        dx = be.array(x)
        be.softmax_rows(dx, r, c, 1.0 / math.sqrt(128.0), causal, period)
        assert_softmax(dx.download(), orc.softmax_rows(x, 1.0 / math.sqrt(128.0), causal, period),
                       f"softmax [{r},{c}] causal={causal} period={period}")

    step("rope")
    for N, S, heads, dim in ((2, 40, 3, 16), (50, 8, 2, 16)):
        cs, sn = orc.rope_tables_half(S, dim, 10000.0)
        for inter in (True, False):
            q = orc.randn((N, S, heads * dim), 15)
            k = orc.randn((N, S, 2 * dim), 16)
            dq, dk = be.array(q), be.array(k)
            be.rope_qk(dq, heads * dim, dk, 2 * dim, N, S, dim, be.array(cs), be.array(sn), inter)
            assert_elementwise(dq.download(), orc.rope(q, dim, cs, sn, inter), f"rope q N={N} S={S} {inter}")
            assert_elementwise(dk.download(), orc.rope(k, dim, cs, sn, inter), f"rope k N={N} S={S} {inter}")

    step("rope_qk_axes")
    for N, S in ((2, 40), (50, 8)):  # parts of one sequence (positions offset), and whole sequences per launch
        pos = np.array([[i % 7, (3 * i) % 11, i] for i in range(S)], np.int32)
        cs, sn = orc.rope_tables_3axis(pos, [4, 6, 6], 16, 256.0)
        q = orc.randn((N, S, 3 * 16), 20)
        k = orc.randn((N, S, 2 * 16), 21)
        dq, dk = be.array(q), be.array(k)
        be.rope_qk_axes(dq, 3 * 16, dk, 2 * 16, N, S, 16, be.array(pos.view(np.float32)), (4, 6, 6), 256.0)
        assert_elementwise(dq.download(), orc.rope(q, 16, cs, sn, True), f"rope_qk_axes q N={N} S={S}")
        assert_elementwise(dk.download(), orc.rope(k, 16, cs, sn, True), f"rope_qk_axes k N={N} S={S}")

    step("group_norm")
    shape, groups = (5, 64, 8, 8), 32
    x = orc.randn(shape, 17, 0.5, 2.0)
    g, b = orc.randn((64,), 18, 1.0, 0.1), orc.randn((64,), 19, 0.0, 0.1)
    for silu in (True, False):
        dx, dy = be.array(x), be.empty(shape)
        be.group_norm(dx, dy, 5, 64, 64, groups, be.array(g), be.array(b), 1e-6, silu=silu)
        assert_reduction(dy.download(), orc.group_norm(x, groups, g, b, 1e-6, silu=silu), f"group_norm silu={silu}")
    print("split ok", flush=True)


if __name__ == "__main__":
    main()
