"""GPU sweep of shapes across every dispatch boundary, through the C ABI,
against the oracle with the usual tolerances (seeded inputs).

The parity tests pin each op at its config shapes and hand-picked edge cases;
the launchers also choose among kernels by row width (the float4 count per
lane, one wave or one workgroup per row), alignment of the width, head size,
group size and key/query tiling. This sweep takes widths just below, at and
just above each of those boundaries, so every dispatch branch runs. Sizes
stay small; the whole sweep takes seconds.
"""
import math

import numpy as np
import pytest

from tolerances import assert_elementwise, assert_reduction, assert_softmax

pytestmark = pytest.mark.gpu

# row widths around the dispatch boundaries of the row kernels (64 * 4 * V floats
# for V in 1, 2, 4, 8, 12, 15, 16, 24, 32) and the row-per-workgroup range
WIDTHS = [4, 8, 12, 60, 64, 68, 252, 256, 260, 508, 512, 516, 1020, 1024, 1028, 2044, 2048, 2052, 3072, 3836,
          3840, 3844, 4096, 4100, 6144, 8188, 8192, 8196, 9000, 5, 7, 33, 255, 1027]


def _rows(C):
    return max(1, min(37, 200_000 // C))


@pytest.mark.parametrize("C", WIDTHS)
def test_row_norms_sweep(be, orc, C):
    rows = _rows(C)
    x, r = orc.randn((rows, C), 4000 + C), orc.randn((rows, C), 4100 + C)
    g, b = orc.randn((C,), 4200 + C, 1.0, 0.1), orc.randn((C,), 4300 + C, 0.0, 0.1)
    dx, dy, dg, db = be.array(x), be.empty((rows, C)), be.array(g), be.array(b)
    be.rms_norm(dx, dy, rows, C, dg, 1e-6)
    assert_reduction(dy.download(), orc.rms_norm(x, g, 1e-6), f"rms_norm C={C}")
    be.layer_norm(dx, dy, rows, C, dg, db, 1e-6)
    assert_reduction(dy.download(), orc.layer_norm(x, g, b, 1e-6), f"layer_norm C={C}")
    be.add_rms_norm(dx, be.array(r), dy, rows, C, dg, 1e-6)
    s_want, y_want = orc.add_rms_norm(x, r, g, 1e-6)
    assert_elementwise(dx.download(), s_want, f"add_rms_norm sum C={C}")
    assert_reduction(dy.download(), y_want, f"add_rms_norm C={C}")


@pytest.mark.parametrize("C", WIDTHS)
def test_modulation_sweep(be, orc, C):
    rows = _rows(C)
    x, res = orc.randn((rows, C), 4400 + C), orc.randn((rows, C), 4500 + C)
    sc, sh, gt = (orc.randn((C,), 4600 + C + i, 0.0, 0.2) for i in range(3))
    dres, dy = be.array(res), be.empty((rows, C))
    be.ln_modulate_gate(be.array(x), dres, be.array(sc), be.array(sh), be.array(gt), dy, rows, C, 1e-6)
    r_want, y_want = orc.ln_modulate_gate(x, res, sc, sh, gt, 1e-6)
    assert_reduction(dy.download(), y_want, f"ln_modulate_gate y C={C}")
    assert_reduction(dres.download(), r_want, f"ln_modulate_gate res C={C}")
    g = orc.randn((C,), 4700 + C, 1.0, 0.1)
    dx = be.array(x)
    be.rms_norm_gated_add(dx, be.array(res), rows, C, be.array(g), be.array(gt), 1e-5)
    assert_reduction(dx.download(), orc.add_rows_scaled(x, orc.rms_norm(res, g, 1e-5), gt), f"gated_add C={C}")


@pytest.mark.parametrize("cols", [1, 3, 4, 60, 64, 100, 256, 260, 512, 1024, 1028, 2048, 2052, 4096, 4100, 8192,
                                  16384, 16388, 20000])
@pytest.mark.parametrize("causal", [False, True])
def test_softmax_sweep(be, orc, cols, causal):
    rows = max(1, min(40, 400_000 // cols))
    x = orc.randn((rows, cols), 4800 + cols, 0.0, 3.0)
    dx = be.array(x)
    be.softmax_rows(dx, rows, cols, 1.0 / math.sqrt(128.0), causal)
    assert_softmax(dx.download(), orc.softmax_rows(x, 1.0 / math.sqrt(128.0), causal), f"softmax cols={cols}")


@pytest.mark.parametrize("dim", [2, 4, 6, 8, 12, 16, 24, 32, 64, 96, 128, 160, 256])
@pytest.mark.parametrize("interleaved", [True, False])
def test_rotary_sweep(be, orc, dim, interleaved):
    N, S, hq, hk = 2, 19, 3, 1
    cs, sn = orc.rope_tables_half(S, dim, 10000.0)
    q, k = orc.randn((N, S, hq * dim), 4900 + dim), orc.randn((N, S, hk * dim), 4950 + dim)
    dq, dk = be.array(q), be.array(k)
    be.rope_qk(dq, hq * dim, dk, hk * dim, N, S, dim, be.array(cs), be.array(sn), interleaved)
    assert_elementwise(dq.download(), orc.rope(q, dim, cs, sn, interleaved), f"rope q dim={dim}")
    assert_elementwise(dk.download(), orc.rope(k, dim, cs, sn, interleaved), f"rope k dim={dim}")
    gq, gk = orc.randn((dim,), 4990, 1.0, 0.1), orc.randn((dim,), 4991, 1.0, 0.1)
    dq, dk = be.array(q), be.array(k)
    be.qknorm_rope(dq, hq * dim, dk, hk * dim, N, S, dim, be.array(gq), be.array(gk), 1e-5, be.array(cs),
                   be.array(sn), interleaved)
    wq, wk = orc.qknorm_rope(q, k, dim, gq, gk, 1e-5, cs, sn, interleaved)
    assert_reduction(dq.download(), wq, f"qknorm_rope q dim={dim}")
    assert_reduction(dk.download(), wk, f"qknorm_rope k dim={dim}")
    h = orc.randn((50, dim), 4992 + dim)
    dh = be.array(h)
    be.rms_norm_heads(dh, 50, dim, be.array(gq), 1e-5)
    assert_reduction(dh.download(), orc.rms_norm_heads(h, dim, gq, 1e-5), f"rms_norm_heads dim={dim}")


@pytest.mark.parametrize("shape,groups", [((1, 32, 1, 1), 32), ((2, 64, 3, 5), 32), ((1, 8, 100, 100), 4),
                                          ((1, 64, 128, 128), 32), ((3, 96, 17, 17), 32), ((1, 32, 512, 129), 32),
                                          ((1, 4, 256, 260), 2), ((2, 6, 7, 9), 3), ((1, 32, 256, 256), 1),
                                          # segments at the single / one-resident-round boundary (24576
                                          # floats) and at the single schedule's 65536-float limit
                                          ((1, 1, 1, 24572), 1), ((1, 1, 1, 24576), 1), ((1, 1, 1, 24580), 1),
                                          ((2, 3, 4, 8196), 3), ((1, 1, 1, 65536), 1), ((1, 1, 1, 65540), 1)])
def test_group_norm_sweep(be, orc, shape, groups):
    x = orc.randn(shape, 5000 + shape[1], 0.5, 2.0)
    g, b = orc.randn((shape[1],), 5001, 1.0, 0.1), orc.randn((shape[1],), 5002, 0.0, 0.1)
    N, Cc = shape[0], shape[1]
    for silu in (True, False):
        dy = be.empty(shape)
        be.group_norm(be.array(x), dy, N, Cc, x.size // (N * Cc), groups, be.array(g), be.array(b), 1e-6, silu=silu)
        assert_reduction(dy.download(), orc.group_norm(x, groups, g, b, 1e-6, silu=silu),
                         f"group_norm {shape} g{groups} silu={silu}")


@pytest.mark.parametrize("dim", WIDTHS[:20])
def test_broadcast_sweep(be, orc, dim):
    rows = _rows(dim)
    x, y = orc.randn((rows, dim), 5100 + dim), orc.randn((rows, dim), 5200 + dim)
    v = orc.randn((dim,), 5300 + dim, 1.0, 0.2)
    dx = be.array(x)
    be.mul_rows(dx, be.array(v), rows, dim)
    assert_elementwise(dx.download(), orc.mul_rows(x, v), f"mul_rows dim={dim}")
    dx = be.array(x)
    be.add_rows_scaled(dx, be.array(y), be.array(v), rows, dim)
    assert_elementwise(dx.download(), orc.add_rows_scaled(x, y, v), f"add_rows_scaled dim={dim}")
    if dim % 2 == 0:
        dz = be.empty((rows, dim // 2))
        be.geglu(be.array(x), dz, rows, dim // 2)
        assert_elementwise(dz.download(), orc.geglu(x), f"geglu D={dim // 2}")


ATTN_TOL = 1e-4  # max-abs on unit-variance inputs, as tests/test_gpu_attention.py


@pytest.mark.parametrize("d", [1, 8, 15, 16, 33, 63, 64, 65, 100, 127, 128, 129, 200, 256])
@pytest.mark.parametrize("Sq,Skv,causal", [(1, 1, False), (17, 70, False), (70, 17, True), (300, 300, True),
                                           (257, 129, False)])
def test_attention_sweep(be, orc, d, Sq, Skv, causal):
    """Head sizes across the MFMA kernel's two paddings (64, 128), its scalar
    loads (d below the padding) and the generic kernel (d > 128); query and key
    counts off the 256-query and 64-key tiles; grouped heads."""
    N, heads, kvh = 1, 4, 2
    q = orc.randn((N, Sq, heads * d), 5400 + d)
    k = orc.randn((N, Skv, kvh * d), 5401 + d)
    v = orc.randn((N, Skv, kvh * d), 5402 + d)
    out = be.empty((N, Sq, heads * d))
    be.attention(be.array(q), be.array(k), be.array(v), out, N, Sq, Skv, heads, kvh, d, causal)
    err = float(np.max(np.abs(out.download() - orc.attention(q, k, v, heads, causal, kvh))))
    assert err <= ATTN_TOL, f"attention d={d} Sq={Sq} Skv={Skv} causal={causal}: max-abs {err:.3g}"
