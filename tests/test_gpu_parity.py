"""GPU parity: every backend_hip entry point vs the CPU oracle (and, where it
was built, vs the compiled reference itself), through the C ABI.

Inputs come from the oracle's seeded generator, are uploaded once, and the
same host arrays feed the oracle, so both sides see identical bits. Shapes:
the reference's own test_ops shapes (tests/test_ops.cpp:389-463), odd and
unaligned shapes that force the generic kernels, and the BASELINE config
shapes (Z-Image 1024^2: T=4096 tokens, D=3840, F=10240; FLUX-VAE and SD 1.5
GroupNorm shapes). Tolerances are defined in tolerances.py.
"""
import math
import os
import subprocess
import sys

import numpy as np
import pytest

import sdhip
from tolerances import assert_elementwise, assert_reduction, assert_softmax

pytestmark = pytest.mark.gpu

T, D, F = 4096, 3840, 10240
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "stablediffusion-cpp_amd")
ORACLE_DIR = os.path.join(ROOT, "oracle")


def _seed(*parts):
    h = 1469598103934665603
    for p in parts:
        for ch in str(p):
            h = ((h ^ ord(ch)) * 1099511628211) % (1 << 64)
    return h


# ---------------------------------------------------------------- elementwise
@pytest.mark.parametrize("n", [1, 3, 1000, 4097, 1 << 20, T * F])
def test_swiglu(be, orc, n):
    g = orc.randn((n,), _seed("sw_g", n), 0.0, 1.5)
    u = orc.randn((n,), _seed("sw_u", n), 0.0, 1.5)
    dg, du, dy = be.array(g), be.array(u), be.empty((n,))
    be.swiglu(dg, du, dy, n)
    assert_elementwise(dy.download(), orc.swiglu(g, u), f"swiglu n={n}")


@pytest.mark.parametrize("op", ["silu", "tanh", "gelu", "quick_gelu"])
@pytest.mark.parametrize("n", [1000, 1 << 18, 12345])
def test_unary(be, orc, op, n):
    x = orc.randn((n,), _seed(op, n), 0.0, 3.0)
    dx = be.array(x)
    getattr(be, op)(dx, n)
    assert_elementwise(dx.download(), getattr(orc, op)(x), f"{op} n={n}")


@pytest.mark.parametrize("n", [1000, 1 << 20, 7])
def test_add_scale_affine(be, orc, n):
    a = orc.randn((n,), _seed("a", n))
    b = orc.randn((n,), _seed("b", n))
    da, db = be.array(a), be.array(b)
    be.add(da, db, n)
    want = orc.add(a, b)
    assert_elementwise(da.download(), want, "add")
    be.scale(da, 0.37, n)
    want = orc.scale(want, 0.37)
    assert_elementwise(da.download(), want, "scale")
    be.affine(da, 1.5, -0.25, n)
    want = orc.affine(want, 1.5, -0.25)
    assert_elementwise(da.download(), want, "affine")


@pytest.mark.parametrize("rows,D2", [(6, 40), (33, 1280 * 2), (4, 7 * 2)])
def test_geglu(be, orc, rows, D2):
    x = orc.randn((rows, D2), _seed("geglu", rows, D2))
    dx, dy = be.array(x), be.empty((rows, D2 // 2))
    be.geglu(dx, dy, rows, D2 // 2)
    assert_elementwise(dy.download(), orc.geglu(x), "geglu")


# ---------------------------------------------------------------- broadcasts
@pytest.mark.parametrize("rows,dim", [(4, 6), (T, D), (37, 64), (5, 7)])
def test_row_broadcasts(be, orc, rows, dim):
    x = orc.randn((rows, dim), _seed("rb_x", rows, dim))
    y = orc.randn((rows, dim), _seed("rb_y", rows, dim))
    v = orc.randn((dim,), _seed("rb_v", rows, dim), 0.0, 0.2)
    dx, dy, dv = be.array(x), be.array(y), be.array(v)
    be.mul_rows(dx, dv, rows, dim)
    want = orc.mul_rows(x, v)
    assert_elementwise(dx.download(), want, "mul_rows")
    be.add_rows_scaled(dx, dy, dv, rows, dim)
    want = orc.add_rows_scaled(want, y, v)
    assert_elementwise(dx.download(), want, "add_rows_scaled")
    be.add_rows(dx, dv, rows, dim)
    want = orc.add_rows_scaled(want, np.ones_like(want), v)  # += v as the CPU composes it
    assert_elementwise(dx.download(), want, "add_rows")


@pytest.mark.parametrize("shape", [(2, 3, 4, 5), (2, 320, 64, 64), (1, 7, 3, 3)])
def test_add_channel_bias(be, orc, shape):
    x = orc.randn(shape, _seed("cb_x", *shape))
    b = orc.randn(shape[:2], _seed("cb_b", *shape))
    dx, db = be.array(x), be.array(b)
    N, Cc = shape[0], shape[1]
    be.add_channel_bias(dx, db, N, Cc, x.size // (N * Cc))
    assert_elementwise(dx.download(), orc.add_channel_bias(x, b), "add_channel_bias")


# ---------------------------------------------------------------- norms
@pytest.mark.parametrize("rows,C", [(21, 64), (T, D), (5, 24), (3, 70), (2, 9000), (130, 5), (1, 1)])
@pytest.mark.parametrize("affine", [True, False])
def test_rms_norm(be, orc, rows, C, affine):
    x = orc.randn((rows, C), _seed("rms", rows, C))
    w = orc.randn((C,), _seed("rms_w", C), 1.0, 0.1) if affine else None
    dx, dy = be.array(x), be.empty((rows, C))
    dw = be.array(w) if affine else None
    be.rms_norm(dx, dy, rows, C, dw, 1e-6)
    assert_reduction(dy.download(), orc.rms_norm(x, w, 1e-6), f"rms_norm [{rows},{C}]")


@pytest.mark.parametrize("rows,C", [(21, 64), (T, D), (3, 70), (2, 9000), (33, 320)])
@pytest.mark.parametrize("gb", ["both", "none", "gamma", "beta"])
def test_layer_norm(be, orc, rows, C, gb):
    x = orc.randn((rows, C), _seed("ln", rows, C), 2.0, 3.0)
    g = orc.randn((C,), _seed("ln_g", C), 1.0, 0.1) if gb in ("both", "gamma") else None
    b = orc.randn((C,), _seed("ln_b", C), 0.0, 0.1) if gb in ("both", "beta") else None
    dx, dy = be.array(x), be.empty((rows, C))
    be.layer_norm(dx, dy, rows, C, be.array(g) if g is not None else None, be.array(b) if b is not None else None,
                  1e-5)
    assert_reduction(dy.download(), orc.layer_norm(x, g, b, 1e-5), f"layer_norm [{rows},{C}] {gb}")


@pytest.mark.parametrize("groups,dim", [(15, 8), (T * 30, 128), (37, 64), (10, 256), (9, 30), (4, 16)])
@pytest.mark.parametrize("affine", [True, False])
def test_rms_norm_heads(be, orc, groups, dim, affine):
    x = orc.randn((groups, dim), _seed("qk", groups, dim))
    w = orc.randn((dim,), _seed("qk_w", dim), 1.0, 0.1) if affine else None
    dx = be.array(x)
    be.rms_norm_heads(dx, groups, dim, be.array(w) if affine else None, 1e-5)
    assert_reduction(dx.download(), orc.rms_norm_heads(x, dim, w, 1e-5), f"rms_norm_heads [{groups},{dim}]")


@pytest.mark.parametrize("rows,C", [(T, D), (13, D), (1, D), (7, 64), (3, 70), (1, 9000)])
@pytest.mark.parametrize("affine", [True, False])
def test_add_rms_norm(be, orc, rows, C, affine):
    """Config 1: fused residual add + RMSNorm vs add_ then rms_norm (also a
    few rows, and one row, at the config width)."""
    x = orc.randn((rows, C), _seed("arn_x", rows, C))
    r = orc.randn((rows, C), _seed("arn_r", rows, C))
    w = orc.randn((C,), _seed("arn_w", C), 1.0, 0.1) if affine else None
    dx, dr, dy = be.array(x), be.array(r), be.empty((rows, C))
    be.add_rms_norm(dx, dr, dy, rows, C, be.array(w) if affine else None, 1e-6)
    s_ref, y_ref = orc.add_rms_norm(x, r, w, 1e-6)
    assert_elementwise(dx.download(), s_ref, "add_rms_norm sum")
    assert_reduction(dy.download(), y_ref, "add_rms_norm norm")


@pytest.mark.parametrize("rows,C", [(T, D), (600, D), (13, D), (1, D), (9, 64), (3, 70), (2, 9000)])
@pytest.mark.parametrize("shift", [True, False])
@pytest.mark.parametrize("store_y", [True, False])
def test_ln_modulate_gate(be, orc, rows, C, shift, store_y):
    """Config 5a: y = LN(x)(1+scale)+shift; res += tanh(gate) y."""
    x = orc.randn((rows, C), _seed("lmg_x", rows, C))
    res = orc.randn((rows, C), _seed("lmg_r", rows, C))
    sc = orc.randn((C,), _seed("lmg_s", C), 0.0, 0.2)
    sh = orc.randn((C,), _seed("lmg_h", C), 0.0, 0.2) if shift else None
    gt = orc.randn((C,), _seed("lmg_g", C), 0.0, 0.2)
    dx, dres = be.array(x), be.array(res)
    dy = be.empty((rows, C)) if store_y else None
    be.ln_modulate_gate(dx, dres, be.array(sc), be.array(sh) if shift else None, be.array(gt), dy, rows, C, 1e-6)
    r_ref, y_ref = orc.ln_modulate_gate(x, res, sc, sh, gt, 1e-6)
    assert_reduction(dres.download(), r_ref, "ln_modulate_gate res")
    if store_y:
        assert_reduction(dy.download(), y_ref, "ln_modulate_gate y")


@pytest.mark.parametrize("mean,std", [(300.0, 0.5), (-40.0, 1e-3), (0.0, 1e-30)])
def test_ln_modulate_gate_offset_rows(be, orc, mean, std):
    """Rows far from zero mean (and nearly constant rows): the statistics in
    one double pass must match the reference's two-pass form (mean, then the
    sum of squared deviations, tensor.cpp:640-648)."""
    rows, C = 64, 3840
    x = orc.randn((rows, C), _seed("lmg_off", int(mean)), mean, std)
    res = orc.randn((rows, C), _seed("lmg_off_r"))
    sc, sh, gt = (orc.randn((C,), _seed("lmg_off_v", i), 0.0, 0.2) for i in range(3))
    dres, dy = be.array(res), be.empty((rows, C))
    be.ln_modulate_gate(be.array(x), dres, be.array(sc), be.array(sh), be.array(gt), dy, rows, C, 1e-6)
    r_ref, y_ref = orc.ln_modulate_gate(x, res, sc, sh, gt, 1e-6)
    assert_reduction(dy.download(), y_ref, f"ln_modulate_gate y, rows ~N({mean}, {std})")
    assert_reduction(dres.download(), r_ref, f"ln_modulate_gate res, rows ~N({mean}, {std})")


GN_SHAPES = [
    ((2, 64, 5, 7), 32, 1e-6),          # test_ops.cpp:391-392
    ((1, 512, 128, 128), 32, 1e-6),     # config 4a (FLUX VAE)
    ((1, 128, 1024, 1024), 32, 1e-6),   # config 4b (FLUX VAE norm_out)
    ((2, 320, 64, 64), 32, 1e-5),       # config 4c (SD 1.5)
    ((2, 1280, 8, 8), 32, 1e-5),        # config 4d (SD 1.5)
    ((1, 96, 33, 17), 32, 1e-6),        # odd plane: generic kernel
    ((1, 16, 300, 300), 2, 1e-6),       # > 64 chunks per segment, plane not a whole number of chunks
    ((3, 8, 4, 4), 4, 1e-6),
]


@pytest.mark.parametrize("shape,groups,eps", GN_SHAPES)
@pytest.mark.parametrize("silu", [True, False])
def test_group_norm(be, orc, shape, groups, eps, silu):
    x = orc.randn(shape, _seed("gn", *shape), 0.0, 2.0)
    Cc = shape[1]
    g = orc.randn((Cc,), _seed("gn_g", Cc), 1.0, 0.1)
    b = orc.randn((Cc,), _seed("gn_b", Cc), 0.0, 0.1)
    dx, dy = be.array(x), be.empty(shape)
    N = shape[0]
    be.group_norm(dx, dy, N, Cc, x.size // (N * Cc), groups, be.array(g), be.array(b), eps, silu=silu)
    assert_reduction(dy.download(), orc.group_norm(x, groups, g, b, eps, silu=silu), f"group_norm{'+silu' if silu else ''} {shape}")


def test_group_norm_inplace_and_repeat(be, orc):
    """y == x is allowed; repeated calls re-arm the split kernel's counters."""
    shape = (1, 64, 256, 256)
    x = orc.randn(shape, 77, 1.0, 2.0)
    g = orc.randn((64,), 78, 1.0, 0.1)
    b = orc.randn((64,), 79, 0.0, 0.1)
    want = orc.group_norm(x, 32, g, b, 1e-6, silu=True)
    dg, db = be.array(g), be.array(b)
    for _ in range(3):
        dx = be.array(x)
        be.group_norm(dx, dx, 1, 64, 256 * 256, 32, dg, db, 1e-6, silu=True)
        assert_reduction(dx.download(), want, "group_norm_silu in place")


def test_group_norm_interleaved_shapes(be, orc):
    """Consecutive calls with different shapes and schedules, in place,
    each checked (scratch partials and statistics are reused across calls)."""
    cases = [((1, 512, 128, 128), 1e-6), ((2, 320, 64, 64), 1e-5), ((1, 64, 256, 256), 1e-6)]
    data = []
    for i, (shape, eps) in enumerate(cases):
        x = orc.randn(shape, 300 + i, 0.5, 2.0)
        g = orc.randn((shape[1],), 310 + i, 1.0, 0.1)
        b = orc.randn((shape[1],), 320 + i, 0.0, 0.1)
        data.append((shape, eps, x, be.array(g), be.array(b), orc.group_norm(x, 32, g, b, eps, silu=True)))
    for rep in range(2):
        for shape, eps, x, dg, db, want in data + data[::-1]:
            dx = be.array(x)
            N, Cc = shape[0], shape[1]
            be.group_norm(dx, dx, N, Cc, x.size // (N * Cc), 32, dg, db, eps, silu=True)
            assert_reduction(dx.download(), want, f"group_norm_silu {shape} rep {rep}")


def test_group_norm_segment_blocks():
    """The split schedule run block by block (SDH_GN_BLOCK_MB=2, in a child
    process): blocks that start inside a sample's groups (channel offset),
    one-segment blocks, and a plane that is not a whole number of chunks."""
    code = (
        "import sys; sys.path[:0] = [%r, %r]\n"
        "import numpy as np, sdhip\n"
        "from oracle import Oracle\n"
        "be, orc = sdhip.Backend(), Oracle()\n"
        "for shape, groups, eps in (((2, 64, 256, 256), 32, 1e-6), ((1, 32, 300, 300), 8, 1e-5), ((1, 512, 128, 128), 32, 1e-6)):\n"
        "    for silu in (True, False):\n"
        "        x = orc.randn(shape, 5, 0.5, 2.0); g = orc.randn((shape[1],), 6, 1.0, 0.1); b = orc.randn((shape[1],), 7, 0.0, 0.1)\n"
        "        d, o = be.array(x), be.empty(shape); N, C = shape[0], shape[1]\n"
        "        be.group_norm(d, o, N, C, x.size // (N * C), groups, be.array(g), be.array(b), eps, silu=silu)\n"
        "        want = orc.group_norm(x, groups, g, b, eps, silu=silu)\n"
        "        err = float(np.max(np.abs(o.download() - want) / np.maximum(np.abs(want), 1.0)))\n"
        "        print(shape, silu, err, flush=True)\n"
        "        assert err <= 1e-4, (shape, silu, err)\n"
        "print('blocks ok')\n"
    ) % (PKG_DIR, ORACLE_DIR)
    env = dict(os.environ, SDH_GN_BLOCK_MB="2")
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=180, env=env)
    print(r.stdout)
    assert r.returncode == 0 and "blocks ok" in r.stdout, r.stdout + r.stderr


# ---------------------------------------------------------------- softmax
@pytest.mark.parametrize("rows,cols", [(9, 9), (64, 4096), (100, 100), (5, 4128), (3, 9000), (7, 1)])
@pytest.mark.parametrize("causal", [False, True])
def test_softmax(be, orc, rows, cols, causal):
    x = orc.randn((rows, cols), _seed("sm", rows, cols), 0.0, 3.0)
    scale = 1.0 / math.sqrt(128.0)
    dx = be.array(x)
    be.softmax_rows(dx, rows, cols, scale, causal)
    assert_softmax(dx.download(), orc.softmax_rows(x, scale, causal), f"softmax [{rows},{cols}] causal={causal}")


def test_softmax_batched_period(be, orc):
    rows, cols, period = 3 * 37, 37, 37
    x = orc.randn((rows, cols), 91, 0.0, 3.0)
    dx = be.array(x)
    be.softmax_rows(dx, rows, cols, 0.25, True, period)
    assert_softmax(dx.download(), orc.softmax_rows(x, 0.25, True, period), "softmax batched causal")


def test_softmax_config_5b(be, orc):
    """Config 5b at full size: [30 heads, 4096, 4096], scale 1/sqrt(128)."""
    rows, cols = 30 * T, T
    x = orc.randn((rows, cols), _seed("sm5b"), 0.0, 3.0)
    scale = 1.0 / math.sqrt(128.0)
    dx = be.array(x)
    be.softmax_rows(dx, rows, cols, scale, False)
    got = dx.download()
    want = orc.softmax_rows(x, scale, False)
    assert_softmax(got, want, "softmax config 5b")
    # size-independent property: every row sums to 1
    assert float(np.max(np.abs(got.sum(axis=1, dtype=np.float64) - 1.0))) < 1e-5


# ---------------------------------------------------------------- rotary
def _zimage_tables(orc, S, side):
    pos = np.array([[0, h, w] for h in range(side) for w in range(side)], np.int32)[:S]
    return orc.rope_tables_3axis(pos, [32, 48, 48], 128, 256.0)


@pytest.mark.parametrize("interleaved", [True, False])
@pytest.mark.parametrize("N,S,heads,dim", [(1, 5, 3, 8), (2, 7, 4, 16), (1, 64, 30, 128), (1, 9, 2, 6)])
def test_rope(be, orc, interleaved, N, S, heads, dim):
    x = orc.randn((N, S, heads * dim), _seed("rope", N, S, heads, dim))
    ang = orc.randn((S, dim), _seed("rope_t", S, dim), 0.0, 1.0)
    cs, sn = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)  # arbitrary, non-paired tables
    dx = be.array(x)
    be.rope(dx, N, S, heads * dim, dim, be.array(cs), be.array(sn), interleaved)
    assert_elementwise(dx.download(), orc.rope(x, dim, cs, sn, interleaved), f"rope inter={interleaved}")


# (heads, dim) chosen to reach every register-resident form: 1/2/4/8/16 float4
# per thread (interleaved) and 1/2/4 pairs (rotate_half), with head sizes that
# divide the 256-thread workgroup (table loaded once) and that do not (dim 24),
# plus rows too wide for registers (the looping kernels).
ROPE_DISPATCH = [
    (True, 40, 24), (True, 100, 24), (True, 200, 24), (True, 350, 24),
    (True, 60, 128), (True, 120, 128), (True, 140, 128),
    (False, 30, 128), (False, 60, 128), (False, 70, 128), (False, 40, 24), (False, 150, 24), (False, 200, 24),
]


@pytest.mark.parametrize("interleaved,heads,dim", ROPE_DISPATCH)
def test_rope_dispatch(be, orc, interleaved, heads, dim):
    N, S = 1, 3
    x = orc.randn((N, S, heads * dim), _seed("ropd", heads, dim))
    ang = orc.randn((S, dim), _seed("ropd_t", dim), 0.0, 1.0)
    cs, sn = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    dx = be.array(x)
    be.rope(dx, N, S, heads * dim, dim, be.array(cs), be.array(sn), interleaved)
    assert_elementwise(dx.download(), orc.rope(x, dim, cs, sn, interleaved), f"rope inter={interleaved} {heads}x{dim}")


def test_rope_qk_config_3(be, orc):
    """Config 3: 3-axis interleaved RoPE on Q and K [4096, 30*128], one launch."""
    cs, sn = _zimage_tables(orc, T, 64)
    q = orc.randn((1, T, 30 * 128), _seed("q3"))
    k = orc.randn((1, T, 30 * 128), _seed("k3"))
    dq, dk, dc, ds = be.array(q), be.array(k), be.array(cs), be.array(sn)
    be.rope_qk(dq, 30 * 128, dk, 30 * 128, 1, T, 128, dc, ds, True)
    assert_elementwise(dq.download(), orc.rope(q, 128, cs, sn, True), "rope_qk q")
    assert_elementwise(dk.download(), orc.rope(k, 128, cs, sn, True), "rope_qk k")


def _pos_array(be, pos):
    """int32 positions [S, 3] on the device (uploaded as their raw bytes)."""
    return be.array(np.ascontiguousarray(pos, np.int32).view(np.float32))


def test_rope_qk_axes_config_3(be, orc):
    """Config 3 with the angles formed on the device (sdh_rope_qk_axes):
    positions (0, h, w) of the 64 x 64 grid, axes (32, 48, 48), theta 256,
    against the oracle's rope_ with its tables (the restatement of
    zimage.cpp:71-88) at max-abs 1e-5, and against the table kernel fed
    those tables."""
    pos = np.array([[0, h, w] for h in range(64) for w in range(64)], np.int32)
    cs, sn = orc.rope_tables_3axis(pos, [32, 48, 48], 128, 256.0)
    q = orc.randn((1, T, 30 * 128), _seed("q3a"))
    k = orc.randn((1, T, 30 * 128), _seed("k3a"))
    dq, dk = be.array(q), be.array(k)
    be.rope_qk_axes(dq, 30 * 128, dk, 30 * 128, 1, T, 128, _pos_array(be, pos), (32, 48, 48), 256.0)
    gq, gk = dq.download(), dk.download()
    assert_elementwise(gq, orc.rope(q, 128, cs, sn, True), "rope_qk_axes q")
    assert_elementwise(gk, orc.rope(k, 128, cs, sn, True), "rope_qk_axes k")
    tq, tk = be.array(q), be.array(k)
    be.rope_qk(tq, 30 * 128, tk, 30 * 128, 1, T, 128, be.array(cs), be.array(sn), True)
    d = max(float(np.max(np.abs(gq - tq.download()))), float(np.max(np.abs(gk - tk.download()))))
    print("device angles vs tables: max |diff|", d)
    assert d <= 1e-6


@pytest.mark.parametrize("N,S,hq,hk,dim,axes,theta", [
    (2, 37, 3, 1, 64, (16, 24, 24), 256.0),     # odd length, unequal head counts
    (1, 160, 30, 30, 128, (32, 48, 48), 256.0),  # Z-Image text rows: positions (1 + i, 0, 0)
    (1, 9, 2, 2, 8, (4, 0, 4), 10000.0),         # an empty axis
    (3, 5, 64, 64, 128, (32, 48, 48), 256.0),    # 8192-float rows (eight float4 per thread)
])
def test_rope_qk_axes_shapes(be, orc, N, S, hq, hk, dim, axes, theta):
    rng = np.random.default_rng(S + dim)
    pos = rng.integers(0, 200, size=(S, 3)).astype(np.int32)
    if S == 160:
        pos = np.array([[1 + i, 0, 0] for i in range(S)], np.int32)
    cs, sn = orc.rope_tables_3axis(pos, list(axes), dim, theta)
    q = orc.randn((N, S, hq * dim), _seed("qax", S, dim))
    k = orc.randn((N, S, hk * dim), _seed("kax", S, dim))
    dq, dk = be.array(q), be.array(k)
    be.rope_qk_axes(dq, hq * dim, dk, hk * dim, N, S, dim, _pos_array(be, pos), axes, theta)
    assert_elementwise(dq.download(), orc.rope(q, dim, cs, sn, True), f"rope_qk_axes q {N}x{S} {axes}")
    assert_elementwise(dk.download(), orc.rope(k, dim, cs, sn, True), f"rope_qk_axes k {N}x{S} {axes}")


def test_rope_qk_axes_rejects(be):
    q, k = be.empty((1, 4, 128)), be.empty((1, 4, 128))
    pos = _pos_array(be, np.zeros((4, 3), np.int32))
    for args, msg in [(((32, 48, 40), 256.0), "add up to dim"), (((33, 47, 48), 256.0), "even"),
                      (((32, 48, 48), 0.0), "theta")]:
        with pytest.raises(sdhip.SdhError, match=msg):
            be.rope_qk_axes(q, 128, k, 128, 1, 4, 128, pos, *args)
    with pytest.raises(sdhip.SdhError, match="distinct"):
        be.rope_qk_axes(q, 128, q, 128, 1, 4, 128, pos, (32, 48, 48), 256.0)


def test_rope_qk_gqa_half(be, orc):
    """rotate_half with fewer K heads (Qwen3-style tables, qwen3.cpp:46-53)."""
    S, dim = 37, 128
    cs, sn = orc.rope_tables_half(S, dim, 1e6)
    q = orc.randn((2, S, 8 * dim), 5)
    k = orc.randn((2, S, 2 * dim), 6)
    dq, dk = be.array(q), be.array(k)
    be.rope_qk(dq, 8 * dim, dk, 2 * dim, 2, S, dim, be.array(cs), be.array(sn), False)
    assert_elementwise(dq.download(), orc.rope(q, dim, cs, sn, False), "rope_qk half q")
    assert_elementwise(dk.download(), orc.rope(k, dim, cs, sn, False), "rope_qk half k")


# ---------------------------------------------------------------- fused QK-norm + RoPE
# (interleaved, N, S, q heads, k heads, dim, gamma): the Z-Image config shape;
# Qwen3-style GQA rotate_half; no gamma; dims 64 and 32; 1, 2 and 4 float4
# steps; and shapes that take the op-by-op path (dim 24; rows wider than 8
# float4 per thread).
QKN = [
    (True, 1, T, 30, 30, 128, True), (False, 2, 37, 8, 2, 128, True), (True, 2, 9, 40, 40, 64, False),
    (False, 1, 11, 100, 100, 32, True), (True, 1, 5, 6, 2, 128, True), (True, 1, 7, 5, 5, 24, True),
    (True, 1, 3, 70, 70, 128, True), (False, 1, 3, 40, 40, 128, False), (True, 1, 4, 12, 12, 128, True),
    (True, 1, 3, 60, 60, 128, False),
]


@pytest.mark.parametrize("inter,N,S,hq,hk,dim,gam", QKN)
def test_qknorm_rope(be, orc, inter, N, S, hq, hk, dim, gam):
    q = orc.randn((N, S, hq * dim), _seed("qkn_q", N, S, hq, dim), 0.5, 2.0)
    k = orc.randn((N, S, hk * dim), _seed("qkn_k", N, S, hk, dim), 0.5, 2.0)
    gq = orc.randn((dim,), _seed("qkn_gq", dim), 1.0, 0.1) if gam else None
    gk = orc.randn((dim,), _seed("qkn_gk", dim), 1.0, 0.1) if gam else None
    if inter and dim == 128 and S == T:
        cs, sn = _zimage_tables(orc, T, 64)
    else:
        ang = orc.randn((S, dim), _seed("qkn_t", S, dim), 0.0, 1.0)
        cs, sn = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    dq, dk, dc, ds = be.array(q), be.array(k), be.array(cs), be.array(sn)
    dgq = be.array(gq) if gam else None
    dgk = be.array(gk) if gam else None
    be.qknorm_rope(dq, hq * dim, dk, hk * dim, N, S, dim, dgq, dgk, 1e-5, dc, ds, inter)
    wq, wk = orc.qknorm_rope(q, k, dim, gq, gk, 1e-5, cs, sn, inter)
    got_q, got_k = dq.download(), dk.download()
    assert_reduction(got_q, wq, f"qknorm_rope q inter={inter} dim={dim}")
    assert_reduction(got_k, wk, f"qknorm_rope k inter={inter} dim={dim}")
    # the same ops unfused on the GPU
    uq, uk = be.array(q), be.array(k)
    be.rms_norm_heads(uq, N * S * hq, dim, dgq, 1e-5)
    be.rms_norm_heads(uk, N * S * hk, dim, dgk, 1e-5)
    be.rope_qk(uq, hq * dim, uk, hk * dim, N, S, dim, dc, ds, inter)
    print(f"fused vs unfused GPU: q {np.max(np.abs(got_q - uq.download())):.3e}, "
          f"k {np.max(np.abs(got_k - uk.download())):.3e}")


# ---------------------------------------------------------------- layout (bit-exact copies)
def _exact(got, want, what):
    assert got.shape == want.shape, what
    assert np.array_equal(got, want), f"{what}: {int(np.sum(got != want))} elements differ"


# (2,3,4,5): the reference test's image (scalar path, odd W); (2,3,4,8) and
# (1,2,3,6): vector path; (1,512,64,64): a VAE decoder upsample input;
# (1,1,1,1): minimal.
@pytest.mark.parametrize("shape", [(2, 3, 4, 5), (2, 3, 4, 8), (1, 2, 3, 6), (1, 512, 64, 64), (1, 1, 1, 1)])
def test_upsample_nearest2x(be, orc, shape):
    x = orc.randn(shape, _seed("up", *shape))
    N, Cc, H, W = shape
    y = be.empty((N, Cc, 2 * H, 2 * W))
    be.upsample_nearest2x(be.array(x), y, N * Cc, H, W)
    _exact(y.download(), orc.upsample_nearest2x(x), f"upsample {shape}")


# vector path (C*HW % 4 == 0), the SD 1.5 UNet skip concat, scalar path (HW = 9),
# and an empty first operand.
@pytest.mark.parametrize("sa,sb", [((2, 3, 4, 5), (2, 2, 4, 5)), ((2, 640, 64, 64), (2, 320, 64, 64)),
                                   ((2, 3, 3, 3), (2, 2, 3, 3)), ((2, 0, 4, 4), (2, 5, 4, 4))])
def test_concat_channels(be, orc, sa, sb):
    a = orc.randn(sa, _seed("cca", *sa))
    b = orc.randn(sb, _seed("ccb", *sb))
    N, Ca, Cb = sa[0], sa[1], sb[1]
    HW = sb[2] * sb[3]
    y = be.empty((N, Ca + Cb) + sb[2:])
    da = be.array(a) if a.size else be.empty((1,))
    be.concat_channels(da, be.array(b), y, N, Ca, Cb, HW)
    _exact(y.download(), orc.concat_channels(a, b), f"concat_channels {sa} {sb}")


# tile-aligned (VAE attention [1,512,128x128], SD 1.5 [2,320,64x64]), partial
# edge tiles (100 x 100), and the scalar path (C = 3).
@pytest.mark.parametrize("shape", [(1, 512, 128, 128), (2, 320, 64, 64), (1, 100, 10, 10), (2, 3, 4, 5), (3, 8, 1, 12)])
def test_nchw_nlc_round_trip(be, orc, shape):
    x = orc.randn(shape, _seed("nlc", *shape))
    N, Cc, H, W = shape
    dx, dn, db = be.array(x), be.empty((N, H * W, Cc)), be.empty(shape)
    be.nchw_to_nlc(dx, dn, N, Cc, H * W)
    nlc = dn.download()
    _exact(nlc, orc.nchw_to_nlc(x), f"nchw_to_nlc {shape}")
    be.nlc_to_nchw(dn, db, N, Cc, H * W)
    _exact(db.download(), orc.nlc_to_nchw(nlc, H, W), f"nlc_to_nchw {shape}")
    _exact(db.download(), x, f"round trip {shape}")


# the reference test's latent (16 x 6 x 8, p 2), the Z-Image 1024^2 latent
# (16 x 128 x 128, p 2), p = 3 and p = 1.
@pytest.mark.parametrize("Cc,H,W,p", [(16, 6, 8, 2), (16, 128, 128, 2), (3, 9, 12, 3), (5, 4, 7, 1)])
def test_patchify_round_trip(be, orc, Cc, H, W, p):
    x = orc.randn((1, Cc, H, W), _seed("pat", Cc, H, W, p))
    ntok, F_ = (H // p) * (W // p), p * p * Cc
    dx, dt, dy = be.array(x), be.empty((ntok, F_)), be.empty((1, Cc, H, W))
    be.patchify(dx, dt, Cc, H, W, p)
    tok = dt.download()
    _exact(tok, orc.patchify(x, p), f"patchify {Cc}x{H}x{W} p{p}")
    be.unpatchify(dt, dy, Cc, H, W, p)
    _exact(dy.download(), orc.unpatchify(tok, Cc, H, W, p), f"unpatchify {Cc}x{H}x{W} p{p}")
    _exact(dy.download(), x, "round trip")


def test_layout_invalid_arguments(be):
    d = be.empty((2 * 4 * 6,))
    o = be.empty((2 * 4 * 6,))
    with pytest.raises(sdhip.SdhError) as e:
        be.patchify(d, o, 2, 4, 6, 4)  # W not a multiple of p
    assert e.value.status == sdhip.SDH_ERR_INVALID
    with pytest.raises(sdhip.SdhError) as e:
        be.unpatchify(d, o, 2, 4, 6, 0)  # p = 0
    assert e.value.status == sdhip.SDH_ERR_INVALID
    with pytest.raises(sdhip.SdhError) as e:
        be.nchw_to_nlc(d, d, 2, 4, 6)  # in place
    assert e.value.status == sdhip.SDH_ERR_INVALID
    with pytest.raises(sdhip.SdhError) as e:
        be.upsample_nearest2x(d, o, 2, 4, 6)  # y smaller than 4x the input
    assert e.value.status == sdhip.SDH_ERR_INVALID


# ---------------------------------------------------------------- vs the compiled reference itself
def test_against_compiled_reference(be, ref, orc):
    """The same checks against oracle/_ref (the reference's tensor.cpp)."""
    x = orc.randn((3, 7, 64), 1)
    g = orc.randn((64,), 2, 1.0, 0.1)
    b = orc.randn((64,), 3, 0.0, 0.1)
    dy = be.empty((3, 7, 64))
    be.layer_norm(be.array(x), dy, 21, 64, be.array(g), be.array(b), 1e-5)
    assert_reduction(dy.download(), ref.layer_norm(x, g, b, 1e-5), "ref layer_norm")
    be.rms_norm(be.array(x), dy, 21, 64, be.array(g), 1e-6)
    assert_reduction(dy.download(), ref.rms_norm(x, g, 1e-6), "ref rms_norm")
    img = orc.randn((2, 64, 5, 7), 4, 0.0, 2.0)
    dyi = be.empty(img.shape)
    be.group_norm(be.array(img), dyi, 2, 64, 35, 32, be.array(g), be.array(b), 1e-6, silu=True)
    assert_reduction(dyi.download(), ref.group_norm(img, 32, g, b, 1e-6, silu=True), "ref group_norm+silu")
    sm = orc.randn((9, 9), 5, 0.0, 3.0)
    dsm = be.array(sm)
    be.softmax_rows(dsm, 9, 9, 0.3, True)
    assert_softmax(dsm.download(), ref.softmax_rows(sm, 0.3, True), "ref softmax causal")
    u = orc.randn((1, 5, 24), 6)
    dsw = be.empty((1, 5, 24))
    be.swiglu(be.array(x.reshape(-1)[:120]), be.array(u), dsw, 120)
    assert_elementwise(dsw.download().reshape(-1), ref.swiglu(x.reshape(-1)[:120], u.reshape(-1)), "ref swiglu")


# ---------------------------------------------------------------- errors and memory
def test_invalid_arguments_fail_cleanly(be):
    d = be.empty((16,))
    with pytest.raises(sdhip.SdhError) as e:
        be.swiglu(d, d, d, 17)  # extent beyond the block
    assert e.value.status == sdhip.SDH_ERR_INVALID
    with pytest.raises(sdhip.SdhError) as e:
        be.group_norm(d, d, 1, 6, 2, 4, d, d, 1e-6)  # C % groups != 0
    assert e.value.status == sdhip.SDH_ERR_INVALID
    host = np.zeros(16, np.float32)
    with pytest.raises(sdhip.SdhError) as e:
        be.silu(host.ctypes.data, 16)  # host pointer
    assert e.value.status == sdhip.SDH_ERR_INVALID
    with pytest.raises(sdhip.SdhError):
        be.rope(d, 1, 2, 8, 3, d, d, True)  # odd dim
    # nothing was launched: the block still holds what we put there
    d.upload(np.arange(16, dtype=np.float32))
    assert np.array_equal(d.download(), np.arange(16, dtype=np.float32))


def test_zero_and_copy(be):
    a = be.array(np.arange(1001, dtype=np.float32))
    b = be.empty((1001,))
    be.check(be.lib.sdh_copy(b.ptr, a.ptr, 1001 * 4))
    assert np.array_equal(b.download(), np.arange(1001, dtype=np.float32))
    be.check(be.lib.sdh_zero(b.ptr + 4, 999 * 4))
    got = b.download()
    assert got[0] == 0.0 and got[1000] == 1000.0 and not np.any(got[1:1000])


def test_arena_reuse(be):
    import gc

    # earlier tests' arrays are freed when the collector finds them: collect
    # first, and keep it off while the bytes in use are compared
    gc.collect()
    gc.disable()
    try:
        before = be.memory_stats()[1]
        for _ in range(5):
            d = be.empty((1 << 20,))
            d.free()
        assert be.memory_stats()[1] == before
    finally:
        gc.enable()
