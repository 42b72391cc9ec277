"""GPU tests of the opt-in reduced-precision attention (sdh_attention_fp16,
no counterpart in the reference), through the C ABI.

The kernel rounds its operands to fp16 after a power-of-two block scaling:
q per (query row, head), k and v per (64-key tile, key/value head), each
block scaled so that its largest magnitude lies in [2^13, 2^14), then
rounded to nearest even. `_round_like_kernel` applies exactly that rounding
in numpy, and the float64 oracle evaluated on the rounded operands is the
reference here. What the kernel adds beyond it is the fp16 rounding of the
softmax weights: each weight moves by at most 2^-11 of itself (weights stay
in fp16's normal range relative to the largest one; the sum of the weights is
kept in fp32 from the unrounded values), so an output moves by at most
2^-11 max|v| (the weighted mean of the |v| perturbations), plus fp32
accumulation error; the bar is 2^-11 max|v| + 2e-6 max|v|. A dropped term, a
wrong index or a wrong scale gives errors of order max|v|.

The end-to-end check: the Z-Image forward with fp16 attention against the
reference's own CPU forward (oracle/_ref), relative RMS 2e-2 (the DiT's bar,
test_zimage.cpp:74-77), on the small model of tests/zimage_model.py.
"""
import numpy as np
import pytest

import zimage_model as zm

pytestmark = pytest.mark.gpu


def _block_exp(amax):
    """The kernel's block exponent (k_attention.hip block_exp): biased
    exponent f of amax, e = f - 140 clamped to [-126, 126]; 0 for zero,
    subnormal, inf or NaN maxima."""
    f = (np.asarray(amax, np.float32).view(np.uint32) >> 23) & 0xFF
    e = np.clip(f.astype(np.int64) - 140, -126, 126)
    return np.where((f == 0) | (f == 255), 0, e)


def _round_blocks(x, e):
    """x * 2^-e rounded to fp16 (round to nearest even), scaled back, in float64."""
    s = np.ldexp(np.ones_like(x, dtype=np.float64), -e)
    return (x.astype(np.float64) * s).astype(np.float32).astype(np.float16).astype(np.float64) / s


def _round_like_kernel(q, k, v, heads, kvh):
    N, Sq, inner = q.shape
    d = inner // heads
    Skv = k.shape[1]
    q4 = q.reshape(N, Sq, heads, d)
    eq = _block_exp(np.max(np.abs(q4), axis=3, keepdims=True))
    qr = _round_blocks(q4, eq).reshape(q.shape)
    nt = (Skv + 63) // 64
    out = []
    for x in (k, v):
        x4 = x.reshape(N, Skv, kvh, d)
        pad = np.zeros((N, nt * 64, kvh, d), np.float32)
        pad[:, :Skv] = x4
        t = pad.reshape(N, nt, 64, kvh, d)
        e = _block_exp(np.max(np.abs(t), axis=(2, 4), keepdims=True))
        out.append(_round_blocks(t, e).reshape(N, nt * 64, kvh, d)[:, :Skv].reshape(x.shape))
    return qr, out[0], out[1]


def _run(be, q, k, v, heads, kvh, causal, out_bf16=False):
    N, Sq, inner = q.shape
    Skv = k.shape[1]
    d = inner // heads
    import sdhip

    out = sdhip.DArray(be, (N, Sq, inner), dtype=np.uint16) if out_bf16 else be.empty((N, Sq, inner))
    be.attention_fp16(be.array(q), be.array(k), be.array(v), out, N, Sq, Skv, heads, kvh, d, causal,
                      out_bf16=out_bf16)
    return out.download()


def _check(orc, got, q, k, v, heads, kvh, causal, what, rows=None):
    qr, kr, vr = _round_like_kernel(q, k, v, heads, kvh)
    want = orc.attention(qr.astype(np.float32), kr.astype(np.float32), vr.astype(np.float32), heads, causal, kvh,
                         **({} if rows is None else {"rows": rows}))
    if rows is not None:
        got = got[:, rows]
    vmax = float(np.max(np.abs(v)))
    bar = (2.0 ** -11 + 2e-6) * vmax
    err = float(np.max(np.abs(got.astype(np.float64) - want)))
    exact = orc.attention(q, k, v, heads, causal, kvh, **({} if rows is None else {"rows": rows}))
    err32 = float(np.max(np.abs(got.astype(np.float64) - exact)))
    print(f"{what}: vs rounded-operand oracle {err:.3g} (bar {bar:.3g}); vs fp32 oracle {err32:.3g}")
    assert err <= bar, f"{what}: {err:.3g} > {bar:.3g}"
    return err32


SHAPES = [  # N, Sq, Skv, heads, kv_heads, d, causal (d <= 128: the fp16 path)
    (2, 9, 9, 3, 3, 8, False), (2, 9, 9, 3, 1, 8, True), (1, 100, 100, 2, 2, 32, False),
    (2, 37, 37, 8, 2, 16, True), (1, 300, 77, 8, 8, 40, False), (2, 257, 257, 5, 5, 64, True),
    (1, 130, 70, 4, 2, 80, False), (1, 513, 513, 2, 1, 128, True), (1, 64, 64, 1, 1, 128, False),
    (1, 1, 1, 1, 1, 64, False), (1, 1, 300, 2, 2, 128, False), (3, 65, 129, 6, 3, 100, True),
]


@pytest.mark.parametrize("N,Sq,Skv,heads,kvh,d,causal", SHAPES)
def test_attention_fp16_parity(be, orc, N, Sq, Skv, heads, kvh, d, causal):
    seed = 8000 + Sq + Skv + d
    q = orc.randn((N, Sq, heads * d), seed)
    k = orc.randn((N, Skv, kvh * d), seed + 1)
    v = orc.randn((N, Skv, kvh * d), seed + 2)
    got = _run(be, q, k, v, heads, kvh, causal)
    _check(orc, got, q, k, v, heads, kvh, causal, f"fp16 attention {N}x{Sq}x{Skv} h{heads}/{kvh} d{d} c={causal}")


@pytest.mark.parametrize("std_qk,std_v", [(3.0, 1.0), (10.0, 1.0), (30.0, 100.0), (1e-3, 1e-3), (1e-20, 1e15)])
def test_attention_fp16_input_range(be, orc, std_qk, std_v):
    """Score spreads of 9 to 900 (near one-hot weights), tiny scores, and
    values beyond fp16's range (the block scaling brings them in)."""
    q = orc.randn((1, 160, 512), 8100, 0.0, std_qk)
    k = orc.randn((1, 200, 512), 8101, 0.0, std_qk)
    v = orc.randn((1, 200, 512), 8102, 0.0, std_v)
    got = _run(be, q, k, v, 4, 4, False)
    _check(orc, got, q, k, v, 4, 4, False, f"fp16 attention std_qk={std_qk} std_v={std_v}")


def test_attention_fp16_zimage_layer(be, orc):
    """The Z-Image DiT layer [1, 4096, 30 x 128] on sampled query rows, both
    output forms (the bf16 one is the fp32 result rounded to bf16)."""
    S, heads, d = 4096, 30, 128
    q = orc.randn((1, S, heads * d), 8200)
    k = orc.randn((1, S, heads * d), 8201)
    v = orc.randn((1, S, heads * d), 8202)
    rows = np.concatenate([np.arange(0, S, 131), [S - 1]])
    got = _run(be, q, k, v, heads, heads, False)
    err32 = _check(orc, got, q, k, v, heads, heads, False, "fp16 attention Z-Image layer", rows=rows)
    assert err32 <= 1e-2  # against exact fp32 attention: operand rounding on unit-variance data
    got16 = _run(be, q, k, v, heads, heads, False, out_bf16=True)
    bits = got.view(np.uint32).astype(np.uint64)
    rne = ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16).astype(np.uint16)
    assert np.array_equal(got16, rne), "bf16 output is not the bf16 rounding of the fp32 output"


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    W = zm.make_weights(0)
    path = tmp_path_factory.mktemp("zimage_fp16") / "model.safetensors"
    zm.write_safetensors(path, W)
    return W, path


@pytest.mark.parametrize("H,W,L,t", [(16, 16, 20, 0.3), (24, 20, 40, 0.9)])
def test_zimage_fp16_attention_vs_reference_cpu(be, ref, orc, model, H, W, L, t):
    import sdhip

    _, path = model
    x, cap = zm.inputs(orc, H=H, W=W, L=L)
    for keep_bf16 in (True, False):
        m = sdhip.ZImage.load(path, heads=zm.SHAPES["heads"], keep_bf16=keep_bf16, bf16_min_numel=zm.BF16_MIN)
        try:
            m.set_fp16_attention(True)
            got = m.forward(x, t, cap)
            m.set_fp16_attention(False)
            exact = m.forward(x, t, cap)
        finally:
            m.close()
        want = ref.zimage_forward(path, x, t, cap, zm.SHAPES["heads"], keep_bf16, zm.BF16_MIN)
        e, e0 = zm.rel_rms(got, want), zm.rel_rms(exact, want)
        print(f"{H}x{W} L{L} keep_bf16={keep_bf16}: relative RMS vs the reference CPU forward: "
              f"fp16 attention {e:.3g}, default attention {e0:.3g}")
        assert e <= 2e-2
        assert not np.array_equal(got, exact)  # the switch took effect
