"""Pins of the attention oracle (oracle/oracle.py: Oracle.attention), without a GPU.

The oracle restates tensor.cpp:776-810 in float64. It is pinned by:
  * the reference's own CPU attention (compiled, oracle/_ref) on the shapes of
    the reference's GPU-vs-CPU checks (test_ops.cpp:440-451) and a few more
    (cross-attention Skv != Sq, d = 40, grouped heads, causal);
  * closed forms: constant values give that constant (the weights sum to
    one); identical keys give the mean of the visible values (uniform
    weights: the causal mask keeps exactly keys 0..i); two keys with scores
    a and 0 give the weights 1/(1 + e^(-a/sqrt(d))) and the rest (the scale);
  * grouped-query heads equal the same heads with k and v expanded
    (test_ops.cpp:259-277);
  * planted mistakes: no 1/sqrt(d), the causal mask one key too wide, key/value
    heads interleaved instead of grouped.
"""
import numpy as np
import pytest

SHAPES = [  # N, Sq, Skv, heads, kv_heads, d, causal
    (2, 9, 9, 3, 3, 8, False), (2, 9, 9, 3, 3, 8, True), (2, 9, 9, 3, 1, 8, False),
    (1, 100, 100, 2, 2, 32, False), (2, 37, 37, 8, 2, 16, True),
    (1, 40, 77, 4, 4, 40, False), (1, 33, 20, 2, 1, 64, True),
]


def _qkv(orc, N, Sq, Skv, heads, kv_heads, d, seed, std=1.0):
    q = orc.randn((N, Sq, heads * d), seed, 0.0, std)
    k = orc.randn((N, Skv, kv_heads * d), seed + 1, 0.0, std)
    v = orc.randn((N, Skv, kv_heads * d), seed + 2)
    return q, k, v


@pytest.mark.parametrize("N,Sq,Skv,heads,kvh,d,causal", SHAPES)
def test_attention_oracle_vs_reference(orc, ref, N, Sq, Skv, heads, kvh, d, causal):
    q, k, v = _qkv(orc, N, Sq, Skv, heads, kvh, d, 1000 + Sq + d)
    want = orc.attention(q, k, v, heads, causal, kvh)
    got = ref.attention(q, k, v, heads, causal, kvh)
    # the reference sums d products and Skv weighted values in fp32
    assert float(np.max(np.abs(got - want))) <= 2e-5


def test_attention_oracle_rows_subset(orc):
    q, k, v = _qkv(orc, 2, 50, 60, 4, 2, 16, 77)
    full = orc.attention(q, k, v, 4, True, 2)
    rows = np.array([0, 7, 31, 49])
    assert np.array_equal(orc.attention(q, k, v, 4, True, 2, rows=rows), full[:, rows])


def _pin_constant_values(orc):
    q, k, _ = _qkv(orc, 1, 12, 12, 2, 2, 8, 5)
    v = np.full((1, 12, 16), 0.75, np.float32)
    for causal in (False, True):
        assert np.allclose(orc.attention(q, k, v, 2, causal), 0.75, rtol=0, atol=1e-12)


def _pin_uniform_weights(orc):
    N, S, heads, d = 1, 10, 2, 8
    q = orc.randn((N, S, heads * d), 6)
    k = np.tile(orc.randn((1, 1, heads * d), 7), (N, S, 1))  # every key the same
    v = orc.randn((N, S, heads * d), 8).astype(np.float64)
    got = orc.attention(q, k, v.astype(np.float32), heads, True)
    want = np.cumsum(v, axis=1) / np.arange(1, S + 1)[None, :, None]  # mean of keys 0..i
    assert np.allclose(got, want, rtol=0, atol=1e-6)
    got = orc.attention(q, k, v.astype(np.float32), heads, False)
    assert np.allclose(got, np.broadcast_to(v.mean(axis=1, keepdims=True), got.shape), rtol=0, atol=1e-6)


def _pin_scale(orc):
    d, a = 4, 1.7
    q = np.array([[[a, 0, 0, 0]]], np.float32)
    k = np.array([[[1, 0, 0, 0], [0, 0, 0, 0]]], np.float32)
    v = np.array([[[1, 0, 0, 0], [0, 1, 0, 0]]], np.float32)
    w0 = 1.0 / (1.0 + np.exp(-a / np.sqrt(d)))
    assert np.allclose(orc.attention(q, k, v, 1)[0, 0], [w0, 1 - w0, 0, 0], rtol=0, atol=1e-7)


def _pin_gqa(orc):
    N, S, heads, kvh, d = 1, 6, 4, 2, 4  # test_ops.cpp:259-277
    q, k, v = _qkv(orc, N, S, S, heads, kvh, d, 9)
    g = np.arange(heads) // (heads // kvh)
    kx = k.reshape(N, S, kvh, d)[:, :, g].reshape(N, S, heads * d)
    vx = v.reshape(N, S, kvh, d)[:, :, g].reshape(N, S, heads * d)
    assert np.allclose(orc.attention(q, k, v, heads, True, kvh), orc.attention(q, kx, vx, heads, True), rtol=0,
                       atol=1e-12)


def test_attention_closed_forms(orc):
    _pin_constant_values(orc)
    _pin_uniform_weights(orc)
    _pin_scale(orc)
    _pin_gqa(orc)


@pytest.mark.parametrize("which,pin", [(10, _pin_scale), (11, _pin_uniform_weights), (12, _pin_gqa)])
def test_attention_pins_catch_planted_mistakes(orc, which, pin):
    pin(orc)
    orc.plant(which)
    try:
        with pytest.raises(AssertionError):
            pin(orc)
    finally:
        orc.plant(0)
