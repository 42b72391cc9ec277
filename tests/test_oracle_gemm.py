"""Pins of the linear (bf16-weight GEMM) oracle, without a GPU.

The oracle (oracle/oracle.py: f32_to_bf16, Oracle.gemm_nt_bf16,
Oracle.linear_swiglu) states the reference's device path: A rounded to bf16
(tensor.cpp:114-121, backend_cuda.cu:183-188), exact bf16 products, and here
an exact (float64) sum. It is pinned by:
  * the rounding: known values (ties to even, carries into the exponent,
    inf/NaN), torch's bfloat16 conversion, and the reference's own
    Tensor::to_bf16 (compiled, oracle/_ref);
  * the GEMM: the reference's CPU linear (tensor.cpp:481-501) fed inputs that
    are already bf16-exact, so that its fp32 sums must agree with the exact
    sums within the fp32 accumulation bound; with and without bias;
  * planted mistakes: A not rounded to bf16, bias broadcast along the wrong
    axis.
The fp32-weight linear (Oracle.gemm_nt_f32) is pinned the same way against the
reference's fp32 CPU path (tensor.cpp:354-406, :498).
"""
import numpy as np
import pytest

from oracle import bf16_to_f32, f32_to_bf16
from tolerances import fp32_sum_bound


def test_bf16_rounding_known_values():
    one = np.float32(1.0)
    ulp = np.float32(2.0 ** -7)  # bf16 spacing at 1.0
    cases = {
        1.0: 0x3F80,
        float(one + ulp / 2): 0x3F80,             # tie, even neighbour below
        float(one + ulp + ulp / 2): 0x3F82,       # tie, even neighbour above
        float(one + ulp / 2 + 2.0 ** -20): 0x3F81,  # just above the tie
        -2.0: 0xC000,
        float(np.float32(3.3895314e38)): 0x7F7F,  # the largest finite bf16, exact
        float(np.finfo(np.float32).max): 0x7F80,  # rounds up into infinity
        float("inf"): 0x7F80,
        float("-inf"): 0xFF80,
        0.0: 0x0000,
    }
    got = f32_to_bf16(np.array(list(cases), np.float32))
    assert [int(g) for g in got] == list(cases.values())
    nan = np.array([0x7FC12345], np.uint32).view(np.float32)
    assert int(f32_to_bf16(nan)[0]) == 0x7FC1  # NaN keeps its top bits


def test_bf16_rounding_matches_torch_and_reference(orc, ref):
    import torch

    x = np.concatenate([orc.randn((4096,), 5, 0.0, 3.0), orc.randn((4096,), 6, 0.0, 1e-30),
                        orc.randn((4096,), 7, 0.0, 1e30)])
    ours = f32_to_bf16(x)
    t = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, t)
    assert np.array_equal(ours, ref.to_bf16(x))


def _bf16_exact(orc, shape, seed, std=1.0):
    return bf16_to_f32(f32_to_bf16(orc.randn(shape, seed, 0.0, std)))


@pytest.mark.parametrize("M,N,K", [(5, 7, 16), (33, 130, 72), (64, 96, 512)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_gemm_oracle_vs_reference_linear(orc, ref, M, N, K, with_bias):
    a = _bf16_exact(orc, (M, K), 11 + K)
    w = _bf16_exact(orc, (N, K), 12 + N, 0.05)
    b = orc.randn((N,), 13, 0.0, 0.1) if with_bias else None
    want, S = orc.gemm_nt_bf16(a, f32_to_bf16(w), b)
    got = ref.linear(a, w, b)
    # the reference sums K products in fp32 (4x4 micro-kernel, k in order) plus the bias
    assert np.all(np.abs(got - want) <= fp32_sum_bound(S, K + 1) + 1e-30), "oracle gemm vs reference linear"


def test_gemm_oracle_accumulate_and_swiglu(orc):
    a = orc.randn((9, 40), 21)
    w1, w3 = f32_to_bf16(orc.randn((24, 40), 22, 0.0, 0.2)), f32_to_bf16(orc.randn((24, 40), 23, 0.0, 0.2))
    c0 = orc.randn((9, 24), 24)
    acc, _ = orc.gemm_nt_bf16(a, w1, None, c0, accumulate=True)
    plain, _ = orc.gemm_nt_bf16(a, w1)
    assert np.allclose(acc, c0.astype(np.float64) + plain, rtol=1e-6, atol=1e-6)
    y, g, u, _, _ = orc.linear_swiglu(a, w1, w3)
    assert np.allclose(y, orc.swiglu(g, u), rtol=2e-6, atol=1e-7)  # same composition as the elementwise swiglu


def _pin_rounding(orc, ref):
    a = orc.randn((8, 64), 31)  # NOT bf16-exact: the reference is given A already rounded
    w = _bf16_exact(orc, (16, 64), 32, 0.1)
    want, S = orc.gemm_nt_bf16(a, f32_to_bf16(w))
    got = ref.linear(bf16_to_f32(f32_to_bf16(a)), w)
    assert np.all(np.abs(got - want) <= fp32_sum_bound(S, 65) + 1e-30)


def _pin_bias(orc, ref):
    a = _bf16_exact(orc, (6, 32), 33)
    w = _bf16_exact(orc, (10, 32), 34, 0.1)
    b = orc.randn((10,), 35, 0.0, 1.0)
    want, S = orc.gemm_nt_bf16(a, f32_to_bf16(w), b)
    got = ref.linear(a, w, b)
    assert np.all(np.abs(got - want) <= fp32_sum_bound(S, 33) + 1e-6)


@pytest.mark.parametrize("which,pin", [(8, _pin_rounding), (9, _pin_bias)])
def test_gemm_pins_catch_planted_mistakes(orc, ref, which, pin):
    pin(orc, ref)
    orc.plant(which)
    try:
        with pytest.raises(AssertionError):
            pin(orc, ref)
    finally:
        orc.plant(0)


@pytest.mark.parametrize("M,N,K", [(5, 7, 16), (70, 130, 64), (9, 64, 200), (1, 256, 33)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_gemm_f32_oracle_vs_reference_linear(orc, ref, M, N, K, with_bias):
    a = orc.randn((M, K), 41 + K)
    w = orc.randn((N, K), 42 + N, 0.0, 0.05)
    b = orc.randn((N,), 43, 0.0, 0.1) if with_bias else None
    want, S = orc.gemm_nt_f32(a, w, b)
    got = ref.linear(a, w, b, bf16=False)
    assert np.all(np.abs(got - want) <= fp32_sum_bound(S + (np.abs(b)[None, :] if with_bias else 0), K + 1) + 1e-30)
    # and the bf16 path differs from it: the pin tells the two apart
    assert float(np.max(np.abs(ref.linear(a, w, b) - want))) > 1e-4
