"""Parity metrics and the tolerances the parity tests apply.

The bar: match the reference's CPU implementation
on identical seeded fp32 inputs within
  * max-abs 1e-5 for pure elementwise ops (swiglu, silu, tanh, gelu,
    quick_gelu, geglu, rope, add, scale, affine, mul_rows, add_rows_scaled,
    add_rows, add_channel_bias);
  * relative 1e-4 for reductions and softmax.
"Relative" is made precise here:
  * reductions (norms and the fused norm ops): max_i |got_i - want_i| /
    max(|want_i|, 1) -- truly relative where |want| >= 1, absolute 1e-4 below
    (the reference's own GPU-vs-CPU norm checks use max-abs 1e-4,
    tests/test_ops.cpp:392-401);
  * softmax: max_i |got_i - want_i| / max(|want_i|, 1e-30), i.e. elementwise
    relative, and entries the reference sets to exactly 0 (causal tail) must be
    exactly 0.
"""
import numpy as np

ELEMENTWISE_ABS = 1e-5
REDUCTION_REL = 1e-4
SOFTMAX_REL = 1e-4


def max_abs(got, want) -> float:
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    return float(np.max(np.abs(got - want))) if got.size else 0.0


def rel_floor1(got, want) -> float:
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    return float(np.max(np.abs(got - want) / np.maximum(np.abs(want), 1.0))) if got.size else 0.0


def rel_softmax(got, want) -> float:
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    zeros = want == 0
    if np.any(got[zeros] != 0):
        return float("inf")
    return float(np.max(np.abs(got - want) / np.maximum(np.abs(want), 1e-30))) if got.size else 0.0


def assert_elementwise(got, want, what=""):
    e = max_abs(got, want)
    assert e <= ELEMENTWISE_ABS, f"{what}: max-abs {e:.3e} > {ELEMENTWISE_ABS}"
    return e


def assert_reduction(got, want, what=""):
    e = rel_floor1(got, want)
    assert e <= REDUCTION_REL, f"{what}: rel {e:.3e} > {REDUCTION_REL}"
    return e


def assert_softmax(got, want, what=""):
    e = rel_softmax(got, want)
    assert e <= SOFTMAX_REL, f"{what}: rel {e:.3e} > {SOFTMAX_REL}"
    return e


# ---------------------------------------------------------------- GEMM
# A bf16-weight GEMM accumulates exact bf16 products in fp32, in an order the
# hardware (MFMA) or the reference's micro-kernel chooses. Against the exact
# sum of the same products the classic recursive-summation bound applies
# whatever the order: |error| <= n u sum_k |a_k b_k| (u = 2^-24, n the number
# of terms, bias and accumulated C counted as terms). It is rigorous, yet
# tight enough that an indexing mistake (a dropped K tile, a transposed
# operand, a missing bf16 rounding of A) exceeds it by orders of magnitude.
U32 = 2.0 ** -24


def fp32_sum_bound(S, n):
    return n * U32 * np.asarray(S, np.float64)


def assert_gemm(got, want, S, n, what=""):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    bound = fp32_sum_bound(S, n) + 1e-30
    ratio = float(np.max(np.abs(got - want) / bound)) if got.size else 0.0
    assert ratio <= 1.0, f"{what}: error {ratio:.3f} x the fp32 accumulation bound"
    return ratio
