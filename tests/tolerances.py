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
U32 = 2.0 ** -24  # unit roundoff of fp32
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


# ---------------------------------------------------------------- true relative error
# The reductions' bar read elementwise: |got - want| <= 1e-4 * max(|want|,
# floor), floor = TRUE_REL_FLOOR * max|want| (so exact zeros do not divide
# by zero). An fp32 result formed as a sum of terms that nearly cancel (a
# GroupNorm output x*a + b near zero, an LN output where x is near the mean,
# a residual that the gated update nearly cancels) carries the rounding of
# its terms, not of itself, in any fp32 evaluation, the reference's included;
# such an element may exceed the relative bar, and then must be within
# CANCEL_ULPS units of 2^-24 of the terms' magnitude `scale` (computed by
# the caller in float64 from the inputs).
TRUE_REL_FLOOR = 1e-6
CANCEL_ULPS = 8.0


def true_relative_report(got, want, scale=None):
    """(max elementwise relative error, elements beyond the relative bar,
    max error of those in units of 2^-24 * scale)."""
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    if not got.size:
        return 0.0, 0, 0.0
    err = np.abs(got - want)
    floor = TRUE_REL_FLOOR * float(np.max(np.abs(want)))
    rel = err / np.maximum(np.abs(want), max(floor, 1e-300))
    beyond = rel > REDUCTION_REL
    n = int(np.count_nonzero(beyond))
    if n == 0:
        return float(np.max(rel)), 0, 0.0
    if scale is None:
        return float(np.max(rel)), n, float("inf")
    sc = np.broadcast_to(np.asarray(scale, np.float64), got.shape)[beyond]
    ulps = float(np.max(err[beyond] / (U32 * np.maximum(sc, 1e-300))))
    return float(np.max(rel)), n, ulps


def assert_true_relative(got, want, scale=None, what=""):
    """Elementwise relative 1e-4 (floor TRUE_REL_FLOOR * max|want|); elements
    beyond it must be cancellation cases within CANCEL_ULPS of their terms."""
    rel, n, ulps = true_relative_report(got, want, scale)
    print(f"{what}: true relative max {rel:.3e}; {n} of {np.size(want)} elements beyond {REDUCTION_REL} "
          f"(cancellation, max {ulps:.2f} ulp of the terms)", flush=True)
    assert n == 0 or ulps <= CANCEL_ULPS, f"{what}: {n} elements beyond relative {REDUCTION_REL}, {ulps:.2f} ulp"
    return rel, n, ulps


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

def fp32_sum_bound(S, n):
    return n * U32 * np.asarray(S, np.float64)


def assert_gemm(got, want, S, n, what=""):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    bound = fp32_sum_bound(S, n) + 1e-30
    ratio = float(np.max(np.abs(got - want) / bound)) if got.size else 0.0
    assert ratio <= 1.0, f"{what}: error {ratio:.3f} x the fp32 accumulation bound"
    return ratio
