"""GPU tests of the Z-Image block's fused entry points against the op
sequences they replace, through the C ABI. Each fused op is claimed equal to
its sequence bit for bit (same fp32 expressions in the same order, then the
same bf16 rounding), so the bar is exact equality:
  * sdh_rms_norm_modulate_bf16 == rms_norm -> mul_rows -> to_bf16
    (zimage.cpp:115-116, :128-129, then gemm_nt_bf16's rounding of A);
  * sdh_rms_norm_gated_add == rms_norm -> add_rows_scaled (or add_)
    (zimage.cpp:124-127, :132-135);
  * sdh_rms_norm_gated_add_modulate_bf16 == sdh_rms_norm_gated_add ->
    sdh_rms_norm_modulate_bf16 (zimage.cpp:124-129, one sublayer's close and
    the next one's input);
  * sdh_modulation_rows == affine_(1, 1) / tanh_ on alternate rows
    (zimage.cpp:104-107);
  * sdh_swiglu_bf16 == swiglu -> to_bf16 (zimage.cpp:130, the input of w2);
  * sdh_gemm_nt_bf16_packed(bf16 A) == sdh_gemm_nt_bf16(the same values in
    fp32), and within the fp32 accumulation bound of the exact sum for the
    strided A and the hand-written kernels' shapes.
Shapes: the Z-Image rows [4224, 3840], small and odd row widths (the generic
kernels), optional gamma / scale / gate.

The second half of the file checks the same fused entry points against the
CPU oracle directly (the reference's composition), not only against the
GPU's op sequence.
"""
import numpy as np
import pytest

from oracle import bf16_to_f32, f32_to_bf16
from tolerances import assert_gemm

pytestmark = pytest.mark.gpu

ROWS = [(4224, 3840), (5, 64), (33, 100), (7, 30)]


def _u16(be, n):
    return be.array(np.zeros(n, np.uint16))


@pytest.mark.parametrize("rows,C", ROWS)
@pytest.mark.parametrize("with_gamma,with_scale", [(True, True), (True, False), (False, True), (False, False)])
def test_rms_norm_modulate_bf16(be, orc, rows, C, with_gamma, with_scale):
    x = orc.randn((rows, C), 700 + C, 0.0, 2.0)
    g = orc.randn((C,), 701, 1.0, 0.1) if with_gamma else None
    s = orc.randn((C,), 702, 1.0, 0.3) if with_scale else None
    dx = be.array(x)
    dg, ds = (be.array(g) if with_gamma else None), (be.array(s) if with_scale else None)
    y16 = _u16(be, rows * C)
    be.rms_norm_modulate_bf16(dx, y16, rows, C, dg, ds, 1e-5)
    h = be.empty((rows, C))
    be.rms_norm(dx, h, rows, C, dg, 1e-5)
    if with_scale:
        be.mul_rows(h, ds, rows, C)
    ref16 = _u16(be, rows * C)
    be.to_bf16(h, ref16, rows * C)
    got, want = y16.download(), ref16.download()
    assert np.array_equal(got, want), f"{int(np.sum(got != want))} of {got.size} differ"
    # and against the oracle's composition: the same value to within one bf16 step
    o = orc.rms_norm(x, g, 1e-5)
    if with_scale:
        o = orc.mul_rows(o, s)
    assert np.max(np.abs(bf16_to_f32(got).reshape(rows, C) - o) / np.maximum(np.abs(o), 1e-30)) <= 2.0 ** -8


@pytest.mark.parametrize("rows,C", ROWS)
@pytest.mark.parametrize("with_gamma,with_gate", [(True, True), (True, False), (False, True)])
def test_rms_norm_gated_add(be, orc, rows, C, with_gamma, with_gate):
    x = orc.randn((rows, C), 710 + C)
    a = orc.randn((rows, C), 711 + C, 0.0, 3.0)
    g = orc.randn((C,), 712, 1.0, 0.1) if with_gamma else None
    gate = orc.randn((C,), 713, 0.0, 0.5) if with_gate else None
    dg, dgate = (be.array(g) if with_gamma else None), (be.array(gate) if with_gate else None)
    dx, da = be.array(x), be.array(a)
    be.rms_norm_gated_add(dx, da, rows, C, dg, dgate, 1e-5)
    seq_x = be.array(x)
    an = be.empty((rows, C))
    be.rms_norm(da, an, rows, C, dg, 1e-5)
    if with_gate:
        be.add_rows_scaled(seq_x, an, dgate, rows, C)
    else:
        be.add(seq_x, an, rows * C)
    assert np.array_equal(dx.download(), seq_x.download())
    assert np.array_equal(da.download(), a)  # a is read only


@pytest.mark.parametrize("n,off", [(4224 * 10240, 0), (1001, 0), (1003, 1)])
def test_swiglu_bf16(be, orc, n, off):
    g = orc.randn((n + off,), 720, 0.0, 1.5)
    u = orc.randn((n + off,), 721, 0.0, 1.5)
    dg, du = be.array(g), be.array(u)
    y16 = _u16(be, n + 1)
    # off = 1: unaligned operands take the scalar kernel
    import sdhip

    gp = sdhip.DArray(be, (n,), ptr=dg.ptr + 4 * off, owned=False)
    upp = sdhip.DArray(be, (n,), ptr=du.ptr + 4 * off, owned=False)
    yp = sdhip.DArray(be, (n,), ptr=y16.ptr + 2 * off, owned=False, dtype=np.uint16)
    be.swiglu_bf16(gp, upp, yp, n)
    y = be.empty((n,))
    be.swiglu(gp, upp, y, n)
    ref16 = _u16(be, n)
    be.to_bf16(y, ref16, n)
    assert np.array_equal(y16.download()[off:off + n], ref16.download())


@pytest.mark.parametrize("M,N,K,lda", [(4224, 3840, 3840, 3840), (300, 200, 128, 136), (70, 130, 64, 64)])
def test_gemm_packed_equals_gemm_on_rounded_a(be, orc, M, N, K, lda):
    A = bf16_to_f32(f32_to_bf16(orc.randn((M, lda), 730 + M))).reshape(M, lda)
    W = f32_to_bf16(orc.randn((N, K), 731, 0.0, 0.05))
    b = orc.randn((N,), 732, 0.0, 0.5)
    dW, db = be.array(W), be.array(b)
    c1 = be.empty((M, N))
    be.gemm_nt_bf16_packed(M, N, K, be.array(f32_to_bf16(A)), lda, dW, K, c1, N, db)
    c0 = be.empty((M, N))
    be.gemm_nt_bf16(M, N, K, be.array(A), lda, dW, K, c0, N, db)
    got = c1.download()
    if lda == K:
        assert np.array_equal(got, c0.download())
    rows = np.arange(0, M, max(1, M // 50))
    want, S = orc.gemm_nt_bf16(A[rows, :K], W, b)
    assert_gemm(got[rows], want, S + np.abs(b)[None, :], K + 2, f"packed gemm {M}x{N}x{K}")


def test_gemm_packed_mfma_kernels(be, orc):
    """ldc not a multiple of 4: the hand-written MFMA kernels (hipBLASLt needs
    aligned leading dimensions), K % 64 == 0 and K % 64 != 0."""
    for (M, N, K) in ((257, 129, 192), (65, 70, 72)):
        A = bf16_to_f32(f32_to_bf16(orc.randn((M, K), 740 + K))).reshape(M, K)
        W = f32_to_bf16(orc.randn((N, K), 741, 0.0, 0.05))
        ldc = N + 1
        C = be.array(np.zeros((M, ldc), np.float32))
        be.gemm_nt_bf16_packed(M, N, K, be.array(f32_to_bf16(A)), K, be.array(W), K, C, ldc)
        want, S = orc.gemm_nt_bf16(A, W)
        assert_gemm(C.download()[:, :N], want, S, K + 1, f"packed mfma {M}x{N}x{K}")


@pytest.mark.parametrize("N,Sq,Skv,heads,kvh,d,causal", [(1, 300, 300, 3, 3, 128, False), (2, 70, 130, 4, 2, 64, True),
                                                          (1, 33, 40, 2, 2, 200, False), (1, 65, 65, 2, 1, 100, True),
                                                          (1, 5, 0, 2, 2, 64, False)])
def test_attention_bf16(be, orc, N, Sq, Skv, heads, kvh, d, causal):
    """sdh_attention_bf16 == sdh_attention then the GEMM's rounding of A, bit
    for bit: the MFMA kernel (d = 64, 128; d = 100 takes its scalar stores),
    the generic kernel (d = 200), grouped heads, causal, no keys."""
    q = orc.randn((N, Sq, heads * d), 750 + d)
    k = orc.randn((N, Skv, kvh * d), 751 + d)
    v = orc.randn((N, Skv, kvh * d), 752 + d)
    dq = be.array(q)
    dk = be.array(k) if Skv else be.empty((1,))
    dv = be.array(v) if Skv else be.empty((1,))
    n = N * Sq * heads * d
    o16 = _u16(be, n)
    be.attention_bf16(dq, dk, dv, o16, N, Sq, Skv, heads, kvh, d, causal)
    o = be.empty((N, Sq, heads * d))
    be.attention(dq, dk, dv, o, N, Sq, Skv, heads, kvh, d, causal)
    ref16 = _u16(be, n)
    be.to_bf16(o, ref16, n)
    got, want = o16.download(), ref16.download()
    assert np.array_equal(got, want), f"{int(np.sum(got != want))} of {got.size} differ"


@pytest.mark.parametrize("pairs,dim", [(2, 3840), (2, 37), (3, 8)])
def test_modulation_rows_equals_affine_and_tanh(be, orc, pairs, dim):
    """sdh_modulation_rows on [2P, D] equals affine_(row 2p, 1, 1) and
    tanh_(row 2p + 1), bit for bit (zimage.cpp:104-107)."""
    x = orc.randn((2 * pairs, dim), 9300 + dim, 0.0, 2.0)
    dx = be.array(x)
    be.modulation_rows(dx, pairs, dim)
    got = dx.download()
    want = be.array(x)
    for p in range(pairs):
        be.affine(_row(be, want, 2 * p, dim), 1.0, 1.0, dim)
        be.tanh(_row(be, want, 2 * p + 1, dim), dim)
    assert np.array_equal(got, want.download())


def _row(be, arr, r, dim):
    import sdhip

    return sdhip.DArray(be, (dim,), ptr=arr.ptr + 4 * r * dim, owned=False)


FUSED_ROWS = [(4224, 3840), (600, 3840), (128, 3840), (1, 3840), (64, 3072), (9, 2080), (70, 512), (33, 1000), (5, 64), (7, 30)]


@pytest.mark.parametrize("rows,C", FUSED_ROWS)
@pytest.mark.parametrize("vecs", [(True, True, True, True), (True, False, True, False), (False, True, False, True)])
def test_rms_norm_gated_add_modulate_bf16(be, orc, rows, C, vecs):
    """residual add + RMSNorm + modulate == sdh_rms_norm_gated_add then
    sdh_rms_norm_modulate_bf16, bit for bit, x and y (every kernel shape:
    workgroup per row with and without paired stores, wave per row with and
    without, the two-op path for rows not a multiple of 4)."""
    has_g1, has_gate, has_g2, has_scale = vecs
    x = orc.randn((rows, C), 730 + C)
    a = orc.randn((rows, C), 731 + C, 0.0, 3.0)
    vec = lambda on, seed, mu, sd: be.array(orc.randn((C,), seed, mu, sd)) if on else None
    g1, gate = vec(has_g1, 732, 1.0, 0.1), vec(has_gate, 733, 0.0, 0.5)
    g2, scale = vec(has_g2, 734, 1.0, 0.1), vec(has_scale, 735, 1.0, 0.3)
    dx, da = be.array(x), be.array(a)
    y16 = _u16(be, rows * C)
    be.rms_norm_gated_add_modulate_bf16(dx, da, y16, rows, C, g1, gate, g2, scale, 1e-5, 1e-6)
    sx = be.array(x)
    be.rms_norm_gated_add(sx, da, rows, C, g1, gate, 1e-5)
    s16 = _u16(be, rows * C)
    be.rms_norm_modulate_bf16(sx, s16, rows, C, g2, scale, 1e-6)
    got_x, want_x = dx.download(), sx.download()
    assert np.array_equal(got_x, want_x), f"x: {int(np.sum(got_x != want_x))} of {got_x.size} differ"
    got, want = y16.download(), s16.download()
    assert np.array_equal(got, want), f"y: {int(np.sum(got != want))} of {got.size} differ"
    assert np.array_equal(da.download(), a)  # a is read only


def test_rms_norm_gated_add_modulate_bf16_unaligned_y(be, orc):
    """y 8 bytes past a 16-byte boundary (the unpaired stores)."""
    import sdhip

    rows, C = 40, 3840
    x = orc.randn((rows, C), 740)
    a = orc.randn((rows, C), 741)
    g = be.array(orc.randn((C,), 742, 1.0, 0.1))
    s = be.array(orc.randn((C,), 743, 1.0, 0.3))
    dx, da = be.array(x), be.array(a)
    buf = _u16(be, rows * C + 4)
    y16 = sdhip.DArray(be, (rows * C,), ptr=buf.ptr + 8, owned=False, dtype=np.uint16)
    be.rms_norm_gated_add_modulate_bf16(dx, da, y16, rows, C, g, s, g, s, 1e-5)
    sx = be.array(x)
    be.rms_norm_gated_add(sx, da, rows, C, g, s, 1e-5)
    s16 = _u16(be, rows * C)
    be.rms_norm_modulate_bf16(sx, s16, rows, C, g, s, 1e-5)
    assert np.array_equal(dx.download(), sx.download())
    assert np.array_equal(y16.download(), s16.download())


def test_rms_norm_gated_add_modulate_bf16_rejects_overlap(be, orc):
    import sdhip

    rows, C = 4, 256
    dx, da = be.array(orc.randn((rows, C), 744)), be.array(orc.randn((rows, C), 745))
    y_on_a = sdhip.DArray(be, (rows * C,), ptr=da.ptr, owned=False, dtype=np.uint16)
    with pytest.raises(sdhip.SdhError, match="overlaps"):
        be.rms_norm_gated_add_modulate_bf16(dx, da, y_on_a, rows, C, None, None, None, None, 1e-5)


# ---------------------------------------------------------------- against the oracle
# The bit-equality tests above compare each fused kernel with the GPU's own
# op sequence. These compare the fused kernels with the CPU oracle directly
# (the reference's composition, zimage.cpp:104-107, :122-133, over
# tensor.cpp:660-679, :889-917, :732-748, :850-853, :884-887):
#   * x, the gated residual: relative 1e-4 elementwise (a reduction's bar),
#     cancellation elements within a few ulp of their terms |x| + |gate * an|;
#   * y16, the next sublayer's bf16 input: the bf16 pattern of the GPU value
#     and the nearest-even bf16 of the oracle's fp32 value (the oracle's
#     RMSNorm and modulate applied to the x the kernel produced) differ by at
#     most one unit in the last place (the fp32 values differ by the
#     reductions' rounding, which moves a value across a bf16 rounding
#     boundary at most);
#   * swiglu_bf16 the same way; modulation rows at max-abs 1e-5.

def _bf16_within_one_ulp(got16, want32, what):
    want16 = f32_to_bf16(np.ascontiguousarray(want32, np.float32)).reshape(-1)
    got16 = np.asarray(got16, np.uint16).reshape(-1)
    # patterns of one sign are ordered like their magnitudes; a sign change
    # across zero is allowed only between the two smallest patterns
    d = np.abs(got16.astype(np.int64) - want16.astype(np.int64))
    sign_flip = (got16 >> 15) != (want16 >> 15)
    tiny = ((got16 & 0x7FFF) <= 1) & ((want16 & 0x7FFF) <= 1)
    bad = np.where(sign_flip, ~tiny, d > 1)
    n_off = int(np.count_nonzero(d != 0))
    print(f"{what}: {n_off} of {d.size} bf16 values one ulp from the oracle's rounding, "
          f"{int(np.count_nonzero(bad))} beyond", flush=True)
    assert not np.any(bad), f"{what}: {int(np.count_nonzero(bad))} bf16 values beyond one ulp of the oracle"


def _gated_add_oracle(orc, x, a, g1, gate, eps1):
    an = orc.rms_norm(a, g1, eps1)
    if gate is None:
        return orc.add(x, an), np.abs(x.astype(np.float64)) + np.abs(an.astype(np.float64))
    return (orc.add_rows_scaled(x, an, gate),
            np.abs(x.astype(np.float64)) + np.abs(an.astype(np.float64) * gate.astype(np.float64)))


ORACLE_ROWS = [(4224, 3840), (128, 3840), (13, 3840), (33, 1000), (7, 30)]


@pytest.mark.parametrize("rows,C", ORACLE_ROWS)
@pytest.mark.parametrize("vecs", [(True, True, True, True), (False, False, False, False), (True, False, False, True)])
def test_rms_norm_gated_add_modulate_bf16_vs_oracle(be, orc, rows, C, vecs):
    """Residual add + RMSNorm + modulate (the north star's fused variant)
    against the oracle's rms_norm -> add_rows_scaled_ -> rms_norm ->
    mul_rows_ (zimage.cpp:124-129)."""
    from tolerances import assert_true_relative

    has_g1, has_gate, has_g2, has_scale = vecs
    x = orc.randn((rows, C), 760 + C)
    a = orc.randn((rows, C), 761 + C, 0.0, 3.0)
    vec = lambda on, seed, mu, sd: orc.randn((C,), seed, mu, sd) if on else None
    g1, gate = vec(has_g1, 762, 1.0, 0.1), vec(has_gate, 763, 0.0, 0.5)
    g2, scale = vec(has_g2, 764, 1.0, 0.1), vec(has_scale, 765, 1.0, 0.3)
    dv = lambda v: be.array(v) if v is not None else None
    dx, da = be.array(x), be.array(a)
    y16 = _u16(be, rows * C)
    be.rms_norm_gated_add_modulate_bf16(dx, da, y16, rows, C, dv(g1), dv(gate), dv(g2), dv(scale), 1e-5, 1e-6)
    want_x, terms = _gated_add_oracle(orc, x, a, g1, gate, 1e-5)
    got_x = dx.download().reshape(rows, C)
    assert_true_relative(got_x, want_x, terms, f"gated add x [{rows},{C}] {vecs}")
    # y from the x the kernel produced: an element of x that its terms nearly
    # cancel carries their rounding (checked just above), and y's element is
    # that x times a row factor, so it carries the same relative error; the
    # modulate stage itself is pinned on its actual input
    h = orc.rms_norm(got_x, g2, 1e-6)
    if has_scale:
        h = orc.mul_rows(h, scale)
    _bf16_within_one_ulp(y16.download(), h, f"modulated y16 [{rows},{C}] {vecs}")


@pytest.mark.parametrize("rows,C", ORACLE_ROWS)
@pytest.mark.parametrize("with_gamma,with_gate", [(True, True), (False, False)])
def test_rms_norm_gated_add_vs_oracle(be, orc, rows, C, with_gamma, with_gate):
    """x += gate * rms_norm(a) * g against the oracle's rms_norm ->
    add_rows_scaled_ (zimage.cpp:124-127), or add_ without a gate."""
    from tolerances import assert_true_relative

    x = orc.randn((rows, C), 770 + C)
    a = orc.randn((rows, C), 771 + C, 0.0, 3.0)
    g = orc.randn((C,), 772, 1.0, 0.1) if with_gamma else None
    gate = orc.randn((C,), 773, 0.0, 0.5) if with_gate else None
    dx = be.array(x)
    be.rms_norm_gated_add(dx, be.array(a), rows, C, be.array(g) if with_gamma else None,
                          be.array(gate) if with_gate else None, 1e-5)
    want_x, terms = _gated_add_oracle(orc, x, a, g, gate, 1e-5)
    assert_true_relative(dx.download().reshape(rows, C), want_x, terms, f"rms_norm_gated_add [{rows},{C}]")


@pytest.mark.parametrize("rows,C", ORACLE_ROWS)
@pytest.mark.parametrize("with_gamma,with_scale", [(True, True), (False, False)])
def test_rms_norm_modulate_bf16_vs_oracle(be, orc, rows, C, with_gamma, with_scale):
    """RMSNorm * scale -> bf16 against the oracle's rms_norm -> mul_rows_
    (zimage.cpp:115-116, :128-129), then nearest-even bf16."""
    x = orc.randn((rows, C), 780 + C, 0.0, 2.0)
    g = orc.randn((C,), 781, 1.0, 0.1) if with_gamma else None
    s = orc.randn((C,), 782, 1.0, 0.3) if with_scale else None
    y16 = _u16(be, rows * C)
    be.rms_norm_modulate_bf16(be.array(x), y16, rows, C, be.array(g) if with_gamma else None,
                              be.array(s) if with_scale else None, 1e-5)
    h = orc.rms_norm(x, g, 1e-5)
    if with_scale:
        h = orc.mul_rows(h, s)
    _bf16_within_one_ulp(y16.download(), h, f"rms_norm_modulate_bf16 [{rows},{C}]")


@pytest.mark.parametrize("n", [4224 * 10240, 1001])
def test_swiglu_bf16_vs_oracle(be, orc, n):
    """silu(g) * u -> bf16 against the oracle's swiglu (tensor.cpp:732-748),
    then nearest-even bf16 (zimage.cpp:130, the input of w2)."""
    g = orc.randn((n,), 790, 0.0, 1.5)
    u = orc.randn((n,), 791, 0.0, 1.5)
    y16 = _u16(be, n)
    be.swiglu_bf16(be.array(g), be.array(u), y16, n)
    _bf16_within_one_ulp(y16.download(), orc.swiglu(g, u), f"swiglu_bf16 n={n}")


@pytest.mark.parametrize("pairs,dim", [(2, 3840), (2, 37)])
def test_modulation_rows_vs_oracle(be, orc, pairs, dim):
    """Rows 2p: affine_(1, 1) (1 + scale); rows 2p + 1: tanh_ (gate), against
    the oracle (zimage.cpp:104-107; tensor.cpp:850-853, :884-887) at the
    elementwise bar."""
    from tolerances import assert_elementwise

    x = orc.randn((2 * pairs, dim), 9400 + dim, 0.0, 2.0)
    dx = be.array(x)
    be.modulation_rows(dx, pairs, dim)
    got = dx.download().reshape(2 * pairs, dim)
    want = np.empty_like(x)
    want[0::2] = orc.affine(x[0::2], 1.0, 1.0)
    want[1::2] = orc.tanh(x[1::2])
    assert_elementwise(got, want, f"modulation_rows [{2 * pairs},{dim}]")
