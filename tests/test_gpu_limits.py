"""GPU tests at the two ends of the size range, through the C ABI.

* Empty inputs: every op accepts zero rows or elements, launches nothing and
  leaves its buffers as they were. The reference's CPU loops simply run zero
  times (tensor.cpp:592-929; `parallel_chunks` over an empty range,
  tensor.cpp:149-265).
* Launches in pieces: one dispatch covers at most 2^32 - 1 work-items per
  grid dimension, so the launchers cover larger tensors in several launches;
  a child process with a small per-launch limit sends ordinary sizes through
  that path.
* Tensors past 2^31 (and 2^34) elements: the 64-bit index paths and the
  pieces at their real sizes. Inputs are filled on the device; the oracle
  checks slices that straddle element 2^31 and the end of the tensor, plus
  the size-independent property of each op (softmax rows sum to 1, RMSNorm
  rows have unit RMS at gamma = 1).
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

TWO31 = 1 << 31


def _view(be, base, off, n):
    """n float32 elements of device array `base` from element `off`."""
    return sdhip.DArray(be, (n,), ptr=base.ptr + 4 * off, owned=False)


# ---------------------------------------------------------------- empty inputs
def test_empty_inputs_launch_nothing(be):
    """Distinct buffers for every operand, so that no aliasing rule applies;
    each call must return 0 and leave all of them as they were."""
    init = [np.arange(64, dtype=np.float32) + 100 * i for i in range(4)]
    a, b, c, d = (be.array(v) for v in init)
    g = be.array(np.ones(64, np.float32))
    calls = [
        ("swiglu", lambda: be.swiglu(a, b, c, 0)),
        ("silu", lambda: be.silu(a, 0)),
        ("tanh", lambda: be.tanh(a, 0)),
        ("gelu", lambda: be.gelu(a, 0)),
        ("quick_gelu", lambda: be.quick_gelu(a, 0)),
        ("add", lambda: be.add(a, b, 0)),
        ("scale", lambda: be.scale(a, 2.0, 0)),
        ("affine", lambda: be.affine(a, 2.0, 1.0, 0)),
        ("geglu", lambda: be.geglu(a, b, 0, 8)),
        ("rms_norm", lambda: be.rms_norm(a, b, 0, 16, g, 1e-6)),
        ("layer_norm", lambda: be.layer_norm(a, b, 0, 16, g, g, 1e-6)),
        ("rms_norm_heads", lambda: be.rms_norm_heads(a, 0, 16, g, 1e-5)),
        ("add_rms_norm", lambda: be.add_rms_norm(a, b, c, 0, 16, g, 1e-6)),
        ("ln_modulate_gate", lambda: be.ln_modulate_gate(a, b, g, g, g, None, 0, 16, 1e-6)),
        ("group_norm N=0", lambda: be.group_norm(a, b, 0, 8, 4, 4, g, g, 1e-6, True)),
        ("group_norm HW=0", lambda: be.group_norm(a, b, 1, 8, 0, 4, g, g, 1e-6, True)),
        ("softmax_rows", lambda: be.softmax_rows(a, 0, 16, 0.5)),
        ("mul_rows", lambda: be.mul_rows(a, g, 0, 16)),
        ("add_rows_scaled", lambda: be.add_rows_scaled(a, b, g, 0, 16)),
        ("add_rows", lambda: be.add_rows(a, g, 0, 16)),
        ("add_channel_bias", lambda: be.add_channel_bias(a, g, 0, 4, 4)),
        ("rope", lambda: be.rope(a, 0, 4, 16, 8, c, d, True)),
        ("rope_qk", lambda: be.rope_qk(a, 16, b, 16, 1, 0, 8, c, d, True)),
        ("qknorm_rope", lambda: be.qknorm_rope(a, 16, b, 16, 1, 0, 8, g, g, 1e-5, c, d, True)),
        ("attention", lambda: be.attention(a, b, c, d, 0, 4, 4, 1, 1, 8)),
        ("gemm_nt_f32", lambda: be.gemm_nt_f32(0, 4, 8, a, 8, b, 8, c, 4)),
        ("upsample_nearest2x", lambda: be.upsample_nearest2x(a, b, 0, 2, 2)),
        ("concat_channels", lambda: be.concat_channels(a, b, c, 0, 2, 2, 4)),
        ("nchw_to_nlc", lambda: be.nchw_to_nlc(a, b, 1, 4, 0)),
        ("nlc_to_nchw", lambda: be.nlc_to_nchw(a, b, 0, 4, 4)),
    ]
    for name, call in calls:
        call()
        be.synchronize()
        for buf, v in zip((a, b, c, d), init):
            assert np.array_equal(buf.download(), v), f"{name} with an empty extent wrote to a buffer"
    assert np.array_equal(g.download(), np.ones(64, np.float32))


# ---------------------------------------------------------------- launches in pieces
def test_split_launches():
    """Every launcher that splits a tensor over several launches, at ordinary
    sizes: a child process with SDH_LAUNCH_ITEMS=4096 (tests/split_launch_check.py)."""
    script = os.path.join(os.path.dirname(os.path.abspath(__file__)), "split_launch_check.py")
    env = dict(os.environ, SDH_LAUNCH_ITEMS="4096")
    r = subprocess.run([sys.executable, script], capture_output=True, text=True, timeout=180, env=env)
    print(r.stdout)
    assert r.returncode == 0 and "split ok" in r.stdout, r.stdout + r.stderr


# ---------------------------------------------------------------- past 2^31 elements
def test_swiglu_past_2_31(be, orc):
    n = TWO31 + 12
    g, u, y = be.randn((n,), 1101, 0.0, 1.5), be.randn((n,), 1102, 0.0, 1.5), be.empty((n,))
    be.swiglu(g, u, y, n)
    for off in (0, TWO31 - 4096, n - 4096):
        m = min(8192, n - off)
        gs, us = _view(be, g, off, m).download(), _view(be, u, off, m).download()
        assert_elementwise(_view(be, y, off, m).download(), orc.swiglu(gs, us), f"swiglu n=2^31+12 at {off}")


def test_add_past_2_31(be, orc):
    n = TWO31 + 5  # odd: the vector body plus a scalar tail
    a, b = be.randn((n,), 1111), be.randn((n,), 1112)
    sl = [(off, min(8192, n - off)) for off in (TWO31 - 4096, n - 4096)]
    before = [(_view(be, a, o, m).download(), _view(be, b, o, m).download()) for o, m in sl]
    be.add(a, b, n)
    for (o, m), (av, bv) in zip(sl, before):
        assert_elementwise(_view(be, a, o, m).download(), orc.add(av, bv), f"add n=2^31+5 at {o}")


def test_rms_norm_past_2_31(be, orc):
    C = 3840
    rows = TWO31 // C + 3  # 559,243 rows: the last rows start past element 2^31
    x, y = be.randn((rows, C), 1121), be.empty((rows, C))
    gamma = be.array(np.ones(C, np.float32))
    be.rms_norm(x, y, rows, C, gamma, 1e-6)
    for r0 in (TWO31 // C - 2, rows - 3):
        xs = _view(be, x, r0 * C, 4 * C if r0 + 4 <= rows else 3 * C).download()
        xs = xs.reshape(-1, C)
        got = _view(be, y, r0 * C, xs.size).download().reshape(-1, C)
        assert_reduction(got, orc.rms_norm(xs, np.ones(C, np.float32), 1e-6), f"rms_norm rows from {r0}")
        assert np.allclose(np.sqrt(np.mean(got.astype(np.float64) ** 2, axis=1)), 1.0, atol=1e-5)


def test_mul_rows_past_2_34(be, orc):
    """More than 2^32 float4 vectors: the broadcast kernel's 64-bit column index."""
    dim = 3840
    rows = (1 << 34) // dim + 2  # 4,473,926 rows, 68.7 GB
    x = be.randn((rows, dim), 1131)
    v = orc.randn((dim,), 1132, 1.0, 0.2)
    dv = be.array(v)
    probe_rows = (0, (1 << 33) // dim, (1 << 34) // dim - 1, rows - 2)
    before = [_view(be, x, r * dim, 2 * dim).download().reshape(2, dim) for r in probe_rows]
    be.mul_rows(x, dv, rows, dim)
    for r, xb in zip(probe_rows, before):
        got = _view(be, x, r * dim, 2 * dim).download().reshape(2, dim)
        assert_elementwise(got, orc.mul_rows(xb, v), f"mul_rows rows {r}..{r + 1}")


def test_softmax_past_2_31(be, orc):
    cols = 4096
    rows = TWO31 // cols + 2  # 524,290 rows
    x = be.randn((rows, cols), 1141, 0.0, 3.0)
    scale = 1.0 / math.sqrt(128.0)
    probe = (TWO31 // cols - 1, rows - 2)
    before = [_view(be, x, r * cols, 2 * cols).download().reshape(2, cols) for r in probe]
    be.softmax_rows(x, rows, cols, scale, False)
    for r, xb in zip(probe, before):
        got = _view(be, x, r * cols, 2 * cols).download().reshape(2, cols)
        assert_softmax(got, orc.softmax_rows(xb, scale, False), f"softmax rows {r}..{r + 1}")
        assert float(np.max(np.abs(got.sum(axis=1, dtype=np.float64) - 1.0))) < 1e-5
