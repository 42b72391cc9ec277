"""GPU tests of graph capture on the library stream (sdh_capture_begin /
sdh_capture_end / sdh_graph_launch / sdh_graph_destroy).

The captured graph must give exactly what the same calls give when run
directly: every replay is compared bit for bit with the direct result, with
the program's own direct work and synchronisations between the replays
(a replay must not depend on state left by the previous one: the resident
GroupNorm's team slots and tickets are cleared by each launch itself). The
direct GroupNorm result is also held to the float64 oracle (tensor.cpp:
592-625 then :843-849) at the reductions' relative 1e-4. While capturing,
calls that would wait on the stream are refused with SDH_ERR_INVALID and the
capture still closes.
"""
import numpy as np
import pytest

import sdhip
from tolerances import assert_reduction

pytestmark = pytest.mark.gpu

GN_SHAPES = [  # the launch-bound GroupNorm configs, 4a and one split-schedule shape
    ((2, 1280, 8, 8), 1e-5),     # 4d: one workgroup per segment
    ((2, 320, 64, 64), 1e-5),    # 4c: pipelined (tags from the device counter a captured call advances)
    ((1, 512, 128, 128), 1e-6),  # 4a: pipelined
    ((2, 1280, 32, 32), 1e-5),   # split schedule, two launches
]


def _gn_inputs(be, orc, shape, seed):
    x = orc.randn(shape, seed, 0.0, 2.0)
    g = orc.randn((shape[1],), seed + 1, 1.0, 0.1)
    b = orc.randn((shape[1],), seed + 2, 0.0, 0.1)
    return x, g, b, be.array(x), be.array(g), be.array(b)


@pytest.mark.parametrize("shape,eps", GN_SHAPES)
def test_group_norm_silu_graph_replays_equal_direct(be, orc, shape, eps):
    N, Cc = shape[0], shape[1]
    HW = shape[2] * shape[3]
    x, g, b, dx, dg, db = _gn_inputs(be, orc, shape, 300 + N)
    direct = be.empty(shape)
    be.group_norm(dx, direct, N, Cc, HW, 32, dg, db, eps, silu=True)
    want = direct.download()
    assert_reduction(want, orc.group_norm(x, 32, g, b, eps, silu=True))

    out = be.empty(shape)
    be.capture_begin()
    for _ in range(3):  # three launches of the op in one graph
        be.group_norm(dx, out, N, Cc, HW, 32, dg, db, eps, silu=True)
    graph = be.capture_end()
    try:
        other = be.empty(shape)
        for rep in range(4):
            out.upload(np.full(shape, np.nan, np.float32))
            be.graph_launch(graph)
            got = out.download()
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"replay {rep}"
            # direct work of the program between replays
            be.group_norm(dx, other, N, Cc, HW, 32, dg, db, eps, silu=True)
            assert np.array_equal(other.download().view(np.uint32), want.view(np.uint32))
    finally:
        be.graph_destroy(graph)


def test_in_place_ops_replay_in_order(be, orc):
    """x += r; y = rms_norm(x) * w, captured twice in one graph: each replay
    advances x by 2r, as four direct calls would."""
    rows, C = 64, 3840
    x = orc.randn((rows, C), 41)
    r = orc.randn((rows, C), 42)
    w = orc.randn((C,), 43, 1.0, 0.1)
    da, dr, dw, dya = be.array(x), be.array(r), be.array(w), be.empty((rows, C))
    db_, dyb = be.array(x), be.empty((rows, C))
    be.capture_begin()
    be.add_rms_norm(db_, dr, dyb, rows, C, dw, 1e-6)
    be.add_rms_norm(db_, dr, dyb, rows, C, dw, 1e-6)
    graph = be.capture_end()
    try:
        for rep in range(3):
            be.graph_launch(graph)
            be.add_rms_norm(da, dr, dya, rows, C, dw, 1e-6)
            be.add_rms_norm(da, dr, dya, rows, C, dw, 1e-6)
            sa, sb = da.download(), db_.download()
            assert np.array_equal(sa.view(np.uint32), sb.view(np.uint32)), f"replay {rep}"
            assert np.array_equal(dya.download().view(np.uint32), dyb.download().view(np.uint32))
    finally:
        be.graph_destroy(graph)


def test_patchify_graph_replay(be, orc):
    C, H, W, p = 16, 128, 128, 2
    x = orc.randn((C, H, W), 51)
    dx = be.array(x)
    direct, out = be.empty((H // p * (W // p), p * p * C)), be.empty((H // p * (W // p), p * p * C))
    be.patchify(dx, direct, C, H, W, p)
    want = direct.download()
    be.capture_begin()
    be.patchify(dx, out, C, H, W, p)
    graph = be.capture_end()
    try:
        for rep in range(3):
            out.upload(np.zeros(want.shape, np.float32))
            be.graph_launch(graph)
            assert np.array_equal(out.download(), want), f"replay {rep}"
    finally:
        be.graph_destroy(graph)


def test_waits_are_refused_while_capturing(be, orc):
    x = be.array(orc.randn((256,), 61))
    host = np.empty(256, np.float32)
    be.capture_begin()
    try:
        be.scale(x, 2.0, 256)
        with pytest.raises(sdhip.SdhError) as e:
            be.download(host, x.ptr)
        assert e.value.status == sdhip.SDH_ERR_INVALID and "captured" in str(e.value)
        with pytest.raises(sdhip.SdhError) as e:
            be.synchronize()
        assert e.value.status == sdhip.SDH_ERR_INVALID
        with pytest.raises(sdhip.SdhError) as e:
            be.capture_begin()  # one capture at a time
        assert e.value.status == sdhip.SDH_ERR_INVALID
    finally:
        graph = be.capture_end()
    be.graph_destroy(graph)
    with pytest.raises(sdhip.SdhError) as e:
        be.capture_end()  # none open
    assert e.value.status == sdhip.SDH_ERR_INVALID
    be.synchronize()  # the stream is usable again
