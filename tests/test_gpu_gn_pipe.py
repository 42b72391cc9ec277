"""GPU tests of GroupNorm's pipelined schedule (k_gn_pipe: one launch in
which stats workgroups publish each 4096-float chunk's (sum, M2) as tagged
64-bit words and apply workgroups, later in dispatch order, merge their
segment's pairs and write y; segments of at most 64 whole chunks that each
lie in one channel, any tensor size, in launches of at most 2^17 chunks).

Against the float64 oracle (tensor.cpp:592-625, then silu :843-849) at the
reductions' relative 1e-4:
  * every shape class the schedule takes: the FLUX VAE's config 4a, SD 1.5's
    config 4c, one and several segments per unit, 3-64 chunks per segment,
    tensors of 128 MB, with and without SiLU, groups other than 32;
  * a tensor of more than 2^17 chunks (two launches): each sample the same
    bits as a call on that sample alone;
  * bit-identical on repeat, in place and interleaved with the other
    schedules (a launch's tags never match pairs an earlier launch left);
  * the apply workgroups' own computation of a missing pair, forced from the
    host (SDH_GN_SPIN_LIMIT=0: no polls, every pair not yet out at the first
    look is computed from x by the apply workgroup; SDH_GN_PIPE_LAG=1: apply
    units dispatched one unit after their stats units, so the first ones
    look before their pairs are out): the same bits as the published pairs
    give;
  * in place with those two: a missing pair cannot be computed
    (its chunk may be overwritten), so the wait fails: NaN, SDH_ERR_HIP at
    the next synchronisation, and from then on the process takes the other
    schedules, which give the right result;
  * SDH_GN_PIPE=0: the split schedule on the same shapes;
  * a captured graph of more than 64 pipelined calls (two advances of the
    device counter per replay), replayed with new inputs between replays.
"""
import hashlib
import os
import subprocess
import sys

import numpy as np
import pytest
import sdhip

from tolerances import assert_reduction

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
PKG_DIR = os.path.join(ROOT, "stablediffusion-cpp_amd")
ORACLE_DIR = os.path.join(ROOT, "oracle")

SHAPES = [  # shape, groups, eps: all take the pipelined schedule
    ((1, 512, 128, 128), 32, 1e-6),  # config 4a: 64 chunks a segment, 4 segments a unit
    ((2, 320, 64, 64), 32, 1e-5),    # config 4c: 10 chunks a segment
    ((1, 512, 64, 64), 32, 1e-6),    # 16 chunks a segment
    ((1, 128, 256, 256), 32, 1e-6),  # 4 channels of 16 chunks each
    ((2, 640, 64, 64), 32, 1e-6),    # 20 chunks a segment, 64 segments
    ((3, 96, 64, 64), 32, 1e-5),     # 3 chunks a segment, 96 segments
    ((1, 64, 128, 128), 8, 1e-6),    # 8 groups: 32 chunks a segment, 8 segments
    ((1, 32, 512, 512), 32, 1e-6),   # one channel of 64 chunks a segment (32 MB)
    ((4, 512, 128, 128), 32, 1e-6),  # 4 x config 4a: 128 segments (128 MB)
    ((2, 64, 256, 256), 16, 1e-6),   # 16 groups: 64 chunks a segment, 32 segments
    ((1, 96, 256, 256), 32, 1e-5),   # 48 chunks a segment, 24 MB
]


def _inputs(be, orc, shape, seed):
    x = orc.randn(shape, seed, 0.5, 2.0)
    C = shape[1]
    g = orc.randn((C,), seed + 1, 1.0, 0.1)
    b = orc.randn((C,), seed + 2, 0.0, 0.1)
    return x, g, b


def _gn(be, dx, dy, shape, groups, dg, db, eps, silu=True):
    N, C = shape[0], shape[1]
    be.group_norm(dx, dy, N, C, int(np.prod(shape)) // (N * C), groups, dg, db, eps, silu=silu)


@pytest.mark.parametrize("shape,groups,eps", SHAPES)
@pytest.mark.parametrize("silu", [True, False])
def test_pipe_matches_oracle(be, orc, shape, groups, eps, silu):
    x, g, b = _inputs(be, orc, shape, 5100 + shape[1])
    dy = be.empty(shape)
    _gn(be, be.array(x), dy, shape, groups, be.array(g), be.array(b), eps, silu)
    assert_reduction(dy.download(), orc.group_norm(x, groups, g, b, eps, silu=silu),
                     f"pipe {shape} g{groups} silu={silu}")


def test_pipe_repeat_in_place_and_interleaved(be, orc):
    """The same bits on repeat, in place, and after launches of the other
    schedules and of other pipelined shapes in between."""
    shape, groups, eps = SHAPES[0]
    x, g, b = _inputs(be, orc, shape, 5200)
    dx, dg, db = be.array(x), be.array(g), be.array(b)
    first = be.empty(shape)
    _gn(be, dx, first, shape, groups, dg, db, eps)
    want = first.download()
    assert_reduction(want, orc.group_norm(x, groups, g, b, eps, silu=True), "pipe 4a")
    others = [((1, 96, 500, 500), 32), ((2, 1280, 8, 8), 32), ((2, 320, 64, 64), 32), ((2, 1280, 32, 32), 32)]
    for rep in range(3):
        for i, (oshape, og) in enumerate(others):  # resident, single, pipelined, split
            ox, ogm, ob = _inputs(be, orc, oshape, 5210 + i)
            od = be.empty(oshape)
            _gn(be, be.array(ox), od, oshape, og, be.array(ogm), be.array(ob), 1e-6)
        again = be.empty(shape)
        _gn(be, dx, again, shape, groups, dg, db, eps)
        assert np.array_equal(again.download(), want), f"repeat {rep}"
    inplace = be.array(x)
    _gn(be, inplace, inplace, shape, groups, dg, db, eps)
    assert np.array_equal(inplace.download(), want), "in place"


def test_pipe_over_several_launches(be):
    """[66,512,128,128]: 2112 segments of 64 chunks, more than the 2^17
    chunks one launch takes, so two launches (2048 segments, then 64, whose
    channels continue from group 0). Samples 0, 63, 64 and 65 (both sides of
    the cut, and the last) must give the same bits as calls on those samples
    alone, which take one launch each. Then the whole call captured in a
    graph (two captured launches, each with its own place among the
    capture's calls), replayed twice over new x: the direct call's bits;
    and the call in place over the last x: the same bits again."""
    shape, groups, eps = (66, 512, 128, 128), 32, 1e-6
    C, HW = shape[1], shape[2] * shape[3]
    per = C * HW * 4  # bytes a sample
    dx = be.randn(shape, 5300, 0.5, 2.0)
    dg, db = be.randn((C,), 5301, 1.0, 0.1), be.randn((C,), 5302, 0.0, 0.1)
    dy = be.empty(shape)
    be.group_norm(dx, dy, shape[0], C, HW, groups, dg, db, eps, silu=True)
    be.synchronize()
    for n0, k in ((0, 1), (63, 2), (65, 1)):
        sub = (k, C, shape[2], shape[3])
        xs = sdhip.DArray(be, sub, ptr=dx.ptr + n0 * per, owned=False)
        ys = sdhip.DArray(be, sub, ptr=dy.ptr + n0 * per, owned=False)
        alone = be.empty(sub)
        be.group_norm(xs, alone, k, C, HW, groups, dg, db, eps, silu=True)
        got, want = ys.download(), alone.download()
        assert np.isfinite(want).all(), f"samples {n0}..{n0 + k - 1}"
        assert np.array_equal(got, want), f"samples {n0}..{n0 + k - 1} differ from a call on them alone"
        alone.free()
    dg2 = be.empty(shape)
    be.capture_begin()
    be.group_norm(dx, dg2, shape[0], C, HW, groups, dg, db, eps, silu=True)
    graph = be.capture_end()
    try:
        for rep in range(2):
            be.check(be.lib.sdh_fill_normal(dx.ptr, dx.size, 5310 + rep, 0.25 * rep, 2.0))
            be.group_norm(dx, dy, shape[0], C, HW, groups, dg, db, eps, silu=True)
            be.graph_launch(graph)
            be.synchronize()
            for n0 in (0, 63, 64, 65):
                sub = (1, C, shape[2], shape[3])
                want = sdhip.DArray(be, sub, ptr=dy.ptr + n0 * per, owned=False).download()
                got = sdhip.DArray(be, sub, ptr=dg2.ptr + n0 * per, owned=False).download()
                assert np.isfinite(want).all() and np.array_equal(got, want), f"replay {rep} sample {n0}"
    finally:
        be.graph_destroy(graph)
    # in place over the last x (two launches whose apply workgroups may only wait): dy's bits
    be.group_norm(dx, dx, shape[0], C, HW, groups, dg, db, eps, silu=True)
    be.synchronize()
    for n0 in (0, 63, 64, 65):
        sub = (1, C, shape[2], shape[3])
        want = sdhip.DArray(be, sub, ptr=dy.ptr + n0 * per, owned=False).download()
        got = sdhip.DArray(be, sub, ptr=dx.ptr + n0 * per, owned=False).download()
        assert np.array_equal(got, want), f"in place, sample {n0}"
    dx.free()
    dy.free()
    dg2.free()


def _child_code(body):
    return (
        "import sys, hashlib; sys.path[:0] = [%r, %r, %r]\n"
        "import numpy as np, sdhip\n"
        "from oracle import Oracle\n"
        "from tolerances import assert_reduction\n"
        "be, orc = sdhip.Backend(), Oracle()\n"
        "def run(shape, groups, eps, seed, inplace=False):\n"
        "    x = orc.randn(shape, seed, 0.5, 2.0); C = shape[1]\n"
        "    g = orc.randn((C,), seed + 1, 1.0, 0.1); b = orc.randn((C,), seed + 2, 0.0, 0.1)\n"
        "    d = be.array(x); o = d if inplace else be.empty(shape); N = shape[0]\n"
        "    be.group_norm(d, o, N, C, x.size // (N * C), groups, be.array(g), be.array(b), eps, silu=True)\n"
        "    return o, orc.group_norm(x, groups, g, b, eps, silu=True)\n"
    ) % (PKG_DIR, ORACLE_DIR, HERE) + body


def _child(env, body):
    r = subprocess.run([sys.executable, "-u", "-c", _child_code(body)], capture_output=True, text=True, timeout=240,
                       env=dict(os.environ, **env))
    print(r.stdout, r.stderr[-2000:])
    return r


def _digest(a):
    return hashlib.sha256(np.ascontiguousarray(a).view(np.uint8)).hexdigest()


def test_missing_pairs_computed_by_apply_workgroups(be, orc):
    """SDH_GN_SPIN_LIMIT=0 and SDH_GN_PIPE_LAG=1: apply workgroups do not
    poll, and the first ones look before their pairs are out; every pair
    missing at their first look is computed from x by them. Same bits as
    this process's default run, on every shape."""
    want = {}
    for i, (shape, groups, eps) in enumerate(SHAPES):
        x, g, b = _inputs(be, orc, shape, 5300 + i)
        d, o = be.array(x), be.empty(shape)
        _gn(be, d, o, shape, groups, be.array(g), be.array(b), eps)
        want[i] = _digest(o.download())
    body = (
        "shapes = %r\n"
        "for i, (shape, groups, eps) in enumerate(shapes):\n"
        "    x = orc.randn(shape, 5300 + i, 0.5, 2.0); C = shape[1]\n"
        "    g = orc.randn((C,), 5301 + i, 1.0, 0.1); b = orc.randn((C,), 5302 + i, 0.0, 0.1)\n"
        "    d, o = be.array(x), be.empty(shape); N = shape[0]\n"
        "    be.group_norm(d, o, N, C, x.size // (N * C), groups, be.array(g), be.array(b), eps, silu=True)\n"
        "    got = o.download()\n"
        "    assert_reduction(got, orc.group_norm(x, groups, g, b, eps, silu=True), f'self {shape}')\n"
        "    print('digest', i, hashlib.sha256(np.ascontiguousarray(got).view(np.uint8)).hexdigest())\n"
        "be.synchronize()\n"
        "print('self-computed ok')\n"
    ) % ([(s, gr, e) for s, gr, e in SHAPES],)
    r = _child({"SDH_GN_SPIN_LIMIT": "0", "SDH_GN_PIPE_LAG": "1"}, body)
    assert r.returncode == 0 and "self-computed ok" in r.stdout
    got = dict((int(ln.split()[1]), ln.split()[2]) for ln in r.stdout.splitlines() if ln.startswith("digest"))
    assert got == want


def test_in_place_expired_wait_is_reported():
    """SDH_GN_SPIN_LIMIT=0 and SDH_GN_PIPE_LAG=1 in place: the first missing
    pair fails the wait;
    the output is NaN where it failed, the download reports SDH_ERR_HIP
    naming the op, the word is then clear, and the next in-place call (now
    on the split schedule) is right."""
    body = (
        "o, want = run((1, 512, 128, 128), 32, 1e-6, 5400, inplace=True)\n"
        "try:\n"
        "    o.download(); print('no error'); sys.exit(1)\n"
        "except sdhip.SdhError as e:\n"
        "    assert e.status == sdhip.SDH_ERR_HIP and 'sdh_group_norm_silu' in str(e) and 'bounded wait' in str(e), e\n"
        "be.synchronize()\n"
        "assert np.isnan(o.download()).any()\n"
        "o2, want2 = run((1, 512, 128, 128), 32, 1e-6, 5401, inplace=True)\n"
        "assert_reduction(o2.download(), want2, 'in place after expiry')\n"
        "o3, want3 = run((2, 320, 64, 64), 32, 1e-5, 5402)\n"
        "assert_reduction(o3.download(), want3, '4c after expiry')\n"
        "print('expiry ok')\n"
    )
    r = _child({"SDH_GN_SPIN_LIMIT": "0", "SDH_GN_PIPE_LAG": "1"}, body)
    assert r.returncode == 0 and "expiry ok" in r.stdout


def test_pipe_off_takes_the_split_schedule():
    """SDH_GN_PIPE=0: the same shapes on the split schedule."""
    body = (
        "for i, (shape, groups) in enumerate((((1, 512, 128, 128), 32), ((2, 320, 64, 64), 32), ((2, 640, 64, 64), 32))):\n"
        "    o, want = run(shape, groups, 1e-6, 5500 + i)\n"
        "    assert_reduction(o.download(), want, f'split {shape}')\n"
        "print('split ok')\n"
    )
    r = _child({"SDH_GN_PIPE": "0"}, body)
    assert r.returncode == 0 and "split ok" in r.stdout


def test_graph_of_more_than_64_calls(be, orc):
    """70 pipelined calls captured in one graph (the device counter advances
    before the 1st and the 65th of each replay), replayed three times with
    new inputs uploaded between replays: each replay gives the direct
    calls' bits for its inputs."""
    shape, groups, eps = (1, 512, 64, 64), 32, 1e-6
    N, C = shape[0], shape[1]
    HW = int(np.prod(shape)) // (N * C)
    dx = be.empty(shape)
    dg, db = be.array(orc.randn((C,), 5601, 1.0, 0.1)), be.array(orc.randn((C,), 5602, 0.0, 0.1))
    outs = [be.empty(shape) for _ in range(70)]
    be.capture_begin()
    for o in outs:
        be.group_norm(dx, o, N, C, HW, groups, dg, db, eps, silu=True)
    graph = be.capture_end()
    try:
        for rep in range(3):
            x = orc.randn(shape, 5610 + rep, 0.5 * rep, 2.0)
            dx.upload(x)
            direct = be.empty(shape)
            be.group_norm(dx, direct, N, C, HW, groups, dg, db, eps, silu=True)
            want = direct.download()
            be.graph_launch(graph)
            for k in (0, 1, 63, 64, 65, 69):
                assert np.array_equal(outs[k].download(), want), f"replay {rep} call {k}"
    finally:
        be.graph_destroy(graph)
