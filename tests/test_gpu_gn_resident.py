"""GPU tests of GroupNorm's resident schedule (k_gn_resident and the
pipelined k_gn_resident_pipe: one launch no larger than the GPU holds at
once; teams of workgroups hold a segment in registers, exchange per-share
(sum, M2) pairs through tagged 64-bit slots and read x once).

Against the float64 oracle (tensor.cpp:592-625, then silu :843-849) at the
reductions' relative 1e-4:
  * plans of several rounds whose shares each lie in one channel (few
    workgroups per team up to the 4b shape), bit-identical on repeat;
  * the team wait through the scalar path (uncached slots) and through
    vector loads (SDH_GN_SCALAR_POLL=0): the same bits;
  * the default choice between the resident and the split schedule;
  * the resident kernels forced (SDH_GN_RESIDENT=2) on every shape, every
    share size (V = 4, 8, 16 float4 per thread: SDH_GN_RESIDENT_V) and each
    kernel alone (SDH_GN_RESIDENT_PIPE), in child processes: segments in
    several rounds per team, shares that span channels or end short;
  * in place, repeated and interleaved with the other GroupNorm schedules,
    bit-identical on repeated calls (the merge order is fixed);
  * the split schedule still reachable with SDH_GN_RESIDENT=0 (and
    SDH_GN_PIPE=0), and with
    each chunk size forced (SDH_GN_CHUNK) and every shape forced onto it
    (SDH_GN_SPLIT=1);
  * two processes running it at the same time (besides this one);
  * the failure path, forced from the host: SDH_GN_SPIN_LIMIT=0 expires
    every wait at once, so every workgroup writes NaN and exits, and the
    next download reports SDH_ERR_HIP.
The shapes the pipelined schedule would take by default (x in whole
4096-float chunks that each lie in one channel) run it in the default-
schedule tests; the tests of the resident kernels themselves force them
(SDH_GN_RESIDENT=2) or switch the pipelined schedule off (SDH_GN_PIPE=0).
"""
import os
import subprocess
import sys

import numpy as np
import pytest

from tolerances import assert_reduction

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
PKG_DIR = os.path.join(ROOT, "stablediffusion-cpp_amd")
ORACLE_DIR = os.path.join(ROOT, "oracle")

SHAPES = [  # shape, groups, eps
    ((1, 512, 128, 128), 32, 1e-6),  # config 4a: pipelined by default; forced: V = 4, one round
    ((1, 256, 256, 256), 32, 1e-6),  # 64 MB: resident (pipelined) by default
    ((2, 640, 64, 64), 32, 1e-6),    # 21 MB: pipelined; forced: one resident round
    ((3, 512, 128, 128), 32, 1e-6),  # 96 segments: three rounds of 32 teams
    ((1, 96, 100, 100), 3, 1e-6),    # shares span channels, last share short
    ((2, 64, 129, 132), 8, 1e-5),    # plane of 17028 floats: shares cross channel ends
    ((1, 16, 300, 300), 2, 1e-6),    # 44 workgroups per segment
    ((16, 64, 100, 100), 8, 1e-6),   # 128 segments: pipelined rounds, shares cross channel ends
    ((1, 128, 512, 512), 32, 1e-6),  # pipelined, uniform shares
]


def _run(be, orc, shape, groups, eps, silu, seed, inplace=False):
    x = orc.randn(shape, seed, 0.5, 2.0)
    Cc = shape[1]
    g = orc.randn((Cc,), seed + 1, 1.0, 0.1)
    b = orc.randn((Cc,), seed + 2, 0.0, 0.1)
    dx = be.array(x)
    dy = dx if inplace else be.empty(shape)
    N = shape[0]
    be.group_norm(dx, dy, N, Cc, x.size // (N * Cc), groups, be.array(g), be.array(b), eps, silu=silu)
    return dy.download(), orc.group_norm(x, groups, g, b, eps, silu=silu)


@pytest.mark.parametrize("shape,groups,eps", SHAPES)
@pytest.mark.parametrize("silu", [True, False])
def test_default_schedule_matches_oracle(be, orc, shape, groups, eps, silu):
    got, want = _run(be, orc, shape, groups, eps, silu, 4100 + shape[1])
    assert_reduction(got, want, f"group_norm{'+silu' if silu else ''} {shape} g{groups}")


def test_resident_deterministic_and_in_place(be, orc):
    shape = (1, 256, 256, 256)
    a, want = _run(be, orc, shape, 32, 1e-6, True, 4200)
    b, _ = _run(be, orc, shape, 32, 1e-6, True, 4200)
    c, _ = _run(be, orc, shape, 32, 1e-6, True, 4200, inplace=True)
    assert np.array_equal(a, b) and np.array_equal(a, c)
    assert_reduction(a, want, "resident in place")


def test_resident_interleaved_with_other_schedules(be, orc):
    """Resident launches of different grids between single-workgroup and
    generic launches: each launch starts from the slots the previous one
    cleared."""
    cases = [((1, 256, 256, 256), 32), ((2, 320, 64, 64), 32), ((2, 640, 64, 64), 32), ((1, 96, 33, 17), 32),
             ((1, 128, 512, 512), 32), ((1, 512, 128, 128), 32), ((1, 16, 300, 300), 2)]
    for rep in range(2):
        for i, (shape, groups) in enumerate(cases):
            got, want = _run(be, orc, shape, groups, 1e-6, True, 4300 + i)
            assert_reduction(got, want, f"interleaved {shape} rep {rep}")


def _child_code(body):
    return (
        "import sys; sys.path[:0] = [%r, %r, %r]\n"
        "import numpy as np, sdhip\n"
        "from oracle import Oracle\n"
        "from tolerances import assert_reduction\n"
        "be, orc = sdhip.Backend(), Oracle()\n"
        "def run(shape, groups, eps, silu, seed):\n"
        "    x = orc.randn(shape, seed, 0.5, 2.0); C = shape[1]\n"
        "    g = orc.randn((C,), seed + 1, 1.0, 0.1); b = orc.randn((C,), seed + 2, 0.0, 0.1)\n"
        "    d, o = be.array(x), be.empty(shape); N = shape[0]\n"
        "    be.group_norm(d, o, N, C, x.size // (N * C), groups, be.array(g), be.array(b), eps, silu=silu)\n"
        "    return o, orc.group_norm(x, groups, g, b, eps, silu=silu)\n"
    ) % (PKG_DIR, ORACLE_DIR, HERE) + body


def _child(env, body):
    code = _child_code(body)
    r = subprocess.run([sys.executable, "-u", "-c", code], capture_output=True, text=True, timeout=240,
                       env=dict(os.environ, **env))
    print(r.stdout, r.stderr[-2000:])
    return r


def test_forced_resident_every_shape():
    """SDH_GN_RESIDENT=2: the resident kernels on every shape above, also
    those the default policy gives to the split schedule."""
    body = (
        "for shape, groups, eps in %r:\n"
        "    for silu in (True, False):\n"
        "        o, want = run(shape, groups, eps, silu, 4150)\n"
        "        assert_reduction(o.download(), want, f'forced {shape} {silu}')\n"
        "        print('ok', shape, silu, flush=True)\n"
        "print('forced ok')\n"
    ) % (SHAPES,)
    r = _child({"SDH_GN_RESIDENT": "2"}, body)
    assert r.returncode == 0 and "forced ok" in r.stdout


@pytest.mark.parametrize("V", [4, 8, 16])
def test_resident_each_share_size(V):
    """Every share size on uniform shapes, and V = 4 and 8 on shares that
    cross channels (V = 16 has no such instantiation: it would spill)."""
    shapes = [((1, 512, 128, 128), 32), ((1, 128, 512, 512), 32), ((2, 64, 256, 256), 16)]
    if V < 16:
        shapes += [((1, 96, 100, 100), 3), ((2, 64, 129, 132), 8)]
    body = (
        "for shape, groups in %r:\n"
        "    for silu in (True, False):\n"
        "        o, want = run(shape, groups, 1e-6, silu, 4400)\n"
        "        assert_reduction(o.download(), want, f'V=%d {shape} {silu}')\n"
        "        print('ok', shape, silu, flush=True)\n"
        "print('shares ok')\n"
    ) % (shapes, V)
    r = _child({"SDH_GN_RESIDENT": "2", "SDH_GN_RESIDENT_V": str(V)}, body)
    assert r.returncode == 0 and "shares ok" in r.stdout


@pytest.mark.parametrize("pipe", [0, 1])
def test_resident_plain_or_pipelined_forced(pipe):
    """SDH_GN_RESIDENT_PIPE=0 (rounds of k_gn_resident only) and =1
    (k_gn_resident_pipe even for one-round tensors, and V = 4 and 8) on
    uniform and channel-crossing shares."""
    shapes = [((1, 128, 512, 512), 32), ((16, 64, 100, 100), 8), ((1, 512, 128, 128), 32), ((3, 96, 100, 100), 3)]
    body = (
        "for shape, groups in %r:\n"
        "    for silu in (True, False):\n"
        "        o, want = run(shape, groups, 1e-6, silu, 4800)\n"
        "        assert_reduction(o.download(), want, f'pipe=%d {shape} {silu}')\n"
        "print('pipe ok')\n"
    ) % (shapes, pipe)
    r = _child({"SDH_GN_RESIDENT": "2", "SDH_GN_RESIDENT_PIPE": str(pipe)}, body)
    assert r.returncode == 0 and "pipe ok" in r.stdout
    if pipe:
        r = _child({"SDH_GN_RESIDENT": "2", "SDH_GN_RESIDENT_PIPE": "1", "SDH_GN_RESIDENT_V": "4"}, body)
        assert r.returncode == 0 and "pipe ok" in r.stdout


# Multi-round resident plans whose shares each lie in one channel, with few
# workgroups per team: the case in which stores that raced the prefetch
# showed as wrong lanes (lanes 12-15 of rows of 16) in the first round.
UNIFORM_ROUNDS = [((4, 64, 256, 256), 32), ((2, 128, 256, 256), 32), ((1, 256, 256, 256), 32),
                  ((1, 128, 1024, 1024), 32)]


@pytest.mark.parametrize("shape,groups", UNIFORM_ROUNDS)
def test_uniform_shares_over_several_rounds(be, orc, shape, groups):
    """Against the oracle, and bit-identical on a second call."""
    a, want = _run(be, orc, shape, groups, 1e-6, True, 4700 + shape[0])
    assert_reduction(a, want, f"uniform rounds {shape}")
    b, _ = _run(be, orc, shape, groups, 1e-6, True, 4700 + shape[0])
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_scalar_and_vector_polls_give_the_same_bits():
    """The team wait read through the scalar path (uncached slots, plans of
    several rounds, the default) and through agent-scope vector loads
    (SDH_GN_SCALAR_POLL=0) merge the same pairs in the same order: the
    outputs are bit-identical, and both match the oracle."""
    body = (
        "import hashlib\n"
        "for shape, groups in %r + [((16, 64, 100, 100), 8), ((4, 96, 300, 300), 3)]:\n"
        "    o, want = run(shape, groups, 1e-6, True, 4750)\n"
        "    got = o.download()\n"
        "    assert_reduction(got, want, f'poll {shape}')\n"
        "    print('digest', shape, hashlib.sha1(got.tobytes()).hexdigest(), flush=True)\n"
        "print('polls ok')\n"
    ) % (UNIFORM_ROUNDS,)
    outs = []
    for sp in ("1", "0"):
        r = _child({"SDH_GN_SCALAR_POLL": sp}, body)
        assert r.returncode == 0 and "polls ok" in r.stdout
        outs.append([l for l in r.stdout.splitlines() if l.startswith("digest")])
    assert outs[0] == outs[1] and len(outs[0]) == len(UNIFORM_ROUNDS) + 2


def test_split_schedule_still_reachable():
    """SDH_GN_RESIDENT=0 and SDH_GN_PIPE=0: the split schedule on the shapes
    the resident and the pipelined ones would take."""
    body = (
        "for shape, groups in (((1, 256, 256, 256), 32), ((2, 640, 64, 64), 32), ((1, 16, 300, 300), 2)):\n"
        "    o, want = run(shape, groups, 1e-6, True, 4500)\n"
        "    assert_reduction(o.download(), want, f'split {shape}')\n"
        "print('split ok')\n"
    )
    r = _child({"SDH_GN_RESIDENT": "0", "SDH_GN_PIPE": "0"}, body)
    assert r.returncode == 0 and "split ok" in r.stdout


def test_expired_wait_is_reported():
    """SDH_GN_SPIN_LIMIT=0: every team wait expires before its first poll,
    every workgroup still finishes (NaN output), the download fails with
    SDH_ERR_HIP naming the op, the word is then clear, and the library keeps
    working (a non-resident GroupNorm and an add afterwards are correct).
    After the expiry the process no longer takes the resident schedule: the
    same shape, whose waits would all expire again, now comes out right."""
    body = (
        "o, want = run((1, 256, 256, 256), 32, 1e-6, True, 4600)\n"
        "try:\n"
        "    o.download(); print('no error'); sys.exit(1)\n"
        "except sdhip.SdhError as e:\n"
        "    assert e.status == sdhip.SDH_ERR_HIP and 'sdh_group_norm_silu' in str(e) and 'bounded wait' in str(e), e\n"
        "be.synchronize()\n"
        "assert np.isnan(o.download()).all()\n"
        "o2, want2 = run((2, 320, 32, 32), 32, 1e-5, True, 4601)\n"
        "assert_reduction(o2.download(), want2, 'single after expiry')\n"
        "o3, want3 = run((1, 256, 256, 256), 32, 1e-6, True, 4602)\n"
        "assert_reduction(o3.download(), want3, 'resident shape after expiry')\n"
        "a = be.array(np.ones(1000, np.float32)); be.add(a, be.array(np.ones(1000, np.float32)), 1000)\n"
        "assert (a.download() == 2.0).all()\n"
        "print('expiry ok')\n"
    )
    r = _child({"SDH_GN_SPIN_LIMIT": "0", "SDH_GN_PIPE": "0"}, body)
    assert r.returncode == 0 and "expiry ok" in r.stdout


def test_expired_waits_in_two_scratch_areas_both_reported():
    """SDH_GN_SPIN_LIMIT=0, a library GroupNorm (team slots and flag word in
    the library's counters) and then an allocation-free one (its own fixed
    scratch), both resident and both expiring, before one synchronisation:
    the failure reported is the first call's (the second arming must not
    hide it), both outputs are NaN, both flag words are cleared (the next
    synchronisation is clean) and the library keeps working afterwards."""
    body = (
        "shape = (1, 256, 256, 256); C = 256; HW = 256 * 256\n"
        "x = orc.randn(shape, 4610, 0.5, 2.0)\n"
        "g = be.array(orc.randn((C,), 4611, 1.0, 0.1)); b = be.array(orc.randn((C,), 4612, 0.0, 0.1))\n"
        "d, o1, o2 = be.array(x), be.empty(shape), be.empty(shape)\n"
        "be.call('sdh_group_norm_silu', d.ptr, o1.ptr, 1, C, HW, 32, g.ptr, b.ptr, 1e-6)\n"
        "be.call('sdh_group_norm_silu_noalloc', d.ptr, o2.ptr, 1, C, HW, 32, g.ptr, b.ptr, 1e-6)\n"
        "try:\n"
        "    be.synchronize(); print('no error'); sys.exit(1)\n"
        "except sdhip.SdhError as e:\n"
        "    assert e.status == sdhip.SDH_ERR_HIP and 'sdh_group_norm_silu: a bounded wait' in str(e), e\n"
        "be.synchronize()\n"
        "assert np.isnan(o1.download()).all() and np.isnan(o2.download()).all()\n"
        "o3, want3 = run(shape, 32, 1e-6, True, 4613)\n"
        "assert_reduction(o3.download(), want3, 'library call after expiry')\n"
        "x4 = orc.randn(shape, 4614, 0.5, 2.0); d4, o4 = be.array(x4), be.empty(shape)\n"
        "be.call('sdh_group_norm_silu_noalloc', d4.ptr, o4.ptr, 1, C, HW, 32, g.ptr, b.ptr, 1e-6)\n"
        "o5 = be.empty(shape)\n"
        "be.call('sdh_group_norm_silu', d4.ptr, o5.ptr, 1, C, HW, 32, g.ptr, b.ptr, 1e-6)\n"
        "assert np.array_equal(o4.download(), o5.download())\n"
        "be.synchronize()\n"
        "print('two areas ok')\n"
    )
    r = _child({"SDH_GN_SPIN_LIMIT": "0", "SDH_GN_PIPE": "0"}, body)
    assert r.returncode == 0 and "two areas ok" in r.stdout


def test_two_processes_at_once():
    """Two child processes run resident GroupNorms at the same time as each
    other, while this process holds its own device context: every result
    within the bound."""
    body = (
        "for rep in range(5):\n"
        "    for shape, groups in (((1, 256, 256, 256), 32), ((2, 640, 64, 64), 32)):\n"
        "        o, want = run(shape, groups, 1e-6, True, 4700 + rep)\n"
        "        assert_reduction(o.download(), want, f'{shape} rep {rep}')\n"
        "print('concurrent ok')\n"
    )
    code = _child_code(body)
    procs = [subprocess.Popen([sys.executable, "-u", "-c", code], stdout=subprocess.PIPE, stderr=subprocess.PIPE,
                              text=True) for _ in range(2)]
    outs = []
    for p in procs:
        try:
            out, err = p.communicate(timeout=240)
        except subprocess.TimeoutExpired:
            p.kill()
            out, err = p.communicate()
        outs.append((p.returncode, out, err[-2000:]))
    print(outs)
    assert all(rc == 0 and "concurrent ok" in out for rc, out, _ in outs)


# Segments of 24577-65536 floats (SD 1.5 UNet shapes): the split schedule
# by default, with chunks of 2048 or 4096 floats so that a pass has enough
# workgroups; one resident round only when forced (SDH_GN_RESIDENT=2,
# shares of 16384 floats, the last short). [2,640,32,32] (20480 floats)
# stays on the single-workgroup kernel.
SMALL_SEG_SHAPES = [((2, 320, 64, 64), 32, 1e-5), ((2, 1280, 32, 32), 32, 1e-5), ((2, 960, 32, 32), 32, 1e-5),
                    ((1, 64, 128, 128), 32, 1e-6), ((2, 512, 64, 64), 32, 1e-5), ((2, 96, 30, 36), 3, 1e-6),
                    ((2, 640, 32, 32), 32, 1e-5)]


@pytest.mark.parametrize("shape,groups,eps", SMALL_SEG_SHAPES)
@pytest.mark.parametrize("silu", [True, False])
def test_small_segments_default_schedule(be, orc, shape, groups, eps, silu):
    got, want = _run(be, orc, shape, groups, eps, silu, 5200 + shape[1])
    assert_reduction(got, want, f"small-segment group_norm {shape} g{groups} silu={silu}")


def test_small_segments_resident_round_forced():
    """SDH_GN_RESIDENT=2: one resident round on the same shapes (those of
    more than 24576 floats per segment)."""
    body = (
        "for shape, groups, eps in %r:\n"
        "    for silu in (True, False):\n"
        "        o, want = run(shape, groups, eps, silu, 5300)\n"
        "        assert_reduction(o.download(), want, f'one round {shape} {silu}')\n"
        "print('one round ok')\n"
    ) % (SMALL_SEG_SHAPES,)
    r = _child({"SDH_GN_RESIDENT": "2"}, body)
    assert r.returncode == 0 and "one round ok" in r.stdout


@pytest.mark.parametrize("chunk", [2048, 4096, 8192])
def test_split_each_chunk_size(chunk):
    """SDH_GN_SPLIT=1 with SDH_GN_CHUNK forced: every shape on the split
    schedule at each chunk size: chunks inside one channel or crossing
    channel ends, a short last chunk, merges inside pass B (at most 64
    chunks per segment) or in the finalize launch (more)."""
    shapes = SMALL_SEG_SHAPES + [((1, 512, 128, 128), 32, 1e-6), ((1, 96, 100, 100), 3, 1e-6),
                                 ((1, 16, 300, 300), 2, 1e-6), ((2, 1280, 8, 8), 32, 1e-5)]
    body = (
        "for shape, groups, eps in %r:\n"
        "    for silu in (True, False):\n"
        "        o, want = run(shape, groups, eps, silu, 5400)\n"
        "        assert_reduction(o.download(), want, f'split %d {shape} {silu}')\n"
        "print('split ok')\n"
    ) % (shapes, chunk)
    r = _child({"SDH_GN_SPLIT": "1", "SDH_GN_CHUNK": str(chunk)}, body)
    assert r.returncode == 0 and "split ok" in r.stdout
