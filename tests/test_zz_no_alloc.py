"""GPU tests of sdh_group_norm_silu_noalloc, the allocation-free variant of
sdh_group_norm_silu (no reference counterpart: for callers that cannot
allocate device memory). Through the C ABI (ctypes):

  * bit-identical to sdh_group_norm_silu on the same inputs, for every
    GroupNorm schedule (resident pipelined, the one-launch pipelined
    schedule, split with chunk statistics, single workgroup), called back
    to back with
    shrinking inputs, so each call starts from the fixed scratch the
    previous one left; also in place;
  * the arena's reserved and in-use bytes do not move across those calls;
  * a tensor whose split statistics exceed the fixed scratch is rejected
    with SDH_ERR_INVALID before anything is launched, and a call before
    sdh_init is rejected too, in child processes.
"""
import gc
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

# largest first: each call of the allocation-free entry point is followed by
# one with a smaller input
SHAPES = [
    ((4, 512, 128, 128), 32, 1e-6),  # 128 MB: pipelined schedule (the fixed exchange array)
    ((1, 96, 500, 500), 32, 1e-6),   # 96 MB, chunks across channels: resident rounds (team slots in the fixed scratch)
    ((1, 512, 128, 128), 32, 1e-6),  # config 4a: pipelined schedule (chunk pairs in the fixed exchange array)
    ((2, 320, 64, 64), 32, 1e-5),    # config 4c: pipelined schedule
    ((2, 1280, 32, 32), 32, 1e-5),   # split schedule (chunk pairs in the fixed scratch)
    ((2, 1280, 8, 8), 32, 1e-5),     # config 4d: one workgroup per segment, no scratch
]


def _inputs(be, orc, shape, seed):
    x = orc.randn(shape, seed, 0.5, 2.0)
    C = shape[1]
    g = orc.randn((C,), seed + 1, 1.0, 0.1)
    b = orc.randn((C,), seed + 2, 0.0, 0.1)
    return x, g, b, be.array(x), be.array(g), be.array(b)


def _call(be, name, dx, dy, shape, groups, dg, db, eps):
    N, C = shape[0], shape[1]
    HW = int(np.prod(shape)) // (N * C)
    be.call(name, dx.ptr, dy.ptr, N, C, HW, groups, dg.ptr, db.ptr, eps)


def test_noalloc_equals_group_norm_silu(be, orc):
    cases, keep = [], []
    for i, (shape, groups, eps) in enumerate(SHAPES):
        x, g, b, dx, dg, db = _inputs(be, orc, shape, 9100 + 10 * i)
        want = be.empty(shape)
        _call(be, "sdh_group_norm_silu", dx, want, shape, groups, dg, db, eps)
        keep.append(want)
        cases.append((shape, groups, eps, x, g, b, dx, dg, db, want.download(), be.empty(shape)))
    be.synchronize()
    gc.collect()  # buffers dropped earlier are freed now, not between the two readings
    gc.disable()
    try:
        before = be.memory_stats()
        for shape, groups, eps, x, g, b, dx, dg, db, want, dy in cases:  # back to back, shrinking
            _call(be, "sdh_group_norm_silu_noalloc", dx, dy, shape, groups, dg, db, eps)
        be.synchronize()
        after = be.memory_stats()
    finally:
        gc.enable()
    for shape, groups, eps, x, g, b, dx, dg, db, want, dy in cases:
        got = dy.download()
        print(shape, "max |noalloc - default|", float(np.max(np.abs(got - want))), flush=True)
        assert np.array_equal(got, want), f"noalloc differs from sdh_group_norm_silu at {shape}"
    # once more in place on the 4a shape, then the smaller 4c shape
    for k in (2, 3):
        shape, groups, eps, x, g, b, dx, dg, db, want, dy = cases[k]
        _call(be, "sdh_group_norm_silu_noalloc", dx, dx, shape, groups, dg, db, eps)
        assert np.array_equal(dx.download(), want), f"noalloc in place differs at {shape}"
    shape, groups, eps, x, g, b = cases[2][:6]
    assert_reduction(cases[2][9], orc.group_norm(x, groups, g, b, eps, silu=True), "noalloc 4a vs oracle")
    assert after == before, f"arena moved across the allocation-free calls: {before} -> {after}"


def _child(env, body):
    code = ("import sys, ctypes as C; sys.path[:0] = [%r, %r]\nimport numpy as np, sdhip\n"
            % (PKG_DIR, os.path.join(ROOT, "oracle"))) + body
    r = subprocess.run([sys.executable, "-u", "-c", code], capture_output=True, text=True, timeout=240,
                       env=dict(os.environ, **env))
    print(r.stdout, r.stderr[-2000:])
    return r


def test_noalloc_rejects_before_init_and_oversize():
    """Before sdh_init: SDH_ERR_INVALID naming sdh_init, no device work.
    Split schedule forced (SDH_GN_RESIDENT=0):
      * 12800 segments of 65540 floats, whose chunk statistics (1,024,000
        bytes) exceed the 983,040 the fixed scratch holds, run in two blocks
        of segments and equal sdh_group_norm_silu (one block, arena scratch)
        bit for bit; the samples cycle through 7 distinct ones, so a block
        that read or wrote another block's segments would show;
      * one segment of 1,006,632,960 floats (122,880 chunks: its own
        statistics exceed the array) is rejected with SDH_ERR_INVALID before
        anything is launched, and the library still works."""
    body = (
        "lib = sdhip.load_library(sdhip.LIB_PATH)\n"
        "st = lib.sdh_group_norm_silu_noalloc(None, None, 1, 32, 64, 32, None, None, 1e-6)\n"
        "msg = lib.sdh_last_error().decode()\n"
        "assert st == sdhip.SDH_ERR_INVALID and 'sdh_init' in msg, (st, msg)\n"
        "from oracle import Oracle\n"
        "orc = Oracle()\n"
        "be = sdhip.Backend()\n"
        "N, C, HW, groups = 400, 32, 65540, 32\n"
        "x = be.empty((N, C, HW)); y1 = be.empty((N, C, HW)); y2 = be.empty((N, C, HW))\n"
        "S = C * HW\n"
        "samples = [be.array(orc.randn((S,), 9600 + i, 0.3 * i, 1.0 + 0.25 * i)) for i in range(7)]\n"
        "for n in range(N):\n"
        "    be.call('sdh_copy', x.ptr + 4 * n * S, samples[n % 7].ptr, 4 * S)\n"
        "g = be.array(orc.randn((C,), 9610, 1.0, 0.1)); b = be.array(orc.randn((C,), 9611, 0.0, 0.1))\n"
        "be.call('sdh_group_norm_silu_noalloc', x.ptr, y1.ptr, N, C, HW, groups, g.ptr, b.ptr, 1e-6)\n"
        "be.call('sdh_group_norm_silu', x.ptr, y2.ptr, N, C, HW, groups, g.ptr, b.ptr, 1e-6)\n"
        "a1, a2 = y1.download(), y2.download()\n"
        "assert np.isfinite(a1).all() and np.array_equal(a1, a2), 'blocked noalloc differs'\n"
        "print('blocked ok', flush=True)\n"
        "del x, y1, y2, a1, a2\n"
        "HW1 = 122880 * 8192\n"
        "big = be.empty((1, 1, HW1))\n"
        "try:\n"
        "    be.call('sdh_group_norm_silu_noalloc', big.ptr, big.ptr, 1, 1, HW1, 1, g.ptr, b.ptr, 1e-6)\n"
        "    print('accepted'); sys.exit(1)\n"
        "except sdhip.SdhError as e:\n"
        "    assert e.status == sdhip.SDH_ERR_INVALID and 'bytes of scratch' in str(e), e\n"
        "    print('rejected:', e)\n"
        "be.synchronize()\n"
        "a = be.array(np.ones(1000, np.float32)); be.add(a, be.array(np.ones(1000, np.float32)), 1000)\n"
        "assert (a.download() == 2.0).all()\n"
        "print('noalloc limits ok')\n"
    )
    r = _child({"SDH_GN_RESIDENT": "0"}, body)
    assert r.returncode == 0 and "noalloc limits ok" in r.stdout
