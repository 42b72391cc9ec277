"""GPU test of arena exhaustion, forced from the host: the arena capped with
SDH_ARENA_LIMIT_MB in a child process (the role of the reference's
allocation-failure path, backend_cuda.cu:139-147, which flushes its cache
and retries once before throwing).

  * an allocation beyond the cap fails with SDH_ERR_OOM and a message that
    names the request, and nothing else changes;
  * with the arena filled, an op that needs library scratch (GroupNorm's
    split schedule) fails with SDH_ERR_OOM before launching anything, while
    the allocation-free GroupNorm entry point still runs;
  * once the fill is freed the same op succeeds and matches the oracle, and
    the arena's reserved bytes never exceeded the cap.
"""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
PKG_DIR = os.path.join(ROOT, "stablediffusion-cpp_amd")
ORACLE_DIR = os.path.join(ROOT, "oracle")

BODY = r"""
import sys
sys.path[:0] = [%r, %r, %r]
import numpy as np, sdhip
from oracle import Oracle
from tolerances import assert_reduction
MB = 1 << 20
be, orc = sdhip.Backend(), Oracle()
shape, groups, eps = (2, 1280, 32, 32), 32, 1e-5   # split schedule (chunks cross channels): needs scratch
N, C, HW = 2, 1280, 32 * 32
x = orc.randn(shape, 8101, 0.0, 2.0)
g = orc.randn((C,), 8102, 1.0, 0.1); b = orc.randn((C,), 8103, 0.0, 0.1)
dx, dy, dg, db = be.array(x), be.empty(shape), be.array(g), be.array(b)
want = orc.group_norm(x, groups, g, b, eps, silu=True)

# 1. one request beyond the cap
try:
    be.malloc(600 * MB); print('600 MB accepted'); sys.exit(1)
except sdhip.SdhError as e:
    assert e.status == sdhip.SDH_ERR_OOM and 'arena exhausted' in str(e) and str(600 * MB) in str(e), e
    print('oom:', e, flush=True)

# 2. fill the arena, then an op that needs scratch
fill = []
for size in (16 * MB, MB, 64 << 10, 4 << 10, 256):  # down to the arena's 256-byte granule
    while True:
        try:
            fill.append(be.malloc(size))
        except sdhip.SdhError as e:
            assert e.status == sdhip.SDH_ERR_OOM, e
            break
reserved, in_use = be.memory_stats()
assert reserved <= 512 * MB, reserved
print('filled:', len(fill), 'blocks; reserved', reserved, 'in use', in_use, flush=True)
try:
    be.group_norm(dx, dy, N, C, HW, groups, dg, db, eps, silu=True)
    be.synchronize(); print('op ran without scratch'); sys.exit(1)
except sdhip.SdhError as e:
    assert e.status == sdhip.SDH_ERR_OOM and 'scratch' in str(e), e
    print('op oom:', e, flush=True)
be.call('sdh_group_norm_silu_noalloc', dx.ptr, dy.ptr, N, C, HW, groups, dg.ptr, db.ptr, eps)
assert_reduction(dy.download(), want, 'allocation-free GroupNorm with the arena full')

# 3. free the fill: the op now runs and is right
for p in fill:
    be.free(p)
be.group_norm(dx, dy, N, C, HW, groups, dg, db, eps, silu=True)
assert_reduction(dy.download(), want, 'GroupNorm after the arena was freed')
assert be.memory_stats()[0] <= 512 * MB
print('arena limit ok', flush=True)
""" % (PKG_DIR, ORACLE_DIR, HERE)


def test_arena_exhaustion_is_reported_and_recovers():
    r = subprocess.run([sys.executable, "-u", "-c", BODY], capture_output=True, text=True, timeout=240,
                       env=dict(os.environ, SDH_ARENA_MB="256", SDH_ARENA_LIMIT_MB="512"))
    print(r.stdout, r.stderr[-3000:])
    assert r.returncode == 0 and "arena limit ok" in r.stdout
