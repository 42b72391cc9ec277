"""GPU test of concurrent callers, through the C ABI.

Every entry point holds the library's op lock while it queues its work, so
the kernels of one op reach the single stream together. Several Python
threads (ctypes releases the GIL during each call, so the calls really run
at once) here run the ops that go through the shared scratch buffer in
several kernels - GroupNorm's split schedule, attention (pack + fused
kernel), the bf16 GEMM (packed A), conv2d (gather + GEMM) - on their own
inputs, many times, and every result must equal the one computed alone.
"""
import threading

import numpy as np
import pytest

from oracle import f32_to_bf16

pytestmark = pytest.mark.gpu


def _jobs(be, orc, t):
    """A list of (run, read) pairs for thread t: run() queues the op, read()
    downloads its output."""
    jobs = []
    x = be.array(orc.randn((1, 32, 300, 300), 7000 + t, 0.5, 2.0))  # > 64K floats per group: split schedule
    g, b = be.array(orc.randn((32,), 7100 + t, 1.0, 0.1)), be.array(orc.randn((32,), 7200 + t))
    y = be.empty((1, 32, 300, 300))
    jobs.append((lambda: be.group_norm(x, y, 1, 32, 90000, 8, g, b, 1e-6, silu=True), y.download))
    q, k, v = (be.array(orc.randn((1, 200, 4 * 64), 7300 + 10 * t + i)) for i in range(3))
    o = be.empty((1, 200, 4 * 64))
    jobs.append((lambda: be.attention(q, k, v, o, 1, 200, 200, 4, 4, 64, True), o.download))
    A = be.array(orc.randn((300, 256), 7400 + t))
    W = be.array(f32_to_bf16(orc.randn((200, 256), 7500 + t, 0.0, 0.05)))
    C = be.empty((300, 200))
    jobs.append((lambda: be.gemm_nt_bf16(300, 200, 256, A, 256, W, 256, C, 200), C.download))
    xc = be.array(orc.randn((1, 16, 40, 40), 7600 + t))
    wc = be.array(orc.randn((24, 16, 3, 3), 7700 + t, 0.0, 0.1))
    oc = be.empty((1, 24, 40, 40))
    jobs.append((lambda: be.conv2d(xc, 1, 16, 40, 40, wc, 24, 3, 3, None, 1, 1, oc, 40, 40), oc.download))
    keep = [x, g, b, y, q, k, v, o, A, W, C, xc, wc, oc]
    return jobs, keep


def test_concurrent_callers_match_serial_results(be, orc):
    threads = 4
    work = [_jobs(be, orc, t) for t in range(threads)]
    want = []
    for jobs, _ in work:  # each op alone
        res = []
        for run, read in jobs:
            run()
            res.append(read())
        want.append(res)
    errors = []

    def worker(t):
        try:
            jobs, _ = work[t]
            for rep in range(6):
                for i, (run, read) in enumerate(jobs):
                    run()
                    got = read()
                    if not np.array_equal(got, want[t][i]):
                        errors.append((t, rep, i))
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append((t, repr(e)))

    pool = [threading.Thread(target=worker, args=(t,)) for t in range(threads)]
    for th in pool:
        th.start()
    for th in pool:
        th.join(timeout=120)
    assert not any(th.is_alive() for th in pool), "a caller did not finish"
    assert not errors, errors[:10]
