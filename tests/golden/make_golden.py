#!/usr/bin/env python3
"""Writes the golden fixtures under tests/golden/ from the COMPILED REFERENCE
(oracle/_ref/libsdref.so = /root/reference/src/tensor.cpp, built by
oracle/Makefile). Run where /root/reference is mounted:

    make -C oracle all ref && python tests/golden/make_golden.py [--small-only]

Outputs (data only: inputs are regenerated from their seeds by the oracle's
portable generator, expected outputs come from the reference):
  ops_small.npz   full outputs of every op on small seeded inputs
  configs.npz     for each BASELINE config at full size: the reference
                  output's float64 checksums (sum, sum of squares, sum of |y|)
                  and a strided sample of elements
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
from oracle import Oracle, Reference  # noqa: E402

T, D, F = 4096, 3840, 10240
STRIDE = 9973  # sample every STRIDE-th element (prime, so it walks all columns)


def small_cases(orc, ref):
    out = {}

    def rnd(name, shape, seed, mean=0.0, std=1.0):
        out[f"in/{name}"] = np.array([seed, mean, std] + list(shape), np.float64)
        return orc.randn(shape, seed, mean, std)

    x = rnd("x", (5, 24), 11)
    g = rnd("g", (24,), 12)
    out["rms_norm"] = ref.rms_norm(x, g, 1e-6)
    z = rnd("z", (3, 7, 64), 13, 2.0, 3.0)
    g64 = rnd("g64", (64,), 14, 1.0, 0.1)
    b64 = rnd("b64", (64,), 15, 0.0, 0.1)
    out["layer_norm"] = ref.layer_norm(z, g64, b64, 1e-5)
    out["layer_norm_noaffine"] = ref.layer_norm(z, None, None, 1e-5)
    img = rnd("img", (2, 64, 5, 7), 16, 0.0, 2.0)
    out["group_norm"] = ref.group_norm(img, 32, g64, b64, 1e-6)
    out["group_norm_silu"] = ref.group_norm(img, 32, g64, b64, 1e-6, silu=True)
    gd = rnd("gd", (8,), 17)
    out["rms_norm_heads"] = ref.rms_norm_heads(x.reshape(15, 8), 8, gd, 1e-6)
    xr = rnd("xr", (1, 5, 24), 18)
    ang = np.array([[0.1 * s * (i % 4 + 1) for i in range(8)] for s in range(5)], np.float32)
    cs, sn = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    out["rope_cos"], out["rope_sin"] = cs, sn
    out["rope_half"] = ref.rope(xr, 8, cs, sn, False)
    out["rope_inter"] = ref.rope(xr, 8, cs, sn, True)
    u = rnd("u", (1, 5, 24), 19)
    out["swiglu"] = ref.swiglu(xr, u)
    gg = rnd("gg", (6, 40), 20)
    out["geglu"] = ref.geglu(gg)
    a = rnd("a", (1000,), 21, 0.0, 3.0)
    for op in ("silu", "tanh", "gelu", "quick_gelu"):
        out[op] = getattr(ref, op)(a)
    b = rnd("b", (1000,), 22)
    out["add"] = ref.add(a, b)
    out["scale"] = ref.scale(a, 0.37)
    out["affine"] = ref.affine(a, 1.5, -0.25)
    m = rnd("m", (4, 6), 23)
    v = rnd("v", (6,), 24)
    my = rnd("my", (4, 6), 25)
    out["mul_rows"] = ref.mul_rows(m, v)
    out["add_rows_scaled"] = ref.add_rows_scaled(m, my, v)
    cimg = rnd("cimg", (2, 3, 4, 5), 26)
    cb = rnd("cb", (2, 3), 27)
    out["add_channel_bias"] = ref.add_channel_bias(cimg, cb)
    sm = rnd("sm", (54, 9), 28, 0.0, 3.0)
    out["softmax_causal"] = ref.softmax_rows(sm, 0.35, True)
    sm2 = rnd("sm2", (33, 100), 29, 0.0, 3.0)
    out["softmax"] = ref.softmax_rows(sm2, 0.125, False)
    lx = rnd("lx", (7, 64), 30)
    lr = rnd("lr", (7, 64), 31)
    lsc = rnd("lsc", (64,), 32, 0.0, 0.2)
    lsh = rnd("lsh", (64,), 33, 0.0, 0.2)
    lgt = rnd("lgt", (64,), 34, 0.0, 0.2)
    out["ln_modulate_gate_res"], out["ln_modulate_gate_y"] = ref.ln_modulate_gate(lx, lr, lsc, lsh, lgt, 1e-6)
    out["add_rms_norm_sum"], out["add_rms_norm_y"] = ref.add_rms_norm(lx, lr, g64, 1e-6)
    # layout ops, on the shapes of the reference's own GPU test (test_ops.cpp:462-476)
    img2 = rnd("img2", (2, 2, 4, 5), 35)
    out["upsample_nearest2x"] = ref.upsample_nearest2x(cimg)
    out["concat_channels"] = ref.concat_channels(cimg, img2)
    out["concat_batch"] = ref.concat_batch(cimg, img2)  # shapes differ: the reference leaves a zero tail
    out["nchw_to_nlc"] = ref.nchw_to_nlc(cimg)
    out["nlc_to_nchw"] = ref.nlc_to_nchw(out["nchw_to_nlc"], 4, 5)
    out["slice_batch"] = ref.slice_batch(cimg, 1)
    out["repeat_batch"] = ref.repeat_batch(cimg, 3)
    out["slice_rows"] = ref.slice_rows(m, 1, 3)
    lat = rnd("lat", (1, 16, 6, 8), 36)
    out["patchify2d"] = ref.patchify(lat, 2)
    out["unpatchify2d"] = ref.unpatchify(out["patchify2d"], 16, 6, 8, 2)
    return out


def checksums(y):
    y64 = y.astype(np.float64).reshape(-1)
    return np.array([y64.sum(), (y64 * y64).sum(), np.abs(y64).sum(), y64.size], np.float64)


def config_cases(orc, ref):
    """Reference outputs at the BASELINE config shapes (same seeds as the GPU
    config-shape test in tests/test_gpu_golden.py)."""
    out = {}

    def keep(name, y):
        out[f"{name}/sum"] = checksums(y)
        out[f"{name}/sample"] = y.reshape(-1)[::STRIDE].copy()

    x, r = orc.randn((T, D), 101), orc.randn((T, D), 102)
    w = orc.randn((D,), 103, 1.0, 0.1)
    s, y = ref.add_rms_norm(x, r, w, 1e-6)
    keep("c1_sum", s)
    keep("c1_norm", y)
    del x, r, s, y
    g, u = orc.randn((T, F), 104, 0.0, 1.5), orc.randn((T, F), 105, 0.0, 1.5)
    keep("c2_swiglu", ref.swiglu(g, u))
    del g, u
    pos = np.array([[0, h, w_] for h in range(64) for w_ in range(64)], np.int32)
    cs, sn = ref_tables = orc.rope_tables_3axis(pos, [32, 48, 48], 128, 256.0)
    q = orc.randn((1, T, D), 106)
    keep("c3_rope_q", ref.rope(q, 128, cs, sn, True))
    del q, ref_tables
    for tag, shape, eps, seed in (("c4a", (1, 512, 128, 128), 1e-6, 107), ("c4b", (1, 128, 1024, 1024), 1e-6, 108),
                                  ("c4c", (2, 320, 64, 64), 1e-5, 109), ("c4d", (2, 1280, 8, 8), 1e-5, 110)):
        xg = orc.randn(shape, seed, 0.0, 2.0)
        gm = orc.randn((shape[1],), seed + 1000, 1.0, 0.1)
        bt = orc.randn((shape[1],), seed + 2000, 0.0, 0.1)
        keep(f"{tag}_gn_silu", ref.group_norm(xg, 32, gm, bt, eps, silu=True))
        del xg
    x, res = orc.randn((T, D), 111), orc.randn((T, D), 112)
    sc, sh, gt = (orc.randn((D,), 113 + i, 0.0, 0.2) for i in range(3))
    r5, _ = ref.ln_modulate_gate(x, res, sc, sh, gt, 1e-6)
    keep("c5a_res", r5)
    del x, res, r5
    sm = orc.randn((30 * T, T), 116, 0.0, 3.0)
    keep("c5b_softmax", ref.softmax_rows(sm, 1.0 / np.sqrt(128.0), False))
    return out


def main():
    orc, ref = Oracle(), Reference()
    small = small_cases(orc, ref)
    np.savez_compressed(os.path.join(HERE, "ops_small.npz"), **small)
    files = ["ops_small.npz"]
    if "--small-only" not in sys.argv:  # the config summaries take a few minutes of CPU
        cfg = config_cases(orc, ref)
        np.savez_compressed(os.path.join(HERE, "configs.npz"), **cfg)
        files.append("configs.npz")
    for f in files:
        print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")


if __name__ == "__main__":
    main()
