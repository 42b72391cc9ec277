"""Golden fixtures written by tests/golden/make_golden.py from the compiled
reference (the reference's own tensor.cpp). CPU side: the oracle must
reproduce every small-op fixture (bit for bit: same compiler family, same
flags, same libm), which pins the oracle without needing /root/reference.
The GPU side of the same fixtures is tests/test_gpu_golden.py.
"""
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def small():
    return dict(np.load(os.path.join(GOLDEN, "ops_small.npz"), allow_pickle=False))


def inputs(orc, small):
    """Regenerates every seeded input named in the fixture file."""
    out = {}
    for k, v in small.items():
        if k.startswith("in/"):
            seed, mean, std = int(v[0]), float(v[1]), float(v[2])
            shape = tuple(int(s) for s in v[3:])
            out[k[3:]] = orc.randn(shape, seed, mean, std)
    return out


def oracle_outputs(orc, small):
    i = inputs(orc, small)
    o = {}
    o["rms_norm"] = orc.rms_norm(i["x"], i["g"], 1e-6)
    o["layer_norm"] = orc.layer_norm(i["z"], i["g64"], i["b64"], 1e-5)
    o["layer_norm_noaffine"] = orc.layer_norm(i["z"], None, None, 1e-5)
    o["group_norm"] = orc.group_norm(i["img"], 32, i["g64"], i["b64"], 1e-6)
    o["group_norm_silu"] = orc.group_norm(i["img"], 32, i["g64"], i["b64"], 1e-6, silu=True)
    o["rms_norm_heads"] = orc.rms_norm_heads(i["x"].reshape(15, 8), 8, i["gd"], 1e-6)
    cs, sn = small["rope_cos"], small["rope_sin"]
    o["rope_half"] = orc.rope(i["xr"], 8, cs, sn, False)
    o["rope_inter"] = orc.rope(i["xr"], 8, cs, sn, True)
    o["swiglu"] = orc.swiglu(i["xr"], i["u"])
    o["geglu"] = orc.geglu(i["gg"])
    for op in ("silu", "tanh", "gelu", "quick_gelu"):
        o[op] = getattr(orc, op)(i["a"])
    o["add"] = orc.add(i["a"], i["b"])
    o["scale"] = orc.scale(i["a"], 0.37)
    o["affine"] = orc.affine(i["a"], 1.5, -0.25)
    o["mul_rows"] = orc.mul_rows(i["m"], i["v"])
    o["add_rows_scaled"] = orc.add_rows_scaled(i["m"], i["my"], i["v"])
    o["add_channel_bias"] = orc.add_channel_bias(i["cimg"], i["cb"])
    o["softmax_causal"] = orc.softmax_rows(i["sm"], 0.35, True)
    o["softmax"] = orc.softmax_rows(i["sm2"], 0.125, False)
    o["ln_modulate_gate_res"], o["ln_modulate_gate_y"] = orc.ln_modulate_gate(i["lx"], i["lr"], i["lsc"], i["lsh"],
                                                                              i["lgt"], 1e-6)
    o["add_rms_norm_sum"], o["add_rms_norm_y"] = orc.add_rms_norm(i["lx"], i["lr"], i["g64"], 1e-6)
    # layout ops: the oracle's restatements, and for the pure memcpy ops
    # (tensor.cpp:970-980, :1025-1039, :1076-1099) their numpy equivalent
    img, img2 = i["cimg"], i["img2"]
    o["upsample_nearest2x"] = orc.upsample_nearest2x(img)
    o["concat_channels"] = orc.concat_channels(img, img2)
    cb = np.zeros((img.shape[0] + img2.shape[0],) + img.shape[1:], np.float32)
    cb.reshape(-1)[:img.size] = img.reshape(-1)
    cb.reshape(-1)[img.size:img.size + img2.size] = img2.reshape(-1)
    o["concat_batch"] = cb
    o["nchw_to_nlc"] = orc.nchw_to_nlc(img)
    o["nlc_to_nchw"] = orc.nlc_to_nchw(o["nchw_to_nlc"], 4, 5)
    o["slice_batch"] = img[1:2].copy()
    o["repeat_batch"] = np.concatenate([img] * 3, axis=0)
    o["slice_rows"] = i["m"][1:3].copy()
    o["patchify2d"] = orc.patchify(i["lat"], 2)
    o["unpatchify2d"] = orc.unpatchify(o["patchify2d"], 16, 6, 8, 2)
    return o


def test_fixture_files_are_data_only():
    for f in ("ops_small.npz", "configs.npz"):
        d = np.load(os.path.join(GOLDEN, f), allow_pickle=False)  # raises if anything needs unpickling
        assert all(d[k].dtype in (np.float32, np.float64) for k in d.files)


def test_oracle_reproduces_reference_fixtures(orc, small):
    got = oracle_outputs(orc, small)
    expected = [k for k in small if not k.startswith("in/") and not k.startswith("rope_cos") and not k.startswith("rope_sin")]
    assert set(got) == set(expected)
    for k in expected:
        assert got[k].shape == small[k].shape, k
        assert np.array_equal(got[k], small[k]), f"{k}: max diff {np.max(np.abs(got[k] - small[k])):.3e}"
