#!/usr/bin/env python3
"""Benchmark of backend_hip's elementwise / reduction / broadcast path on one
MI355X, against the HBM roofline, with the reference's CPU path timed beside it.

Metric: achieved HBM GB/s (% of peak) per op at Z-Image 1024^2
shapes; speedup vs CPU. The headline line is the SwiGLU configuration
(configs[1]: gate, up [4096, 10240] fp32); every other BASELINE config is
measured too and reported in the same JSON line under "ops".

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]
                  [--no-cpu] [--cpu-all] [--list]

A step is one call of the op over one batch of synthetic input that is already
resident in HBM. Inputs are rotated over the fewest buffer sets (at least
two) that hold at least 512 MB of distinct data (2x the 256 MB Infinity
Cache), so repeated steps read HBM, not cache. Larger rotations are not "more honest": measured on
MI355X, streaming kernels lose ~15 points of HBM peak once the buffers touched
between two uses of the same set exceed ~0.6-0.9 GB (GPU TLB reach), which is
a property of the benchmark loop, not of the kernel. GB/s = algorithmic bytes (each input read once, each output written
once) / time. Kernel time comes from HIP events recorded on the library's
stream around the timed steps; ms_per_step from the host clock around the same
steps (both bracketed by a device synchronize).

The CPU baseline is the reference's own tensor.cpp (oracle/_ref, compiled from
/root/reference) timed in this process on the host's cores; if it is absent,
the C restatement (oracle/liboracle.so) is timed instead ("port"). It is timed
on every BASELINE config line by default (median of 5 runs after one, 3 for
tensors over 1 GB); --cpu-all adds the other lines.

Ops whose step is shorter than 10 us are launch-bound: a ctypes loop (5-7 us
per call) cannot issue them as fast as the GPU runs them. Their steps are also
captured into one graph (sdh_capture_begin) and replayed, and us_per_op is
that replay's device time; the host-paced figure is kept as
us_per_op_host_paced. Ops of 10-25 us are replayed too, and keep the
host-paced figure, the GPU being the bound there, with the replay's as
us_per_op_graph.

Every line is measured on the GPU first, back to back, and the CPU legs and
parity checks run after the last one: a CPU leg between two measurements
leaves the GPU idle for seconds, and the next line would time its clocks
coming back up (measured: 4b 191 us per op over the first 20 steps after 5
warm-up steps, 181 us once settled). The headline takes exactly --warmup
untimed steps and times exactly --steps; every other line warms up for at
least 30 ms of its own steps (and at least 3 of them) and times at least 10 ms
of steps (at least --op-steps; `timed_steps` in its entry; a captured graph
at most 256 of them).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import re
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "stablediffusion-cpp_amd"))

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFS = 2500.0  # dense bf16 MFMA peak of the MI355X (no sparsity)
METRIC = "achieved HBM GB/s (% of peak) per op at Z-Image 1024² shapes; speedup vs CPU"
T, D, F = 4096, 3840, 10240
MIN_ROTATION_BYTES = 512_000_000  # 2x the 256 MB Infinity Cache
MAX_SETS = 32
# ops whose host-paced step is shorter than GRAPH_ALSO_MS are also timed as
# one captured graph of the same steps; below GRAPH_BELOW_MS the graph's time
# is the line's figure (the ctypes loop, 5-7 us per call, cannot keep the GPU
# busy), above it the host-paced loop's (the GPU is then the bound, and a
# replay adds the graph's own per-node cost: GroupNorm 4a 12.0 us host-paced,
# 12.8 us replayed), with the other figure kept beside it
GRAPH_BELOW_MS = 0.010
GRAPH_ALSO_MS = 0.025
# per-op lines: the warm-up runs for at least this long (and at least its
# step count), in batches with a synchronisation after each, so the GPU's
# clocks are at their loaded level when the timed steps start
OP_WARM_S = 0.03
OP_WARM_BATCH = 8
# per-op lines time at least this long (more than --op-steps steps for ops
# under 500 us): the first launches after the warm-up's synchronisation run
# slower than the rest (kernel trace: GroupNorm 4b's first 191-204 us against
# 172-190 us, 4a's first two 0.5-1.7 us slower), a bias of 0.75 us per op
# over 20 steps of 4b
OP_TIMED_S = 0.01
# the captured graph of a launch-bound line holds at most this many steps
GRAPH_MAX_STEPS = 256


# ------------------------------------------------------------------ workloads
class Workload:
    """One BASELINE config (or calibration / model line): its inputs, one step
    on the device, and the reference's CPU composition of the same step.

    inputs:  (name, shape, mean, std, seed) of each fp32 input ~N(mean, std),
             generated on the device by the library's seeded generator
             (sdh_fill_normal: splitmix64 + Box-Muller), seed + 1000 i for
             set i. Set 0 is downloaded before the timed steps, and the
             reference's CPU step runs on exactly those arrays.
    outputs: (name, shape) allocated uninitialised on the device.
    results: the arrays compared with the reference after one step (outputs,
             or inputs updated in place), with the tolerance of each:
             ("abs", b) max-abs, ("rel", b) |d| / max(|want|, 1),
             ("softmax", b) elementwise relative with exact causal zeros,
             ("normrel", b) max|d| / max|want|."""

    name = ""
    desc = ""
    kernel = ""  # substring of the dominant kernel's name (for rocprof)
    algo_bytes = 0
    inputs = ()
    outputs = ()
    results = {}

    def make(self, be, i):
        d = {}
        for n, shape, mean, std, seed in self.inputs:
            d[n] = be.randn(shape, seed + 1000 * i, mean, std)
        for n, shape in self.outputs:
            d[n] = be.empty(shape)
        return d

    def host_inputs(self, s):
        """Set s's inputs on the host (what the reference's CPU step gets)."""
        return {n: s[n].download() for n, *_ in self.inputs}

    def reload(self, be, s, host):
        """Set 0's inputs uploaded again (in-place steps changed them)."""
        for n, *_ in self.inputs:
            s[n].upload(host[n])

    def step(self, be, s):
        raise NotImplementedError

    def gpu_results(self, be, s):
        return {n: s[n].download() for n in self.results}

    def cpu(self, R, h):
        """(run, handles, collect): run() executes the reference composition
        once and returns the handles it allocated; collect(outs) copies the
        results of one run out of the reference's tensors."""
        return None

    def seeds(self):
        return {n: seed for n, _, _, _, seed in self.inputs}


def _tables_3axis(S, side):
    """Z-Image interleaved cos/sin [S, 128] for positions (0, h, w) (zimage.cpp:71-88)."""
    pos = np.array([[0, h, w] for h in range(side) for w in range(side)], np.int64)[:S]
    cs = np.empty((S, 128), np.float32)
    sn = np.empty((S, 128), np.float32)
    off = 0
    for a, da in enumerate((32, 48, 48)):
        freq = 1.0 / np.power(256.0, np.arange(da // 2) * 2.0 / da)
        ang = (pos[:, a:a + 1].astype(np.float64) * freq).astype(np.float32)
        c, s = np.cos(ang.astype(np.float64)).astype(np.float32), np.sin(ang.astype(np.float64)).astype(np.float32)
        cs[:, off:off + da:2], cs[:, off + 1:off + da:2] = c, c
        sn[:, off:off + da:2], sn[:, off + 1:off + da:2] = s, s
        off += da
    return cs, sn


def _peek(R, h, shape):
    return R.view(h).copy().reshape(shape)


class AddRmsNorm(Workload):
    config_line = True  # a BASELINE config: the reference CPU path is timed beside it
    name, kernel = "add_rms_norm", "k_add_rms"
    desc = "config 1: x += r; y = rms_norm(x) * w; x, r [4096,3840], w [3840], eps 1e-6"
    algo_bytes = 4 * T * D * 4 + D * 4
    inputs = (("x", (T, D), 0.0, 1.0, 1), ("r", (T, D), 0.0, 1.0, 2), ("w", (D,), 1.0, 0.1, 3))
    outputs = (("y", (T, D)),)
    results = {"x": ("abs", 1e-5), "y": ("rel", 1e-4)}

    def step(self, be, s):
        be.add_rms_norm(s["x"], s["r"], s["y"], T, D, s["w"], 1e-6)

    def cpu(self, R, h):
        hx, hr, hw = R.new((T, D), h["x"]), R.new((T, D), h["r"]), R.new((D,), h["w"])

        def run():
            R._chk(R.lib.ref_add_(hx, hr))
            return [R._ptr(R.lib.ref_rms_norm(hx, hw, 1e-6))]

        return run, [hx, hr, hw], lambda outs: {"x": _peek(R, hx, (T, D)), "y": _peek(R, outs[0], (T, D))}


class SwiGLU(Workload):
    config_line = True  # a BASELINE config: the reference CPU path is timed beside it
    name, kernel = "swiglu", "k_swiglu"
    desc = "config 2: y = silu(g) * u; g, u [4096,10240] ~N(0,1.5)"
    algo_bytes = 3 * T * F * 4
    inputs = (("g", (T, F), 0.0, 1.5, 4), ("u", (T, F), 0.0, 1.5, 5))
    outputs = (("y", (T, F)),)
    results = {"y": ("abs", 1e-5)}

    def step(self, be, s):
        be.swiglu(s["g"], s["u"], s["y"], T * F)

    def cpu(self, R, h):
        hg, hu = R.new((T, F), h["g"]), R.new((T, F), h["u"])
        return (lambda: [R._ptr(R.lib.ref_swiglu(hg, hu))]), [hg, hu], lambda outs: {"y": _peek(R, outs[0], (T, F))}


class RopeQK(Workload):
    config_line = True  # a BASELINE config: the reference CPU path is timed beside it
    name, kernel = "rope_qk", "k_rope_il_reg"
    desc = ("config 3: 3-axis interleaved RoPE in place on q and k [4096,30*128] in one launch, axes (32,48,48), "
            "theta 256, reference-format duplicated cos/sin tables [4096,128]")
    algo_bytes = 4 * T * D * 4 + 2 * T * 128 * 4
    inputs = (("q", (T, D), 0.0, 1.0, 6), ("k", (T, D), 0.0, 1.0, 7))
    results = {"q": ("abs", 1e-5), "k": ("abs", 1e-5)}

    def __init__(self):
        self.cs, self.sn = _tables_3axis(T, 64)

    def make(self, be, i):
        d = super().make(be, i)
        d.update(c=be.array(self.cs), s=be.array(self.sn))
        return d

    def step(self, be, s):
        be.rope_qk(s["q"], D, s["k"], D, 1, T, 128, s["c"], s["s"], True)

    def cpu(self, R, h):
        hq, hk = R.new((1, T, D), h["q"]), R.new((1, T, D), h["k"])
        hc, hs = R.new(self.cs.shape, self.cs), R.new(self.sn.shape, self.sn)

        def run():
            R._chk(R.lib.ref_rope_(hq, 128, hc, hs, 1))
            R._chk(R.lib.ref_rope_(hk, 128, hc, hs, 1))
            return []

        return run, [hq, hk, hc, hs], lambda outs: {"q": _peek(R, hq, (T, D)), "k": _peek(R, hk, (T, D))}


class RopeQKAxes(RopeQK):
    """Config 3 with sin/cos computed on the device (sdh_rope_qk_axes): the
    angles come from the positions (0, h, w) of the 64 x 64 grid [4096, 3]
    int32, axes (32, 48, 48), theta 256; no table crosses HBM. The reference's
    CPU rope_ runs with the tables of the same positions."""

    name, kernel = "rope_qk_axes", "k_rope_il_axes"
    desc = ("config 3: 3-axis interleaved RoPE in place on q and k [4096,30*128] in one launch, axes (32,48,48), "
            "theta 256, sin/cos computed on the device from the [4096,3] int32 positions (0,h,w)")
    algo_bytes = 4 * T * D * 4 + T * 3 * 4

    def __init__(self):
        super().__init__()
        self.pos = np.array([[0, h, w] for h in range(64) for w in range(64)], np.int32)

    def make(self, be, i):
        d = Workload.make(self, be, i)
        d["p"] = be.array(self.pos.view(np.float32))
        return d

    def step(self, be, s):
        be.rope_qk_axes(s["q"], D, s["k"], D, 1, T, 128, s["p"], (32, 48, 48), 256.0)


class QKNormRope(Workload):
    """Fused QK-norm + RoPE at the config-3 shape (zimage.cpp:117-120). With
    unfused=True the same result through the op sequence the reference calls
    (two rms_norm_heads_ and the two rope_), for comparison; both are rated
    on the fused op's algorithmic bytes."""

    results = {"q": ("rel", 1e-4), "k": ("rel", 1e-4)}
    inputs = (("q", (T, D), 0.0, 1.0, 17), ("k", (T, D), 0.0, 1.0, 18), ("gq", (128,), 1.0, 0.1, 19),
              ("gk", (128,), 1.0, 0.1, 20))

    def __init__(self, unfused=False):
        self.unfused = unfused
        self.name = "qknorm_rope_unfused" if unfused else "qknorm_rope"
        self.kernel = "k_heads" if unfused else "k_qknorm_rope_il"
        self.desc = ("QK-norm (eps 1e-5, gamma [128]) then 3-axis interleaved RoPE on q and k [4096,30*128] in place" +
                     (": the unfused GPU sequence (2 x rms_norm_heads + rope_qk), rated on the fused bytes"
                      if unfused else ", one launch"))
        self.algo_bytes = 4 * T * D * 4 + 2 * T * 128 * 4 + 2 * 128 * 4
        self.cs, self.sn = _tables_3axis(T, 64)

    def make(self, be, i):
        d = super().make(be, i)
        d.update(c=be.array(self.cs), s=be.array(self.sn))
        return d

    def step(self, be, s):
        if self.unfused:
            be.rms_norm_heads(s["q"], T * 30, 128, s["gq"], 1e-5)
            be.rms_norm_heads(s["k"], T * 30, 128, s["gk"], 1e-5)
            be.rope_qk(s["q"], D, s["k"], D, 1, T, 128, s["c"], s["s"], True)
        else:
            be.qknorm_rope(s["q"], D, s["k"], D, 1, T, 128, s["gq"], s["gk"], 1e-5, s["c"], s["s"], True)

    def cpu(self, R, h):
        hq, hk = R.new((1, T, D), h["q"]), R.new((1, T, D), h["k"])
        hgq, hgk = R.new((128,), h["gq"]), R.new((128,), h["gk"])
        hc, hs = R.new(self.cs.shape, self.cs), R.new(self.sn.shape, self.sn)

        def run():
            R._chk(R.lib.ref_rms_norm_heads_(hq, 128, hgq, 1e-5))
            R._chk(R.lib.ref_rms_norm_heads_(hk, 128, hgk, 1e-5))
            R._chk(R.lib.ref_rope_(hq, 128, hc, hs, 1))
            R._chk(R.lib.ref_rope_(hk, 128, hc, hs, 1))
            return []

        return run, [hq, hk, hgq, hgk, hc, hs], lambda outs: {"q": _peek(R, hq, (T, D)), "k": _peek(R, hk, (T, D))}


class GNSiLU(Workload):
    config_line = True  # a BASELINE config: the reference CPU path is timed beside it
    kernel = "k_gn_"
    results = {"y": ("rel", 1e-4)}

    def __init__(self, tag, shape, eps, note):
        self.shape, self.eps = shape, eps
        self.name = f"group_norm_silu_{tag}"
        self.desc = f"config {note}: y = silu(group_norm(x, 32 groups, eps {eps:g})), x {list(shape)} ~N(0,2)"
        n = int(np.prod(shape))
        self.algo_bytes = 2 * n * 4 + 2 * shape[1] * 4
        Cc = shape[1]
        self.inputs = (("x", shape, 0.0, 2.0, 8), ("g", (Cc,), 1.0, 0.1, 9), ("b", (Cc,), 0.0, 0.1, 10))
        self.outputs = (("y", shape),)

    def step(self, be, s):
        N, Cc = self.shape[0], self.shape[1]
        HW = int(np.prod(self.shape[2:]))
        be.group_norm(s["x"], s["y"], N, Cc, HW, 32, s["g"], s["b"], self.eps, silu=True)

    def cpu(self, R, h):
        Cc = self.shape[1]
        hx, hg, hb = R.new(self.shape, h["x"]), R.new((Cc,), h["g"]), R.new((Cc,), h["b"])

        def run():
            o = R._ptr(R.lib.ref_group_norm(hx, 32, hg, hb, self.eps))
            R._chk(R.lib.ref_silu_(o))
            return [o]

        return run, [hx, hg, hb], lambda outs: {"y": _peek(R, outs[0], self.shape)}


class LNModGate(Workload):
    config_line = True  # a BASELINE config: the reference CPU path is timed beside it
    name, kernel = "ln_modulate_gate", "k_ln_mod_gate"
    desc = ("config 5a: y = layer_norm(x)*(1+scale)+shift; res += tanh(gate)*y (y not stored); x, res [4096,3840]; "
            "scale, shift, gate [3840] ~N(0,0.2); eps 1e-6")
    algo_bytes = 3 * T * D * 4 + 3 * D * 4
    inputs = (("x", (T, D), 0.0, 1.0, 11), ("res", (T, D), 0.0, 1.0, 12), ("sc", (D,), 0.0, 0.2, 13),
              ("sh", (D,), 0.0, 0.2, 14), ("gt", (D,), 0.0, 0.2, 15))
    results = {"res": ("rel", 1e-4)}

    def step(self, be, s):
        be.ln_modulate_gate(s["x"], s["res"], s["sc"], s["sh"], s["gt"], None, T, D, 1e-6)

    def cpu(self, R, h):
        hx, hr = R.new((T, D), h["x"]), R.new((T, D), h["res"])
        hsc, hsh, hgt = R.new((D,), h["sc"]), R.new((D,), h["sh"]), R.new((D,), h["gt"])
        hones = R.new((T, D), np.ones((T, D), np.float32))

        def run():
            # scale and gate are transformed in place by the composition: fresh copies each run
            R.view(hsc)[...] = h["sc"]
            R.view(hgt)[...] = h["gt"]
            y = R._ptr(R.lib.ref_layer_norm(hx, None, None, 1e-6))
            R._chk(R.lib.ref_affine_(hsc, 1.0, 1.0))
            R._chk(R.lib.ref_tanh_(hgt))
            R._chk(R.lib.ref_mul_rows_(y, hsc))
            R._chk(R.lib.ref_add_rows_scaled_(y, hones, hsh))
            R._chk(R.lib.ref_add_rows_scaled_(hr, y, hgt))
            return [y]

        return run, [hx, hr, hsc, hsh, hgt, hones], lambda outs: {"res": _peek(R, hr, (T, D))}


def _bf16_bits(a):
    """fp32 -> bf16 bit patterns, nearest even (inf/NaN keep their top half):
    the device's rounding of a GEMM's A (backend_cuda.cu:183-188)."""
    w = np.ascontiguousarray(a, np.float32).view(np.uint32)
    top = (w >> np.uint32(16)).astype(np.uint32)
    r = (w + np.uint32(0x7FFF) + (top & np.uint32(1))) >> np.uint32(16)
    special = (w & np.uint32(0x7F800000)) == np.uint32(0x7F800000)
    return np.where(special, top, r).astype(np.uint16)


def _bf16_to_f32(b):
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)


class RmsModBf16(Workload):
    """The Z-Image block's norm before the projections, as the bf16 A of the GEMMs."""
    name, kernel = "rms_norm_modulate_bf16", "k_rms_mod_bf16"
    desc = ("Z-Image block: y16 = bf16(rms_norm(x) * w * (1 + scale)) (zimage.cpp:115-116, the GEMMs' bf16 A); "
            "x [4096,3840], w, scale [3840]; eps 1e-5")
    algo_bytes = T * D * 4 + T * D * 2 + 2 * D * 4
    inputs = (("x", (T, D), 0.0, 1.0, 21), ("w", (D,), 1.0, 0.1, 22), ("sc", (D,), 1.0, 0.2, 23))
    results = {"y16": ("rel", 1e-2)}  # bf16 output: half an ulp of bf16 is 2^-9 relative

    def make(self, be, i):
        d = super().make(be, i)
        d["y16"] = be.array(np.zeros(T * D, np.uint16))
        return d

    def step(self, be, s):
        be.rms_norm_modulate_bf16(s["x"], s["y16"], T, D, s["w"], s["sc"], 1e-5)

    def gpu_results(self, be, s):
        return {"y16": _bf16_to_f32(s["y16"].download()).reshape(T, D)}

    def cpu(self, R, h):
        hx, hw, hsc = R.new((T, D), h["x"]), R.new((D,), h["w"]), R.new((D,), h["sc"])

        def run():
            y = R._ptr(R.lib.ref_rms_norm(hx, hw, 1e-5))
            R._chk(R.lib.ref_mul_rows_(y, hsc))
            return [y]

        # the reference's device path rounds the GEMM's A to bf16 (backend_cuda.cu:183-188)
        return run, [hx, hw, hsc], lambda outs: {"y16": _bf16_to_f32(_bf16_bits(_peek(R, outs[0], (T, D))))}


class RmsGatedAdd(Workload):
    """The Z-Image block's norm + gated residual after to_out and w2."""
    name, kernel = "rms_norm_gated_add", "k_rms_gated_add"
    desc = ("Z-Image block: x += gate * rms_norm(a) * w (zimage.cpp:124-127); x, a [4096,3840], w, gate [3840]; "
            "eps 1e-5")
    algo_bytes = 3 * T * D * 4 + 2 * D * 4
    inputs = (("x", (T, D), 0.0, 1.0, 24), ("a", (T, D), 0.0, 3.0, 25), ("w", (D,), 1.0, 0.1, 26),
              ("g", (D,), 0.0, 0.5, 27))
    results = {"x": ("rel", 1e-4)}

    def step(self, be, s):
        be.rms_norm_gated_add(s["x"], s["a"], T, D, s["w"], s["g"], 1e-5)

    def cpu(self, R, h):
        hx, ha, hw, hg = R.new((T, D), h["x"]), R.new((T, D), h["a"]), R.new((D,), h["w"]), R.new((D,), h["g"])

        def run():
            y = R._ptr(R.lib.ref_rms_norm(ha, hw, 1e-5))
            R._chk(R.lib.ref_add_rows_scaled_(hx, y, hg))
            return [y]

        return run, [hx, ha, hw, hg], lambda outs: {"x": _peek(R, hx, (T, D))}


class RmsGatedAddMod(Workload):
    """The Z-Image block's residual add + RMSNorm + modulate: one sublayer's
    norm + gated residual and the next sublayer's bf16 input, x read once."""
    name, kernel = "rms_norm_gated_add_modulate_bf16", "k_rms_gated_add_mod"
    desc = ("Z-Image block: x += gate * rms_norm(a) * w1, then y16 = bf16(rms_norm(x) * w2 * (1 + scale)) "
            "(zimage.cpp:124-129); x, a [4096,3840], w1, gate, w2, scale [3840]; eps 1e-5")
    algo_bytes = 3 * T * D * 4 + T * D * 2 + 4 * D * 4
    inputs = (("x", (T, D), 0.0, 1.0, 24), ("a", (T, D), 0.0, 3.0, 25), ("w", (D,), 1.0, 0.1, 26),
              ("g", (D,), 0.0, 0.5, 27), ("w2", (D,), 1.0, 0.1, 22), ("sc", (D,), 1.0, 0.2, 23))
    results = {"x": ("rel", 1e-4), "y16": ("rel", 1e-2)}

    def make(self, be, i):
        d = super().make(be, i)
        d["y16"] = be.array(np.zeros(T * D, np.uint16))
        return d

    def step(self, be, s):
        be.rms_norm_gated_add_modulate_bf16(s["x"], s["a"], s["y16"], T, D, s["w"], s["g"], s["w2"], s["sc"], 1e-5)

    def gpu_results(self, be, s):
        return {"x": s["x"].download().reshape(T, D), "y16": _bf16_to_f32(s["y16"].download()).reshape(T, D)}

    def cpu(self, R, h):
        hx, ha = R.new((T, D), h["x"]), R.new((T, D), h["a"])
        hw, hg, hw2, hsc = (R.new((D,), h[k]) for k in ("w", "g", "w2", "sc"))

        def run():
            y = R._ptr(R.lib.ref_rms_norm(ha, hw, 1e-5))
            R._chk(R.lib.ref_add_rows_scaled_(hx, y, hg))
            z = R._ptr(R.lib.ref_rms_norm(hx, hw2, 1e-5))
            R._chk(R.lib.ref_mul_rows_(z, hsc))
            return [y, z]

        return run, [hx, ha, hw, hg, hw2, hsc], lambda outs: {
            "x": _peek(R, hx, (T, D)), "y16": _bf16_to_f32(_bf16_bits(_peek(R, outs[1], (T, D))))}


class Softmax(Workload):
    config_line = True  # a BASELINE config: the reference CPU path is timed beside it
    name, kernel = "softmax_rows", "k_softmax"
    desc = "config 5b: in-place row softmax of scores [30,4096,4096] ~N(0,3), scale 1/sqrt(128), non-causal"
    algo_bytes = 2 * 30 * T * T * 4
    inputs = (("x", (30 * T, T), 0.0, 3.0, 28),)
    results = {"x": ("softmax", 1e-4)}

    def step(self, be, s):
        be.softmax_rows(s["x"], 30 * T, T, 1.0 / math.sqrt(128.0), False)

    def cpu(self, R, h):
        hx = R.new((30 * T, T), h["x"])

        def run():
            R._chk(R.lib.ref_softmax_rows_(hx, 30 * T, T, 1.0 / math.sqrt(128.0), 0))
            return []

        return run, [hx], lambda outs: {"x": _peek(R, hx, (30 * T, T))}


class Layout(Workload):
    """Layout ops of the tensor library (tensor.cpp:931-1099) at the shapes
    their callers use: bit-exact copies, HBM-bound at (read + write) bytes."""

    SPECS = {
        # name: (description, input shapes, output shape, kernel)
        "upsample_nearest2x": ("VAE decoder upsample (vae.cpp:46): x [1,512,256,256] -> [1,512,512,512]",
                               [(1, 512, 256, 256)], (1, 512, 512, 512), "k_upsample2x_vec"),
        "nchw_to_nlc": ("VAE attention input (modules.cpp:136): [1,512,128,128] -> [1,16384,512]",
                        [(1, 512, 128, 128)], (1, 16384, 512), "k_transpose_vec"),
        "nlc_to_nchw": ("VAE attention output (modules.cpp:138): [1,16384,512] -> [1,512,128,128]",
                        [(1, 16384, 512)], (1, 512, 128, 128), "k_transpose_vec"),
        "concat_channels": ("SD 1.5 UNet skip concat (unet.cpp:113): [2,640,64,64] ++ [2,320,64,64]",
                            [(2, 640, 64, 64), (2, 320, 64, 64)], (2, 960, 64, 64), "k_concat_vec"),
        "patchify2d": ("Z-Image latent to tokens (zimage.cpp:165): [1,16,128,128], p 2 -> [4096,64]",
                       [(1, 16, 128, 128)], (4096, 64), "k_patchify"),
    }
    results = {"y": ("abs", 0.0)}

    def __init__(self, name):
        self.name = name
        self.desc, self.ins, self.out, self.kernel = self.SPECS[name]
        n_in = sum(int(np.prod(s)) for s in self.ins)
        self.algo_bytes = 4 * (n_in + int(np.prod(self.out)))
        self.inputs = tuple((f"x{k}", sh, 0.0, 1.0, 30 + k) for k, sh in enumerate(self.ins))
        self.outputs = (("y", self.out),)

    def step(self, be, s):
        a, y = s["x0"], s["y"]
        if self.name == "upsample_nearest2x":
            N, Cc, H, W = self.ins[0]
            be.upsample_nearest2x(a, y, N * Cc, H, W)
        elif self.name == "nchw_to_nlc":
            N, Cc, H, W = self.ins[0]
            be.nchw_to_nlc(a, y, N, Cc, H * W)
        elif self.name == "nlc_to_nchw":
            N, HW, Cc = self.ins[0]
            be.nlc_to_nchw(a, y, N, Cc, HW)
        elif self.name == "concat_channels":
            (N, Ca, H, W), (_, Cb, _, _) = self.ins
            be.concat_channels(a, s["x1"], y, N, Ca, Cb, H * W)
        else:
            _, Cc, H, W = self.ins[0]
            be.patchify(a, y, Cc, H, W, 2)

    def cpu(self, R, h):
        hs = [R.new(sh, h[f"x{k}"]) for k, sh in enumerate(self.ins)]
        L = R.lib
        fn = {"upsample_nearest2x": lambda: L.ref_upsample_nearest2x(hs[0]),
              "nchw_to_nlc": lambda: L.ref_nchw_to_nlc(hs[0]),
              "nlc_to_nchw": lambda: L.ref_nlc_to_nchw(hs[0], 128, 128),
              "concat_channels": lambda: L.ref_concat_channels(hs[0], hs[1]),
              "patchify2d": lambda: L.ref_patchify2d(hs[0], 2)}[self.name]
        return (lambda: [R._ptr(fn())]), hs, lambda outs: {"y": _peek(R, outs[0], self.out)}


def _bf16_weights(shape, seed, std):
    """Synthetic bf16 weights (uint16 bit patterns): seeded normals rounded to
    nearest even."""
    w = (np.random.default_rng(seed).standard_normal(shape, dtype=np.float32) * np.float32(std))
    return _bf16_bits(w)


class Linear(Workload):
    """The linear layer with bf16 weights on the MFMA units (backend_cuda.h:42)
    at the Z-Image DiT shapes, 4096 image tokens: an attention projection
    [4096,3840] x [3840,3840]^T + bias, and the FFN front half
    swiglu(x w1^T, x w3^T) with w1, w3 [10240,3840] -- fused, and unfused as the
    reference runs it (two GEMMs, then swiglu). Rated in TFLOP/s against the
    dense bf16 MFMA peak. Parity: the reference's CPU linear on the same
    weights with x rounded to bf16 as its device path rounds it
    (backend_cuda.cu:466-467); then only the fp32 summation order differs."""

    _want = {}  # the swiglu lines share one reference result

    def __init__(self, kind):
        self.name = kind
        self.kernel = "Cijk"  # hipBLASLt's GEMM kernels
        if kind == "linear_bf16":
            self.M, self.N, self.K = T, D, D
            self.flops = 2 * self.M * self.N * self.K
            self.algo_bytes = self.M * self.K * 4 + self.N * self.K * 2 + self.M * self.N * 4 + self.N * 4
            self.desc = "linear, bf16 weights: y = x W^T + b, x [4096,3840] fp32, W [3840,3840] bf16 (Z-Image to_q/k/v/out)"
            self.inputs = (("x", (T, D), 0.0, 1.0, 40), ("b", (D,), 0.0, 0.1, 41))
            self.wseeds = {"w": 42}
        else:
            self.M, self.N, self.K = T, F, D
            self.flops = 2 * 2 * self.M * self.N * self.K
            self.algo_bytes = self.M * self.K * 4 + 2 * self.N * self.K * 2 + self.M * self.N * 4
            self.desc = ("swiglu(x w1^T, x w3^T), x [4096,3840] fp32, w1, w3 [10240,3840] bf16 (Z-Image FFN, zimage.cpp:130)" +
                         (": the reference's sequence (two GEMMs, then swiglu)" if kind.endswith("unfused") else ", one GEMM"))
            self.inputs = (("x", (T, D), 0.0, 1.0, 43),)
            self.wseeds = {"w1": 44, "w3": 45}
        self.outputs = (("y", (self.M, self.N)),)
        self.results = {"y": ("normrel", 1e-5)}
        self.weights = {n: _bf16_weights((self.N, self.K), sd, 0.02) for n, sd in self.wseeds.items()}
        if kind != "linear_bf16":
            self.cpu_time = False  # tens of seconds per step on the host: parity only, no timing

    def make(self, be, i):
        d = super().make(be, i)
        for n, w in self.weights.items():
            d[n] = be.array(w)
        if self.name.endswith("unfused"):
            d["g"], d["u"] = be.empty((self.M, self.N)), be.empty((self.M, self.N))
        return d

    def step(self, be, s):
        M, N, K = self.M, self.N, self.K
        if self.name == "linear_bf16":
            be.gemm_nt_bf16(M, N, K, s["x"], K, s["w"], K, s["y"], N, s["b"])
        elif self.name == "linear_swiglu":
            be.linear_swiglu(s["x"], s["w1"], s["w3"], s["y"], M, K, N)
        else:
            be.gemm_nt_bf16(M, N, K, s["x"], K, s["w1"], K, s["g"], N)
            be.gemm_nt_bf16(M, N, K, s["x"], K, s["w3"], K, s["u"], N)
            be.swiglu(s["g"], s["u"], s["y"], M * N)

    def _ref_weight(self, R, n):
        hw = R.new((self.N, self.K), _bf16_to_f32(self.weights[n]))
        R._chk(R.lib.ref_tensor_to_bf16(hw))  # exact: the values are bf16 already
        return hw

    def cpu(self, R, h):
        hx = R.new((self.M, self.K), _bf16_to_f32(_bf16_bits(h["x"])))
        hws = {n: self._ref_weight(R, n) for n in self.weights}
        if self.name == "linear_bf16":
            hb = R.new((self.N,), h["b"])
            return ((lambda: [R._ptr(R.lib.ref_linear(hx, hws["w"], hb))]), [hx, hb] + list(hws.values()),
                    lambda outs: {"y": _peek(R, outs[0], (self.M, self.N))})

        def run():
            g = R._ptr(R.lib.ref_linear(hx, hws["w1"], None))
            u = R._ptr(R.lib.ref_linear(hx, hws["w3"], None))
            y = R._ptr(R.lib.ref_swiglu(g, u))
            R.free(g, u)
            return [y]

        return run, [hx] + list(hws.values()), lambda outs: {"y": _peek(R, outs[0], (self.M, self.N))}

    def reference_results(self, R, h):
        """The swiglu lines have the same inputs: one reference computation."""
        key = "swiglu" if self.name != "linear_bf16" else self.name
        if key not in Linear._want:
            run, handles, collect = self.cpu(R, h)
            outs = run()
            Linear._want[key] = collect(outs)
            R.free(*outs, *handles)
        return Linear._want[key]


class Attention(Workload):
    """Multi-head attention fused on the MFMA units (backend_cuda.h:57-59;
    tensor.cpp:776-810) at the Z-Image DiT layer: q, k, v [1,4096,30*128]
    fp32, no mask (zimage.cpp:121). Rated in TFLOP/s by the reference's own
    formula 4 S^2 d H (test_ops.cpp:352); the MFMA units execute three bf16
    products per fp32 product (split operands), which pct_mfma_peak counts.
    The CPU baseline times the reference's attention on one of the 30 heads
    and scales it by 30 (heads are independent, tensor.cpp:793-808); parity
    runs the reference on all 30 heads."""

    name, kernel = "attention", "k_attn_fwd"
    S, H, d = T, 30, 128
    flops = 4 * T * T * 128 * 30
    mfma_mult = 3
    algo_bytes = 4 * T * 30 * 128 * 4
    cpu_scale = 30
    desc = "attention, q k v [1,4096,30x128] fp32, softmax(q k^T / sqrt(128)) v per head (Z-Image DiT layer)"
    inputs = (("q", (1, T, 30 * 128), 0.0, 1.0, 50), ("k", (1, T, 30 * 128), 0.0, 1.0, 51),
              ("v", (1, T, 30 * 128), 0.0, 1.0, 52))
    outputs = (("o", (1, T, 30 * 128)),)
    results = {"o": ("abs", 1e-4)}  # the reference's attention bar (test_ops.cpp:442-451)

    def step(self, be, s):
        be.attention(s["q"], s["k"], s["v"], s["o"], 1, self.S, self.S, self.H, self.H, self.d, False)

    def _head(self, h, n, i):
        return np.ascontiguousarray(h[n].reshape(T, 30, 128)[:, i, :]).reshape(1, T, 128)

    def cpu(self, R, h):
        shp = (1, self.S, self.d)  # one head timed
        hq, hk, hv = (R.new(shp, self._head(h, n, 0)) for n in ("q", "k", "v"))
        return (lambda: [R._ptr(R.lib.ref_attention(hq, hk, hv, 1, 0, 1))]), [hq, hk, hv], None

    _ref_cache = {}  # the attention lines share their inputs (same seeds): one reference run

    def reference_results(self, R, h):
        key = tuple(sorted(self.seeds().items()))
        if key in Attention._ref_cache:
            return Attention._ref_cache[key]
        o = np.empty((T, 30, 128), np.float32)
        for i in range(30):
            hs = [R.new((1, T, 128), self._head(h, n, i)) for n in ("q", "k", "v")]
            ho = R._ptr(R.lib.ref_attention(*hs, 1, 0, 1))
            o[:, i, :] = _peek(R, ho, (T, 128))
            R.free(ho, *hs)
        Attention._ref_cache[key] = {"o": o.reshape(1, T, 30 * 128)}
        return Attention._ref_cache[key]


class AttentionFp16(Attention):
    """The opt-in reduced-precision attention (sdh_attention_fp16, no
    counterpart in the reference) on the same layer and inputs: every product
    formed once from block-scaled fp16 operands (one MFMA per product, half the
    packed bytes). Parity against the reference's fp32 attention at abs 1e-2,
    the error fp16 operands give on unit-variance inputs (the kernel's own
    rounding bound is checked against a rounded-operand oracle in
    tests/test_gpu_attention_fp16.py). Not timed on the CPU: the reference has
    no such mode."""

    name = "attention_fp16"
    mfma_mult = 1
    cpu_time = False
    desc = "opt-in fp16-operand attention (no reference counterpart), q k v [1,4096,30x128], same inputs as attention"
    results = {"o": ("abs", 1e-2)}

    def step(self, be, s):
        be.attention_fp16(s["q"], s["k"], s["v"], s["o"], 1, self.S, self.S, self.H, self.H, self.d, False)


class AttentionVAE(Workload):
    """The VAE decoder's mid-block attention (VAEAttention, modules.cpp:133-141:
    one head over the 512 channels, tokens = the latent's pixels) at the FLUX
    VAE's 1024x1024 decode: q k v [1, 16384, 512] fp32. Head dimensions above
    128 on long sequences take the score-matrix route on the fp32 library GEMM
    (score blocks, the row softmax, a GEMM against v^T), so the rate is quoted
    against the 157.3 TFLOP/s fp32 MFMA peak. Parity: the reference's
    attention on the same arrays, abs 1e-4."""

    name, kernel = "attention_vae", "Cijk"
    S, d = 16384, 512
    flops = 4 * 16384 * 16384 * 512
    mfma_peak = (157.3, "157.3 TF fp32")
    algo_bytes = 4 * 16384 * 512 * 4
    cpu_time = False
    desc = "VAE mid-block attention, q k v [1,16384,512] fp32, one head (FLUX VAE decode at 1024x1024)"
    inputs = (("q", (1, 16384, 512), 0.0, 1.0, 54), ("k", (1, 16384, 512), 0.0, 1.0, 55),
              ("v", (1, 16384, 512), 0.0, 1.0, 56))
    outputs = (("o", (1, 16384, 512)),)
    results = {"o": ("abs", 1e-4)}

    def step(self, be, s):
        be.attention(s["q"], s["k"], s["v"], s["o"], 1, self.S, self.S, 1, 1, self.d, False)

    def cpu(self, R, h):
        hs = [R.new((1, self.S, self.d), h[n]) for n in ("q", "k", "v")]
        return (lambda: [R._ptr(R.lib.ref_attention(*hs, 1, 0, 1))]), hs, \
            lambda outs: {"o": _peek(R, outs[0], (1, self.S, self.d))}


class ZImageStep(Workload):
    """One denoising step of the Z-Image transformer (ZImageTransformer::forward,
    zimage.cpp:138-228) on the device at 1024x1024: latent [1,16,128,128] ->
    4096 image tokens, 128 text tokens of 2560 features, 2 noise and 2 context
    refiner blocks, 30 main blocks of dim 3840 (30 heads x 128, FFN 10240),
    weights seeded random with the checkpoint's shapes (BF16 from 2^20
    elements, as pipeline.cpp:113 loads them). Rated in TFLOP/s over the
    linear layers and attention (2 flop per multiply-add). Its parity against
    the reference's own forward runs in tests/test_gpu_zimage.py on a model of
    the same layout and fewer layers (the full model's CPU forward takes
    minutes)."""

    name, kernel = "zimage_step_1024", "k_gemm_dl"
    H = W = 128
    L, cap_dim = 128, 2560
    D, F, heads, layers = 3840, 10240, 30, 30
    algo_bytes = 0
    desc = "Z-Image DiT step at 1024x1024 (4096 image + 128 text tokens, 30+4 blocks, dim 3840), random BF16 weights"

    @property
    def flops(self):
        D, F = self.D, self.F

        def block(S):
            return 2 * S * (4 * D * D + 3 * D * F) + 4 * S * S * D

        n_img, n_cap = (self.H // 2) * (self.W // 2), self.L
        return (2 * block(n_img) + 2 * block(n_cap) + self.layers * block(n_img + n_cap) +
                2 * n_img * 64 * D * 2 + 2 * n_cap * self.cap_dim * D)

    def measure(self, steps, warmup):
        import sdhip

        m = sdhip.ZImage.random(dim=self.D, heads=self.heads, ffn=self.F, layers=self.layers, seed=7)
        try:
            ms = m.time(self.H, self.W, self.L, self.cap_dim, steps, warmup)
            params = m.params()
        finally:
            m.close()
        return dict(event_ms=ms, wall_ms=ms, nsets=1, footprint=0, params=params)


class ZImageStepFp16Attention(ZImageStep):
    """The same step with the opt-in fp16-operand attention
    (ZImageTransformer::set_fp16_attention, no counterpart in the reference);
    its forward stays within the DiT's 2e-2 of the reference's CPU forward
    (tests/test_gpu_attention_fp16.py, measured 2.4e-3 with BF16 weights, as
    with the default attention)."""

    name = "zimage_step_1024_fp16_attention"
    desc = "Z-Image DiT step at 1024x1024 as zimage_step_1024, attention from fp16 operands (opt-in)"

    def measure(self, steps, warmup):
        import sdhip

        m = sdhip.ZImage.random(dim=self.D, heads=self.heads, ffn=self.F, layers=self.layers, seed=7)
        try:
            m.set_fp16_attention(True)
            ms = m.time(self.H, self.W, self.L, self.cap_dim, steps, warmup)
            params = m.params()
        finally:
            m.close()
        return dict(event_ms=ms, wall_ms=ms, nsets=1, footprint=0, params=params)


class CopyCalibration(Workload):
    """Not a BASELINE config: an in-place x *= 1 stream over [4096,10240]
    (one read + one write of 168 MB, non-temporal loads and stores), the
    plain-copy reference for what HBM streaming reaches on this box and the
    calibration for the traffic counters."""

    name, kernel = "copy_calibration", "k_unary"
    desc = "calibration (not a config): in-place x *= 1.0 over [4096,10240] fp32, 1 read + 1 write"
    algo_bytes = 2 * T * F * 4
    inputs = (("x", (T, F), 0.0, 1.0, 60),)
    results = {"x": ("abs", 0.0)}

    def step(self, be, s):
        be.scale(s["x"], 1.0, T * F)

    def cpu(self, R, h):
        hx = R.new((T, F), h["x"])
        return (lambda: (R._chk(R.lib.ref_scale_(hx, 1.0)), [])[1]), [hx], lambda outs: {"x": _peek(R, hx, (T, F))}


class BlitCalibration(Workload):
    """Not a BASELINE config: the HIP runtime's device-to-device copy
    (sdh_copy -> hipMemcpyAsync) of [4096,10240] fp32, a second calibration
    kernel of known traffic whose loads and stores are ordinary (cached)
    ones, to check the counters' scale on kernels that do not stream
    non-temporally."""

    name, kernel = "blit_calibration", "copyBuffer"
    desc = "calibration (not a config): hipMemcpyAsync device-to-device of [4096,10240] fp32, 1 read + 1 write"
    algo_bytes = 2 * T * F * 4
    inputs = (("x", (T, F), 0.0, 1.0, 61),)
    outputs = (("y", (T, F)),)
    results = {"y": ("abs", 0.0)}

    def step(self, be, s):
        be.copy(s["y"], s["x"], T * F * 4)

    def cpu(self, R, h):
        hx = R.new((T, F), h["x"])
        return (lambda: []), [hx], lambda outs: {"y": _peek(R, hx, (T, F))}


def all_workloads():
    return [
        CopyCalibration(),
        BlitCalibration(),
        AddRmsNorm(),
        SwiGLU(),
        RopeQK(),
        RopeQKAxes(),
        GNSiLU("4a", (1, 512, 128, 128), 1e-6, "4a (FLUX VAE)"),
        GNSiLU("4b", (1, 128, 1024, 1024), 1e-6, "4b (FLUX VAE norm_out)"),
        GNSiLU("4c", (2, 320, 64, 64), 1e-5, "4c (SD 1.5, reported only)"),
        GNSiLU("4d", (2, 1280, 8, 8), 1e-5, "4d (SD 1.5, reported only)"),
        LNModGate(),
        Softmax(),
        QKNormRope(),
        QKNormRope(unfused=True),
        RmsModBf16(),
        RmsGatedAdd(),
        RmsGatedAddMod(),
    ] + [Layout(n) for n in Layout.SPECS] + [Linear(k) for k in ("linear_bf16", "linear_swiglu", "linear_swiglu_unfused")] + [
        Attention(), AttentionFp16(), AttentionVAE(), ZImageStep(), ZImageStepFp16Attention()]


# ------------------------------------------------------------------ GPU timing
def measure_gpu(be, w, steps, warmup, check=False, min_warm_s=0.0, min_timed_s=0.0):
    """Times `steps` steps over rotating buffer sets, after `warmup` untimed
    steps (continued in batches until `min_warm_s` seconds have passed; with
    `min_timed_s`, more steps when `steps` would take less than that at the
    warm-up's pace). With
    check, set 0's inputs are downloaded before the timed steps, and
    afterwards, outside the timed region, set 0 is reloaded from them, stepped
    once and its results returned for the parity check."""
    first = w.make(be, 0)
    host = w.host_inputs(first) if check and w.results else None
    footprint = sum(a.nbytes for a in first.values())
    nsets = max(2, min(MAX_SETS, math.ceil(MIN_ROTATION_BYTES / max(footprint, 1))))
    sets = [first] + [w.make(be, i) for i in range(1, nsets)]
    be.synchronize()
    t_warm = time.perf_counter()
    for i in range(warmup):
        w.step(be, sets[i % nsets])
    be.synchronize()
    i = warmup
    while time.perf_counter() - t_warm < min_warm_s:
        for _ in range(OP_WARM_BATCH):
            w.step(be, sets[i % nsets])
            i += 1
        be.synchronize()
    if min_timed_s > 0 and i > 0:
        per = (time.perf_counter() - t_warm) / i
        steps = max(steps, min(100 * steps, math.ceil(min_timed_s / max(per, 1e-9))))
    t0 = time.perf_counter()
    be.timer_record(0)
    for i in range(steps):
        w.step(be, sets[i % nsets])
    be.timer_record(1)
    be.synchronize()
    wall = time.perf_counter() - t0
    ev_ms = be.timer_elapsed(0, 1)
    graph_ms = None
    if ev_ms / steps < GRAPH_ALSO_MS:
        # launch-bound: the host's ctypes loop, not the GPU, sets the pace of
        # the loop above; the same steps captured into one graph run back to
        # back on the device (sdh_capture_begin), which is the GPU's time
        gsteps = min(steps, GRAPH_MAX_STEPS)
        be.capture_begin()
        try:
            for i in range(gsteps):
                w.step(be, sets[i % nsets])
        finally:
            g = be.capture_end()
        try:
            be.graph_launch(g)  # warm-up replay
            be.synchronize()
            be.timer_record(0)
            be.graph_launch(g)
            be.timer_record(1)
            be.synchronize()
            graph_ms = be.timer_elapsed(0, 1) * steps / gsteps  # per `steps` steps, as ev_ms
        finally:
            be.graph_destroy(g)
    got = None
    if host is not None and w.results:
        w.reload(be, sets[0], host)
        w.step(be, sets[0])
        got = w.gpu_results(be, sets[0])
    for st in sets:
        for a in st.values():
            a.free()
    out = dict(nsets=nsets, footprint=footprint * nsets, wall_ms=wall * 1e3 / steps, event_ms=ev_ms / steps,
               got=got, host=host, steps=steps)
    if graph_ms is not None:
        if ev_ms / steps < GRAPH_BELOW_MS:
            out.update(host_paced_ms=ev_ms / steps, event_ms=graph_ms / steps, graph=True, graph_steps=gsteps)
        else:
            out.update(graph_ms=graph_ms / steps, graph_steps=gsteps)
    return out


# ------------------------------------------------------------------ CPU leg: reference timing and parity
REF_V3 = os.path.join(ROOT, "oracle", "_ref", "libsdref.so")
REF_V4 = os.path.join(ROOT, "oracle", "_ref", "libsdref_v4.so")
REF_FLAGS = "g++ -std=c++17 -O3 {march} -pthread -fPIC (the reference Makefile's flags; -march=native there)"


def _host_has_avx512():
    try:
        flags = next(l for l in open("/proc/cpuinfo") if l.startswith("flags")).split()
    except Exception:
        return False
    return all(f in flags for f in ("avx512f", "avx512bw", "avx512cd", "avx512dq", "avx512vl"))


def reference_library():
    """The compiled reference tensor library (oracle/_ref) for the CPU leg:
    the x86-64-v4 (AVX-512) build where this host has AVX-512, else the
    x86-64-v3 (AVX2 + FMA) build the parity tests pin. None if neither is
    built (the reference tree was absent when build() ran)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from oracle import Reference

    if os.path.exists(REF_V4) and _host_has_avx512():
        return Reference(REF_V4), REF_FLAGS.format(march="-march=x86-64-v4")
    if os.path.exists(REF_V3):
        return Reference(REF_V3), REF_FLAGS.format(march="-march=x86-64-v3")
    return None, None


def cpu_threads():
    """Threads for the reference's pool: this process's CPU share -- the
    OMP_NUM_THREADS the GPU box sets (its CPUs per GPU), else the CPUs this
    process may run on."""
    try:
        avail = len(os.sched_getaffinity(0))
    except Exception:
        avail = os.cpu_count() or 1
    share = os.environ.get("OMP_NUM_THREADS", "")
    n = int(share) if share.isdigit() and int(share) > 0 else avail
    return max(1, min(n, avail)), avail


def run_reference(R, w, host, reps):
    """The reference's CPU composition of one step on the host inputs: its
    results after exactly one run (for parity) and, when reps > 0, the
    median time of reps further runs after that one (output allocation
    included, as the op is called)."""
    if hasattr(w, "reference_results"):
        want = w.reference_results(R, host)
        if reps <= 0 or getattr(w, "cpu_time", True) is False:
            return dict(want=want, ms=None)
        made = w.cpu(R, host)
        run, handles, _ = made
        collect = None
    else:
        made = w.cpu(R, host)
        if made is None:
            return None
        run, handles, collect = made
        want = None
    times = []
    for i in range((reps if getattr(w, "cpu_time", True) else 0) + 1):
        t0 = time.perf_counter()
        outs = run()
        dt = time.perf_counter() - t0
        if i == 0 and collect is not None:
            want = collect(outs)
        R.free(*outs)
        if i:
            times.append(dt)
    R.free(*handles)
    ms = statistics.median(times) * 1e3 * getattr(w, "cpu_scale", 1) if times else None
    return dict(want=want, ms=ms)


def parity(got, want, results):
    """max-abs error and the tolerance metric of each result, GPU against the
    reference on the same inputs."""
    per, worst = {}, None
    for n, (kind, bound) in results.items():
        g = np.asarray(got[n], np.float64).reshape(-1)
        r = np.asarray(want[n], np.float64).reshape(-1)
        d = np.abs(g - r)
        mx = float(np.max(d)) if d.size else 0.0
        if kind == "softmax":
            zeros = r == 0
            metric = float("inf") if np.any(g[zeros] != 0) else float(np.max(d / np.maximum(np.abs(r), 1e-30)))
        elif kind == "normrel":
            metric = mx / max(float(np.max(np.abs(r))), 1e-30)
        elif kind == "rel":
            metric = float(np.max(d / np.maximum(np.abs(r), 1.0)))
        else:  # abs
            metric = mx
        e = dict(max_abs_err=mx, rel_err=float(np.max(d / np.maximum(np.abs(r), 1.0))) if kind != "softmax" else metric,
                 metric=kind, bound=bound, value=metric, within_tolerance=bool(metric <= bound),
                 bitexact=bool(mx == 0.0))
        per[n] = e
        if worst is None or e["max_abs_err"] > worst["max_abs_err"]:
            worst = e
    return per, worst


# ------------------------------------------------------------------ traffic (rocprof pmc)
def read_traffic(name):
    """HBM bytes per launch from profiles/hbm_traffic.txt (rocprofv3 --pmc
    runs of the L2-to-memory request counters by size; see rocprof_summary)."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        m = re.match(r"^\s*" + re.escape(name) + r"\s+.*traffic_bytes=(\d+)", line)
        if m:
            return int(m.group(1))
    return None


# ------------------------------------------------------------------ rocprofv3 summaries
KERNEL_OF = {  # kernel (template) name -> workload whose step launches it
    "k_unary<4>": "copy_calibration", "k_add_rms": "add_rms_norm", "k_swiglu": "swiglu",
    "k_rope_il_reg": "rope_qk", "k_rope_il_axes": "rope_qk_axes", "k_ln_mod_gate": "ln_modulate_gate", "k_softmax_block": "softmax_rows",
    "k_upsample2x_vec": "upsample_nearest2x", "k_concat_vec": "concat_channels", "k_patchify": "patchify2d",
    "k_qknorm_rope_il": "qknorm_rope", "k_attn_fwd<128, false, false, true>": "attention",
    "k_attn_fwd<128, false, false, false>": "attention_fp16", "k_rms_mod_bf16": "rms_norm_modulate_bf16",
    "k_rms_gated_add_mod": "rms_norm_gated_add_modulate_bf16", "k_rms_gated_add": "rms_norm_gated_add",
    "copyBuffer": "blit_calibration",
}


# Resident workgroups per CU of the gfx950 build of each resident GroupNorm
# kernel (its VGPR count at 1024 threads; the library plans with the
# vector-poll variants): k_gn_resident V=4 (60-62 VGPRs) 2, V=8 (76-89) 1,
# V=16 (112) 1; k_gn_resident_pipe V=4 (82-86) 1, V=8 (114-126) 1.
GN_RESIDENT_OCC = {(False, 4): 2, (False, 8): 1, (False, 16): 1, (True, 4): 1, (True, 8): 1}


def gn_split_chunk(nseg, L):
    """run_gn's split_chunk: the largest of 8192, 4096 and 2048 floats that
    gives 768 workgroups per pass, else 2048."""
    for c in (8192, 4096):
        if nseg * -(-L // c) >= 768:
            return c
    return 2048


def gn_dispatches(shape, groups=32, cus=256):
    """(kernel prefix, grid work-items) of the launches that carry a GroupNorm
    workload's HBM traffic, following run_gn's choice of schedule: one
    k_gn_single launch for segments up to 24576 floats; else, for segments
    cut into whole 4096-float chunks that each lie in one channel (at most
    64 per segment), k_gn_pipe launches of two workgroups per chunk (the
    first launch, of at most 2^17 chunks); else, for x of at least 64 MB,
    the resident plan of run_gn_resident (one launch of
    k_gn_resident or k_gn_resident_pipe); else k_gn_partial and k_gn_apply
    over chunks of gn_split_chunk floats (k_gn_finalize moves a few KB and
    is left out)."""
    N, Cc = shape[0], shape[1]
    HW = int(np.prod(shape[2:]))
    L, nseg = Cc // groups * HW, N * groups
    if L <= 24576:
        n4 = L // 4
        tpb = 256 if n4 <= 2048 else 1024
        return [("k_gn_single", nseg * tpb)]
    if HW % 4096 == 0 and L // 4096 <= 64:
        cps = L // 4096
        return [("k_gn_pipe", 2 * min(nseg, (1 << 17) // cps) * cps * 256)]
    if nseg * L * 4 >= 64 << 20:
        best = {}
        for pipe in (False, True):
            for V in (4, 8, 16):
                share = 4096 * V
                P = -(-L // share)
                if (pipe, V) not in GN_RESIDENT_OCC or P > (128 if pipe else 64) or (V == 16 and HW % share):
                    continue
                T = GN_RESIDENT_OCC[(pipe, V)] * cus // P
                if T == 0:
                    continue
                rounds = -(-nseg // T)
                key = "pipe" if pipe else "plain"
                if key not in best or rounds < best[key][0]:
                    best[key] = (rounds, pipe, P, T)
        plan = best.get("pipe") or best.get("plain")
        if plan:
            _, pipe, P, T = plan
            return [("k_gn_resident_pipe<" if pipe else "k_gn_resident<", min(T, nseg) * P * 1024)]
    chunk = gn_split_chunk(nseg, L)
    grid = -(-L // chunk) * (256 if chunk == 8192 else 64) * nseg
    return [("k_gn_partial", grid), ("k_gn_apply", grid)]


def _kernel_key(full_name):
    if "copyBuffer" in full_name:  # the HIP runtime's device-to-device copy kernel
        return "copyBuffer"
    if full_name.startswith("Cijk_"):  # a hipBLASLt GEMM kernel: the library and its macro tile
        t = re.search(r"_MT(\d+x\d+x\d+)_", full_name)
        return "hipBLASLt Cijk MT" + (t.group(1) if t else "?")
    m = re.search(r"(k_\w+)(<[^>]*>)?\(", full_name)
    return (m.group(1) + (m.group(2) or "")) if m else full_name


def rocprof_summary(trace_dir, read_dir=None, write_dir=None):
    """Markdown summary of a `rocprofv3 --kernel-trace --stats --output-format
    csv` run of this script and, optionally, of its two counter runs:
      read_dir:  --pmc TCC_EA0_RDREQ_sum TCC_EA0_RDREQ_128B_sum
                       TCC_EA0_RDREQ_64B_sum TCC_EA0_RDREQ_32B_sum
      write_dir: --pmc TCC_EA0_WRREQ_sum TCC_EA0_WRREQ_64B_sum
    HBM bytes per dispatch come from the L2-to-memory requests by size:
    read = 128 n128 + 64 n64 + 32 n32, write = 64 n64 + 32 (n - n64). No
    calibration factor: the derived FETCH_SIZE of this ROCm counts a 128-byte
    request as 64 bytes (its expression takes 128-byte requests from
    TCC_BUBBLE), which a factor of 2 used to correct. The two copy kernels
    (non-temporal and the runtime's ordinary-load copy) check the method
    against their known traffic."""
    import collections
    import csv
    import glob

    def rows_of(d, suffix):
        files = glob.glob(os.path.join(d, "**", "*" + suffix), recursive=True)
        return [r for f in files for r in csv.DictReader(open(f))]

    trace = rows_of(trace_dir, "_kernel_trace.csv")
    dur = collections.defaultdict(list)
    for r in trace:
        k = (_kernel_key(r["Kernel_Name"]), int(r["Grid_Size_X"]) * int(r.get("Grid_Size_Y", 1) or 1))
        dur[k].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0)
    out = ["| kernel | grid (work-items) | dispatches | avg us | median us | min us |", "|---|---|---|---|---|---|"]
    for (k, g), v in sorted(dur.items(), key=lambda kv: -sum(kv[1])):
        if k.startswith("k_fill_normal") or k.startswith("k_zero"):
            continue
        v = sorted(v)
        out.append(f"| `{k}` | {g} | {len(v)} | {statistics.mean(v):.2f} | {v[len(v) // 2]:.2f} | {v[0]:.2f} |")
    text = "\n".join(out) + "\n"
    traffic_lines = []
    if read_dir and write_dir:
        def counters(d):
            per = collections.defaultdict(lambda: collections.defaultdict(float))
            for r in rows_of(d, "_counter_collection.csv"):
                key = (_kernel_key(r["Kernel_Name"]), int(r["Grid_Size"]), r.get("Dispatch_Id", r.get("Correlation_Id")))
                per[key][r["Counter_Name"]] += float(r["Counter_Value"])
            agg = collections.defaultdict(list)
            for (kn, g, _), c in per.items():
                agg[(kn, g)].append(c)
            return agg

        rd, wr = counters(read_dir), counters(write_dir)

        def med(cs, name):
            return statistics.median(c.get(name, 0.0) for c in cs)

        def read_bytes(cs):
            n128, n64, n32 = med(cs, "TCC_EA0_RDREQ_128B_sum"), med(cs, "TCC_EA0_RDREQ_64B_sum"), med(cs, "TCC_EA0_RDREQ_32B_sum")
            return 128 * n128 + 64 * n64 + 32 * n32, med(cs, "TCC_EA0_RDREQ_sum") - (n128 + n64 + n32)

        def write_bytes(cs):
            n, n64 = med(cs, "TCC_EA0_WRREQ_sum"), med(cs, "TCC_EA0_WRREQ_64B_sum")
            return 64 * n64 + 32 * (n - n64)

        text += ("\nHBM traffic per dispatch from the L2/EA request counters by size (read = 128 n128 + 64 n64 + "
                 "32 n32; write = 64 n64 + 32 n32); no calibration factor.\n\n")
        mapped = set()
        text += ("| kernel | grid | read bytes | write bytes | HBM bytes per dispatch | requests of no listed size |\n"
                 "|---|---|---|---|---|---|\n")
        for k in sorted(rd, key=lambda k: -read_bytes(rd[k])[0]):
            if k[0].startswith("k_fill_normal") or k[0].startswith("k_zero"):
                continue
            rb, other = read_bytes(rd[k])
            wb = write_bytes(wr[k]) if k in wr else 0.0
            tb = int(round(rb + wb))
            text += f"| `{k[0]}` | {k[1]} | {rb:,.0f} | {wb:,.0f} | {tb:,} | {other:.0f} |\n"
            wl = next((v for kk, v in KERNEL_OF.items() if k[0].startswith(kk)), None)
            if wl and wl not in mapped:  # rows run largest first: a workload's own launch, not a stray one
                mapped.add(wl)
                traffic_lines.append(f"{wl} kernel={k[0]} grid={k[1]} read_bytes={rb:.0f} write_bytes={wb:.0f} "
                                     f"traffic_bytes={tb}")
        for wl in all_workloads():
            if not isinstance(wl, GNSiLU):
                continue
            ks = [k for pre, g in gn_dispatches(wl.shape) for k in rd if k[0].startswith(pre) and k[1] == g]
            if ks:
                rb = sum(read_bytes(rd[k])[0] for k in ks)
                wb = sum(write_bytes(wr[k]) for k in ks if k in wr)
                names = "+".join(k[0] for k in ks)
                traffic_lines.append(f"{wl.name} kernel={names} grid={ks[0][1]} read_bytes={rb:.0f} write_bytes={wb:.0f} "
                                     f"traffic_bytes={int(round(rb + wb))}")
    return text, traffic_lines


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="swiglu", help="headline workload (default: swiglu = configs[1])")
    ap.add_argument("--only", default=None, help="comma list: measure only these workloads (profiling runs)")
    ap.add_argument("--op-steps", type=int, default=20,
                    help="timed steps per op in the per-op table, at least (ops under 500 us time 10 ms of steps)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-all", action="store_true",
                    help="time the reference CPU path on every line (the BASELINE config lines always are)")
    ap.add_argument("--cpu-reps", type=int, default=5)
    ap.add_argument("--list", action="store_true")
    ap.add_argument("--rocprof-summary", nargs="+", metavar="DIR",
                    help="print a markdown summary of rocprofv3 csv output: TRACE_DIR [READ_DIR WRITE_DIR]")
    args = ap.parse_args()

    if args.rocprof_summary:
        d = args.rocprof_summary
        text, lines = rocprof_summary(d[0], d[1] if len(d) > 2 else None, d[2] if len(d) > 2 else None)
        print(text)
        if lines:
            print("traffic lines (profiles/hbm_traffic.txt format):")
            print("\n".join(lines))
        return 0

    wls = {w.name: w for w in all_workloads()}
    if args.list:
        for w in wls.values():
            print(f"{w.name:24s} {w.algo_bytes:>14,d} B  {w.desc}")
        return 0
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this build measures one GPU only (every op shards by rows with no exchange); "
                                   "run with --gpus 1"}), flush=True)
        return 2
    if args.workload not in wls:
        print(f"unknown workload {args.workload}; --list shows them", file=sys.stderr)
        return 2

    import sdhip

    be = sdhip.Backend()
    head = wls[args.workload]
    names = [n.strip() for n in args.only.split(",")] if args.only else list(wls)
    R, ref_build = (None, None) if args.no_cpu else reference_library()
    threads, avail = cpu_threads()
    if R is not None:
        R.lib.ref_set_threads(threads)

    ops = []
    head_res, head_cpu, head_err = None, None, None
    # every GPU measurement first, back to back, then the CPU legs: a CPU leg
    # between two measurements leaves the GPU idle for seconds, and the next
    # line (the headline too, whose warm-up is exactly --warmup steps) would
    # time the GPU's clocks coming back up
    measured = []
    for n in names:
        w = wls[n]
        steps = args.steps if w is head else args.op_steps
        warm = args.warmup if w is head else 3
        if hasattr(w, "measure"):  # a whole model step, timed by the model library itself
            r = w.measure(max(3, min(steps, 10)), 2)
        else:
            r = measure_gpu(be, w, steps, warm, check=R is not None, min_warm_s=0.0 if w is head else OP_WARM_S,
                            min_timed_s=0.0 if w is head else OP_TIMED_S)
        measured.append((w, r))
        print(f"# gpu {w.name:22s} {r['event_ms'] * 1e3:10.2f} us", file=sys.stderr, flush=True)
    for w, r in measured:
        gbs = w.algo_bytes / (r["event_ms"] * 1e-3) / 1e9
        entry = dict(op=w.name, desc=w.desc, algo_bytes=w.algo_bytes, us_per_op=round(r["event_ms"] * 1e3, 2),
                     GBps=round(gbs, 1), pct_hbm_peak=round(100 * gbs / HBM_PEAK_GBS, 1), rotation_sets=r["nsets"],
                     rotation_MB=round(r["footprint"] / 2**20), traffic_bytes=read_traffic(w.name))
        if r.get("steps") is not None:
            entry["timed_steps"] = r["graph_steps"] if r.get("graph") else r["steps"]
        if r.get("graph"):
            entry.update(timing="device: the steps captured into one graph and replayed (sdh_capture_begin)",
                         us_per_op_host_paced=round(r["host_paced_ms"] * 1e3, 2))
        elif r.get("graph_ms") is not None:
            entry.update(timing="host-paced loop (the GPU is the bound above 10 us per step)",
                         us_per_op_graph=round(r["graph_ms"] * 1e3, 2))
        if w.inputs:
            entry["seeds"] = w.seeds()
        if "params" in r:
            entry.update(params=r["params"], ms_per_step=round(r["event_ms"], 3))
        flops = getattr(w, "flops", None)
        if flops:
            tfs = flops / (r["event_ms"] * 1e-3) / 1e12
            mult = getattr(w, "mfma_mult", 1)  # MFMA products per counted product
            peak, peak_name = getattr(w, "mfma_peak", (MFMA_BF16_PEAK_TFS, "2.5 PF bf16"))
            entry.update(flops=flops, TFLOPs=round(tfs, 1), pct_mfma_peak=round(100 * tfs * mult / peak, 1),
                         mfma_peak=peak_name)
        if r.get("got") is not None:
            heavy = w.algo_bytes > (1 << 30) or (flops or 0) > 1e10
            # every BASELINE config line carries the reference CPU time by
            # default; --cpu-all adds the other lines
            timed = w is head or getattr(w, "config_line", False) or args.cpu_all
            reps = (args.cpu_reps if w is head else
                    (1 if (flops or 0) > 1e10 else 3 if heavy else args.cpu_reps) if timed else 0)
            c = run_reference(R, w, r["host"], reps)
            if c is not None and c["want"] is not None:
                per, worst = parity(r["got"], c["want"], w.results)
                entry.update(max_abs_err=float(f"{worst['max_abs_err']:.3e}"), rel_err=float(f"{worst['rel_err']:.3e}"),
                             within_tolerance=all(e["within_tolerance"] for e in per.values()),
                             parity={k: {kk: (float(f"{vv:.3e}") if isinstance(vv, float) else vv)
                                         for kk, vv in e.items()} for k, e in per.items()})
                if w is head:
                    head_err = entry
            if c is not None and c["ms"]:
                entry.update(cpu_ms=round(c["ms"], 3), cpu_threads=threads, speedup_vs_cpu=round(c["ms"] / r["event_ms"], 1))
                if w is head:
                    head_cpu = c
        r.pop("got", None)
        r.pop("host", None)
        ops.append(entry)
        rate = (f"{entry['TFLOPs']:8.1f} TFLOP/s {entry['pct_mfma_peak']:5.1f}% of {entry['mfma_peak']}" if flops else
                f"{entry['GBps']:8.1f} GB/s  {entry['pct_hbm_peak']:5.1f}% of 8 TB/s")
        err = (f"  err {entry['max_abs_err']:.1e} abs {entry['rel_err']:.1e} rel "
               f"{'ok' if entry['within_tolerance'] else 'OUT OF TOLERANCE'}") if "max_abs_err" in entry else ""
        print(f"# {w.name:22s} {entry['us_per_op']:10.2f} us  {rate}" +
              (f"  cpu {entry['cpu_ms']:.2f} ms" if 'cpu_ms' in entry else "") + err, file=sys.stderr, flush=True)
        if w is head:
            head_res = r

    if head_res is None:
        print(json.dumps({"ops": ops}), flush=True)
        return 0

    achieved = head.algo_bytes / (head_res["event_ms"] * 1e-3) / 1e9
    traffic = read_traffic(head.name)
    cpu = None
    if head_cpu is not None:
        cpu = dict(value=round(head.algo_bytes / (head_cpu["ms"] * 1e-3) / 1e9, 2), unit="GB/s", cores=threads,
                   cores_available=avail, kind="reference",
                   sample=f"the full {head.name} step at the config shape through the reference's tensor.cpp "
                          f"(oracle/_ref, compiled from /root/reference), on the same input arrays as the GPU's "
                          f"set 0, output allocation included, median of {args.cpu_reps} runs after 1 warm-up: "
                          f"{head_cpu['ms']:.2f} ms per step",
                   build=ref_build, ms_per_step=round(head_cpu["ms"], 3),
                   threads_note="the reference's thread pool sized to this process's CPU share (OMP_NUM_THREADS "
                                "where set, which the GPU box sets to its CPUs per GPU; else the CPUs it may run on)")
    value = head.algo_bytes / (head_res["wall_ms"] * 1e-3) / 1e9
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head_res["wall_ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded N(mu,sigma) fp32 inputs generated on the device (sdh_fill_normal, seeds per "
                "tensor under ops[].seeds), resident in HBM; set 0 is also the reference CPU path's input",
        "config": {"workload": head.desc, "algorithmic_bytes": head.algo_bytes,
                   "rotation_sets": head_res["nsets"], "rotation_MB": round(head_res["footprint"] / 2**20)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": head.kernel, "kernel_us": round(head_res["event_ms"] * 1e3, 3)},
        "cpu_baseline": cpu,
        "speedup_vs_cpu": round(cpu["ms_per_step"] / head_res["wall_ms"], 1) if cpu else None,
        "max_abs_err": head_err["max_abs_err"] if head_err else None,
        "rel_err": head_err["rel_err"] if head_err else None,
        "within_tolerance": head_err["within_tolerance"] if head_err else None,
        "parity_note": ("every op line compares the GPU result of set 0 with the reference's tensor.cpp on the same "
                        "arrays, outside the timed region: max_abs_err = max|gpu - ref|, rel_err = max |gpu - ref| / "
                        "max(|ref|, 1); within_tolerance applies the op's bar (parity.metric, parity.bound)"),
        "ops": ops,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
