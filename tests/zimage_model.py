"""A small Z-Image transformer for tests: the checkpoint's tensor names and
layout (zimage.cpp:38-68) at toy sizes, seeded random weights, written as a
.safetensors file with every tensor in BF16, as the released checkpoint stores
them. Head size 128 (the 32 + 48 + 48 rotary axes need it), two heads."""
import json
import struct

import numpy as np

from oracle import bf16_to_f32, f32_to_bf16

# dim 256 = 2 heads x 128; FFN 512; 16 latent channels in 2x2 patches; text
# hidden size 64; timestep MLP 256 -> 64 -> 64; one refiner of each kind and
# two main layers. With bf16_min_numel = BF16_MIN every block linear is BF16
# and the embedders, the timestep MLP and the final layer stay F32, so both
# GEMM paths run.
SHAPES = dict(dim=256, heads=2, ffn=512, in_channels=16, cap_dim=64, t_freq=256, t_hidden=64, adaln_dim=64,
              noise_refiners=1, context_refiners=1, layers=2, patch=2)
BF16_MIN = 20000


def make_weights(seed=0, s=SHAPES):
    """name -> float32 array of bf16-exact values (what the file holds)."""
    rng = np.random.default_rng(seed)
    W = {}
    D, pp = s["dim"], s["patch"] ** 2

    def lin(p, out, inn, bias):
        W[p + ".weight"] = rng.standard_normal((out, inn), dtype=np.float32) / np.float32(np.sqrt(inn))
        if bias:
            W[p + ".bias"] = rng.standard_normal((out,), dtype=np.float32) * np.float32(0.1)

    def norm(name, n):
        W[name] = np.float32(1.0) + rng.standard_normal((n,), dtype=np.float32) * np.float32(0.1)

    lin("all_x_embedder.2-1", D, pp * s["in_channels"], True)
    norm("cap_embedder.0.weight", s["cap_dim"])
    lin("cap_embedder.1", D, s["cap_dim"], True)
    lin("t_embedder.mlp.0", s["t_hidden"], s["t_freq"], True)
    lin("t_embedder.mlp.2", s["adaln_dim"], s["t_hidden"], True)
    lin("all_final_layer.2-1.linear", pp * s["in_channels"], D, True)
    lin("all_final_layer.2-1.adaLN_modulation.1", D, s["adaln_dim"], True)
    W["x_pad_token"] = rng.standard_normal((1, D), dtype=np.float32)
    W["cap_pad_token"] = rng.standard_normal((1, D), dtype=np.float32)
    hd = D // s["heads"]

    def block(p, modulated):
        for n in ("attention_norm1", "attention_norm2", "ffn_norm1", "ffn_norm2"):
            norm(f"{p}.{n}.weight", D)
        norm(f"{p}.attention.norm_q.weight", hd)
        norm(f"{p}.attention.norm_k.weight", hd)
        for n in ("to_q", "to_k", "to_v", "to_out.0"):
            lin(f"{p}.attention.{n}", D, D, False)
        lin(f"{p}.feed_forward.w1", s["ffn"], D, False)
        lin(f"{p}.feed_forward.w2", D, s["ffn"], False)
        lin(f"{p}.feed_forward.w3", s["ffn"], D, False)
        if modulated:
            lin(f"{p}.adaLN_modulation.0", 4 * D, s["adaln_dim"], True)

    for i in range(s["noise_refiners"]):
        block(f"noise_refiner.{i}", True)
    for i in range(s["context_refiners"]):
        block(f"context_refiner.{i}", False)
    for i in range(s["layers"]):
        block(f"layers.{i}", True)
    return {k: bf16_to_f32(f32_to_bf16(v)).reshape(v.shape) for k, v in W.items()}


def write_safetensors(path, weights):
    """Every tensor as BF16: 8-byte header length, JSON header, raw bytes."""
    header, blobs, off = {}, [], 0
    for name in sorted(weights):
        b = f32_to_bf16(weights[name]).tobytes()
        header[name] = {"dtype": "BF16", "shape": list(weights[name].shape), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    header["__metadata__"] = {"format": "pt"}
    h = json.dumps(header).encode()
    h += b" " * ((8 - len(h) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


def bf16_names(weights, min_numel=BF16_MIN):
    return {k for k, v in weights.items() if v.size >= min_numel}


def inputs(orc, seed=0, H=16, W=16, L=20, s=SHAPES):
    x = orc.randn((1, s["in_channels"], H, W), 900 + seed)
    cap = orc.randn((1, L, s["cap_dim"]), 901 + seed)
    return x, cap


def rel_rms(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.sqrt(np.sum((got - want) ** 2) / np.sum(want ** 2)))
