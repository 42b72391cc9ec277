"""Small AutoencoderKL decoders for tests: the checkpoint's tensor names and
layout (vae.cpp:15-32, modules.cpp:12-31, :119-130) at toy sizes, seeded
random F32 weights, written as a .safetensors file.

Two shapes:
  * SMALL: 16 latent channels -> 64 -> mid block at 64 (one-head attention
    over 64 channels) -> up blocks 64, 64 (each with an upsampler), 32 (a
    shortcut conv on the channel change) -> 3 channels; a latent h x w
    decodes to 3 x 4h x 4w.
  * WIDE: the mid block at the FLUX VAE's 512 channels (its one-head
    attention then takes the head-size > 128 route), up blocks 256, 128;
    3 x 2h x 2w.
GroupNorm has 32 groups (modules.h), so every width is a multiple of 32.
"""
import json
import struct

import numpy as np

SMALL = dict(latent=16, conv_in=64, mid=64, up=[(64, 2, True), (64, 2, True), (32, 2, False)], out=3)
WIDE = dict(latent=16, conv_in=512, mid=512, up=[(256, 1, True), (128, 1, False)], out=3)


def make_weights(seed=0, s=SMALL):
    """name -> float32 array."""
    rng = np.random.default_rng(seed)
    W = {}

    def conv(p, cout, cin, k=3):
        W[p + ".weight"] = rng.standard_normal((cout, cin, k, k), dtype=np.float32) / np.float32(np.sqrt(cin * k * k))
        W[p + ".bias"] = rng.standard_normal((cout,), dtype=np.float32) * np.float32(0.05)

    def lin(p, cout, cin):
        W[p + ".weight"] = rng.standard_normal((cout, cin), dtype=np.float32) / np.float32(np.sqrt(cin))
        W[p + ".bias"] = rng.standard_normal((cout,), dtype=np.float32) * np.float32(0.05)

    def norm(p, c):
        W[p + ".weight"] = np.float32(1.0) + rng.standard_normal((c,), dtype=np.float32) * np.float32(0.1)
        W[p + ".bias"] = rng.standard_normal((c,), dtype=np.float32) * np.float32(0.1)

    def resnet(p, cin, cout):
        norm(p + ".norm1", cin)
        conv(p + ".conv1", cout, cin)
        norm(p + ".norm2", cout)
        conv(p + ".conv2", cout, cout)
        if cin != cout:
            conv(p + ".conv_shortcut", cout, cin, 1)

    conv("decoder.conv_in", s["conv_in"], s["latent"])
    c = s["conv_in"]
    resnet("decoder.mid_block.resnets.0", c, s["mid"])
    c = s["mid"]
    a = "decoder.mid_block.attentions.0"
    norm(a + ".group_norm", c)
    for n in ("to_q", "to_k", "to_v", "to_out.0"):
        lin(f"{a}.{n}", c, c)
    resnet("decoder.mid_block.resnets.1", c, c)
    for i, (cout, nres, upsample) in enumerate(s["up"]):
        for j in range(nres):
            resnet(f"decoder.up_blocks.{i}.resnets.{j}", c, cout)
            c = cout
        if upsample:
            conv(f"decoder.up_blocks.{i}.upsamplers.0.conv", c, c)
    norm("decoder.conv_norm_out", c)
    conv("decoder.conv_out", s["out"], c)
    return W


def write_safetensors_f32(path, weights):
    """Every tensor as F32: 8-byte header length, JSON header, raw bytes."""
    header, blobs, off = {}, [], 0
    for name in sorted(weights):
        b = np.ascontiguousarray(weights[name], dtype="<f4").tobytes()
        header[name] = {"dtype": "F32", "shape": list(weights[name].shape), "data_offsets": [off, off + len(b)]}
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
