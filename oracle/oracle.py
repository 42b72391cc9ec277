"""ctypes bindings of the parity checkers. TEST INFRASTRUCTURE ONLY.

Two libraries live here, both built by ``oracle/Makefile``:

* ``liboracle.so`` -- the C restatement of the reference's ops (sd_oracle.c).
  ``Oracle`` wraps it with numpy arrays in, numpy arrays out.
* ``_ref/libsdref.so`` -- the reference's own ``src/tensor.cpp`` compiled from
  /root/reference.  ``Reference`` wraps it the same way, and also exposes the
  handle API used to time the reference CPU path as it is called.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's cpu_baseline leg may
import this module, and only as the checker: the product never routes a
computation through it.
"""
from __future__ import annotations

import ctypes as C
import os
import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libsdref.so")

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_i64 = C.c_int64
_fl = C.c_float
_vp = C.c_void_p


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


class _NullableF32:
    """ctypes argtype accepting a float32 array or None."""

    @classmethod
    def from_param(cls, obj):
        if obj is None:
            return None
        if not (isinstance(obj, np.ndarray) and obj.dtype == np.float32 and obj.flags.c_contiguous):
            raise TypeError("expected a C-contiguous float32 array or None")
        return obj.ctypes.data_as(C.c_void_p)


def f32_to_bf16(a) -> np.ndarray:
    """bf16 bit patterns of float32 values: nearest even, inf and NaN keep
    their top 16 bits (tensor.cpp:114-121, and the device pack kernel
    backend_cuda.cu:183-188)."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32)
    r = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)
    special = (u & np.uint32(0x7F800000)) == np.uint32(0x7F800000)
    r[special] = (u[special] >> np.uint32(16)).astype(np.uint16)
    return r


def bf16_to_f32(h) -> np.ndarray:
    return (np.asarray(h, np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


class Oracle:
    """numpy-level wrapper of liboracle.so (the C restatement)."""

    def __init__(self, path: str = ORACLE_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} not built (run make -C oracle)")
        L = self.lib = C.CDLL(path)
        N = _NullableF32
        sig = {
            "orc_set_threads": (None, [C.c_int]),
            "orc_num_threads": (C.c_int, []),
            "orc_plant_mistake": (None, [C.c_int]),
            "orc_fill_normal": (None, [_f32p, _i64, C.c_uint64, C.c_double, C.c_double]),
            "orc_group_norm": (None, [_f32p, _f32p, _i64, _i64, _i64, C.c_int, _f32p, _f32p, _fl]),
            "orc_group_norm_silu": (None, [_f32p, _f32p, _i64, _i64, _i64, C.c_int, _f32p, _f32p, _fl]),
            "orc_layer_norm": (None, [_f32p, _f32p, _i64, _i64, N, N, _fl]),
            "orc_rms_norm": (None, [_f32p, _f32p, _i64, _i64, N, _fl]),
            "orc_rms_norm_heads": (None, [_f32p, _i64, _i64, N, _fl]),
            "orc_rope": (None, [_f32p, _i64, _i64, _i64, _i64, _f32p, _f32p, C.c_int]),
            "orc_rope_tables_3axis": (None, [_i32p, _i64, _i32p, _i64, C.c_double, _f32p, _f32p]),
            "orc_rope_tables_half": (None, [_i64, _i64, C.c_double, _f32p, _f32p]),
            "orc_swiglu": (None, [_f32p, _f32p, _f32p, _i64]),
            "orc_geglu": (None, [_f32p, _f32p, _i64, _i64]),
            "orc_silu": (None, [_f32p, _i64]),
            "orc_tanh": (None, [_f32p, _i64]),
            "orc_gelu": (None, [_f32p, _i64]),
            "orc_quick_gelu": (None, [_f32p, _i64]),
            "orc_softmax_rows": (None, [_f32p, _i64, _i64, _fl, C.c_int]),
            "orc_softmax_rows_period": (None, [_f32p, _i64, _i64, _fl, C.c_int, _i64]),
            "orc_add": (None, [_f32p, _f32p, _i64]),
            "orc_scale": (None, [_f32p, _fl, _i64]),
            "orc_affine": (None, [_f32p, _fl, _fl, _i64]),
            "orc_mul_rows": (None, [_f32p, _f32p, _i64, _i64]),
            "orc_add_rows_scaled": (None, [_f32p, _f32p, _f32p, _i64, _i64]),
            "orc_add_channel_bias": (None, [_f32p, _f32p, _i64, _i64, _i64]),
            "orc_add_rms_norm": (None, [_f32p, _f32p, _f32p, _i64, _i64, N, _fl]),
            "orc_ln_modulate_gate": (None, [_f32p, _f32p, _f32p, N, _f32p, N, _i64, _i64, _fl]),
            "orc_qknorm_rope": (None, [_f32p, _i64, _f32p, _i64, _i64, _i64, _i64, N, N, _fl, _f32p, _f32p, C.c_int]),
            "orc_upsample_nearest2x": (None, [_f32p, _f32p, _i64, _i64, _i64]),
            "orc_concat_channels": (None, [_f32p, _f32p, _f32p, _i64, _i64, _i64, _i64]),
            "orc_nchw_to_nlc": (None, [_f32p, _f32p, _i64, _i64, _i64]),
            "orc_nlc_to_nchw": (None, [_f32p, _f32p, _i64, _i64, _i64]),
            "orc_patchify": (None, [_f32p, _f32p, _i64, _i64, _i64, C.c_int]),
            "orc_unpatchify": (None, [_f32p, _f32p, _i64, _i64, _i64, C.c_int]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args

    # -- control --
    def set_threads(self, n: int):
        self.lib.orc_set_threads(n)

    def num_threads(self) -> int:
        return self.lib.orc_num_threads()

    def plant(self, which: int):
        self.lib.orc_plant_mistake(which)
        self._plant_py = which  # plants of the numpy-level functions

    # -- generator --
    def randn(self, shape, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
        n = int(np.prod(shape)) if len(shape) else 1
        out = np.empty(n, np.float32)
        self.lib.orc_fill_normal(out, n, seed, mean, std)
        return out.reshape(shape)

    # -- ops (inputs are never modified; in-place ops return a new array) --
    def group_norm(self, x, groups, gamma, beta, eps, silu=False):
        x = _f32(x)
        N, Cc = x.shape[0], x.shape[1]
        HW = x.size // (N * Cc)
        y = np.empty_like(x)
        fn = self.lib.orc_group_norm_silu if silu else self.lib.orc_group_norm
        fn(x, y, N, Cc, HW, groups, _f32(gamma), _f32(beta), eps)
        return y

    def layer_norm(self, x, gamma, beta, eps):
        x = _f32(x)
        Cc = x.shape[-1]
        y = np.empty_like(x)
        self.lib.orc_layer_norm(x, y, x.size // Cc, Cc, None if gamma is None else _f32(gamma),
                                None if beta is None else _f32(beta), eps)
        return y

    def rms_norm(self, x, gamma, eps):
        x = _f32(x)
        Cc = x.shape[-1]
        y = np.empty_like(x)
        self.lib.orc_rms_norm(x, y, x.size // Cc, Cc, None if gamma is None else _f32(gamma), eps)
        return y

    def rms_norm_heads(self, x, dim, gamma, eps):
        y = _f32(x).copy()
        self.lib.orc_rms_norm_heads(y, y.size // dim, dim, None if gamma is None else _f32(gamma), eps)
        return y

    def rope(self, x, dim, cos_t, sin_t, interleaved):
        """x [..., S, inner] rotated in a copy; cos/sin [S, dim]."""
        y = _f32(x).copy()
        inner, S = y.shape[-1], y.shape[-2]
        N = y.size // (S * inner)
        self.lib.orc_rope(y, N, S, inner, dim, _f32(cos_t), _f32(sin_t), int(bool(interleaved)))
        return y

    def rope_tables_3axis(self, pos, axes_dims, dim, theta):
        pos = np.ascontiguousarray(pos, dtype=np.int32)
        S = pos.shape[0]
        c = np.empty((S, dim), np.float32)
        s = np.empty((S, dim), np.float32)
        self.lib.orc_rope_tables_3axis(pos, S, np.ascontiguousarray(axes_dims, dtype=np.int32), dim, theta, c, s)
        return c, s

    def rope_tables_half(self, S, dim, theta):
        c = np.empty((S, dim), np.float32)
        s = np.empty((S, dim), np.float32)
        self.lib.orc_rope_tables_half(S, dim, theta, c, s)
        return c, s

    def swiglu(self, g, u):
        g, u = _f32(g), _f32(u)
        y = np.empty_like(g)
        self.lib.orc_swiglu(g, u, y, g.size)
        return y

    def geglu(self, x):
        x = _f32(x)
        D = x.shape[-1] // 2
        y = np.empty(x.shape[:-1] + (D,), np.float32)
        self.lib.orc_geglu(x, y, x.size // (2 * D), D)
        return y

    def _unary(self, fn, x):
        y = _f32(x).copy()
        fn(y, y.size)
        return y

    def silu(self, x):
        return self._unary(self.lib.orc_silu, x)

    def tanh(self, x):
        return self._unary(self.lib.orc_tanh, x)

    def gelu(self, x):
        return self._unary(self.lib.orc_gelu, x)

    def quick_gelu(self, x):
        return self._unary(self.lib.orc_quick_gelu, x)

    def softmax_rows(self, x, scale, causal=False, period=None):
        y = _f32(x).copy()
        cols = y.shape[-1]
        rows = y.size // cols
        if period is None:
            self.lib.orc_softmax_rows(y, rows, cols, scale, int(bool(causal)))
        else:
            self.lib.orc_softmax_rows_period(y, rows, cols, scale, int(bool(causal)), period)
        return y

    def add(self, a, b):
        y = _f32(a).copy()
        self.lib.orc_add(y, _f32(b), y.size)
        return y

    def scale(self, x, s):
        y = _f32(x).copy()
        self.lib.orc_scale(y, s, y.size)
        return y

    def affine(self, x, a, b):
        y = _f32(x).copy()
        self.lib.orc_affine(y, a, b, y.size)
        return y

    def mul_rows(self, x, v):
        y = _f32(x).copy()
        dim = y.shape[-1]
        self.lib.orc_mul_rows(y, _f32(v), y.size // dim, dim)
        return y

    def add_rows_scaled(self, x, yv, g):
        o = _f32(x).copy()
        dim = o.shape[-1]
        self.lib.orc_add_rows_scaled(o, _f32(yv), _f32(g), o.size // dim, dim)
        return o

    def add_channel_bias(self, x, b):
        y = _f32(x).copy()
        N, Cc = y.shape[0], y.shape[1]
        self.lib.orc_add_channel_bias(y, _f32(b), N, Cc, y.size // (N * Cc))
        return y

    def add_rms_norm(self, x, r, gamma, eps):
        """Returns (x + r, rms_norm(x + r) * gamma)."""
        s = _f32(x).copy()
        y = np.empty_like(s)
        Cc = s.shape[-1]
        self.lib.orc_add_rms_norm(s, _f32(r), y, s.size // Cc, Cc, None if gamma is None else _f32(gamma), eps)
        return s, y

    def ln_modulate_gate(self, x, res, scale, shift, gate, eps):
        """Returns (res + tanh(gate) * y, y) with y = LN(x) * (1 + scale) + shift."""
        x = _f32(x)
        r = _f32(res).copy()
        y = np.empty_like(x)
        Cc = x.shape[-1]
        self.lib.orc_ln_modulate_gate(x, r, _f32(scale), None if shift is None else _f32(shift), _f32(gate), y,
                                      x.size // Cc, Cc, eps)
        return r, y

    def qknorm_rope(self, q, k, dim, gamma_q, gamma_k, eps, cos_t, sin_t, interleaved):
        """q [N, S, inner_q], k [N, S, inner_k] -> (q', k'): QK-norm then RoPE."""
        q2, k2 = _f32(q).copy(), _f32(k).copy()
        N, S = q2.shape[0], q2.shape[1]
        self.lib.orc_qknorm_rope(q2, q2.shape[-1], k2, k2.shape[-1], N, S, dim,
                                 None if gamma_q is None else _f32(gamma_q), None if gamma_k is None else _f32(gamma_k),
                                 eps, _f32(cos_t), _f32(sin_t), 1 if interleaved else 0)
        return q2, k2

    # -- linear with bf16 weights (the reference's device path) --
    # backend_cuda.cu:466-479: A is rounded to bf16, products of bf16 pairs are
    # exact, the device sums them in fp32. Here they are summed exactly
    # (float64 products of bf16 values are exact, and the sums of K <= 2^20
    # terms are far inside float64), so a GPU result differs from this only
    # by its fp32 accumulation. Returns (C, S) with S = sum_k |a_k b_k| per
    # element, the scale of that accumulation error.
    def gemm_nt_bf16(self, A, B16, bias=None, C=None, accumulate=False):
        a = bf16_to_f32(f32_to_bf16(A)).astype(np.float64)
        if getattr(self, "_plant_py", 0) == 8:  # planted: A not rounded to bf16
            a = np.asarray(A, np.float64)
        b = bf16_to_f32(B16).astype(np.float64)
        acc = a @ b.T
        if accumulate:
            acc = np.asarray(C, np.float64) + acc
        if bias is not None:
            bb = np.asarray(bias, np.float64)
            if getattr(self, "_plant_py", 0) == 9:  # planted: bias indexed by row
                acc = acc + bb[: acc.shape[0], None]
            else:
                acc = acc + bb[None, :]
        return acc.astype(np.float32), np.abs(a) @ np.abs(b).T

    def gemm_nt_f32(self, A, B, bias=None, C=None, accumulate=False):
        """C = A B^T (+ C) (+ bias) with fp32 operands, summed exactly
        (float64): the reference's fp32 linear (tensor.cpp:354-406,
        backend_cuda.cu:453-464) differs from this only by its fp32 sums.
        Returns (C, S), S = sum_k |a_k b_k| per element."""
        a = np.asarray(A, np.float32).astype(np.float64)
        b = np.asarray(B, np.float32).astype(np.float64)
        acc = a @ b.T
        if accumulate:
            acc = np.asarray(C, np.float64) + acc
        if bias is not None:
            acc = acc + np.asarray(bias, np.float64)[None, :]
        return acc.astype(np.float32), np.abs(a) @ np.abs(b).T

    def conv2d(self, x, w, b=None, stride=1, pad=0):
        """float64 conv2d as the reference defines it (tensor.cpp:520-560): out
        [N, Cout, Ho, Wo], Ho = (H + 2 pad - kh) / stride + 1, out[n, co, oy, ox]
        = b[co] + sum over (ci, ky, kx) of w[co, ci, ky, kx] x[n, ci, oy*stride
        - pad + ky, ox*stride - pad + kx], zero outside the image. Returns
        (out as fp32, S = the same sum of absolute products) for the fp32
        accumulation bound."""
        x = np.asarray(x, np.float32).astype(np.float64)
        w = np.asarray(w, np.float32).astype(np.float64)
        N, Cin, H, W = x.shape
        Cout, _, kh, kw = w.shape
        Ho, Wo = (H + 2 * pad - kh) // stride + 1, (W + 2 * pad - kw) // stride + 1
        xp = np.zeros((N, Cin, H + 2 * pad, W + 2 * pad))
        xp[:, :, pad:pad + H, pad:pad + W] = x
        plant = getattr(self, "_plant_py", 0)
        cols = np.empty((N, Ho, Wo, Cin, kh, kw))
        for ky in range(kh):
            for kx in range(kw):
                win = xp[:, :, ky:ky + stride * (Ho - 1) + 1:stride, kx:kx + stride * (Wo - 1) + 1:stride]
                if plant == 15 and kh == kw:  # planted: kernel taps transposed (ky, kx swapped)
                    cols[..., kx, ky] = win.transpose(0, 2, 3, 1)
                else:
                    cols[..., ky, kx] = win.transpose(0, 2, 3, 1)
        cols = cols.reshape(N, Ho * Wo, Cin * kh * kw)
        wm = w.reshape(Cout, -1)
        out = np.matmul(cols, wm.T).transpose(0, 2, 1)
        S = np.matmul(np.abs(cols), np.abs(wm).T).transpose(0, 2, 1)
        if b is not None and plant != 16:  # planted 16: bias dropped
            out = out + np.asarray(b, np.float64)[None, :, None]
            S = S + np.abs(np.asarray(b, np.float64))[None, :, None]
        return out.reshape(N, Cout, Ho, Wo).astype(np.float32), S.reshape(N, Cout, Ho, Wo)

    def linear_swiglu(self, x, w1_16, w3_16):
        """y = swiglu(x w1^T, x w3^T) with exact products, plus the exact g,
        u and their accumulation scales (for the test's error bound)."""
        g, sg = self.gemm_nt_bf16(x, w1_16)
        u, su = self.gemm_nt_bf16(x, w3_16)
        g64, u64 = g.astype(np.float64), u.astype(np.float64)
        y = (g64 / (1.0 + np.exp(-g64)) * u64).astype(np.float32)
        return y, g, u, sg, su

    # -- attention (tensor.cpp:776-810) --
    def attention(self, q, k, v, heads, causal=False, kv_heads=0, rows=None):
        """float64 restatement of the reference's attention, as its own test
        restates it in double (test_ops.cpp:84-114): per head h, key/value
        head g = h / (heads / kv_heads) (tensor.cpp:795-797), scores
        q_h k_g^T scaled by the fp32 1/sqrt(d) (tensor.cpp:784), causal rows
        keep keys j <= i (softmax_rows_, tensor.cpp:756), softmax, then P v_g.
        q [N, Sq, heads*d], k and v [N, Skv, kv_heads*d]. `rows` restricts
        the result to those query rows (returned [N, len(rows), heads*d])."""
        plant = getattr(self, "_plant_py", 0)
        if kv_heads <= 0:
            kv_heads = heads
        q, k, v = (np.asarray(a, np.float32) for a in (q, k, v))
        N, Sq, inner = q.shape
        Skv = k.shape[1]
        d = inner // heads
        group = heads // kv_heads
        rows = np.arange(Sq) if rows is None else np.asarray(rows)
        scale = np.float64(np.float32(1.0) / np.sqrt(np.float32(d)))
        if plant == 10:  # planted: no 1/sqrt(d)
            scale = np.float64(1.0)
        qh = q[:, rows].reshape(N, len(rows), heads, d).transpose(0, 2, 1, 3).astype(np.float64)
        kh = k.reshape(N, Skv, kv_heads, d).transpose(0, 2, 1, 3).astype(np.float64)
        vh = v.reshape(N, Skv, kv_heads, d).transpose(0, 2, 1, 3).astype(np.float64)
        g = np.arange(heads) % kv_heads if plant == 12 else np.arange(heads) // group  # planted 12: heads interleaved
        kh, vh = kh[:, g], vh[:, g]
        s = np.matmul(qh, kh.transpose(0, 1, 3, 2)) * scale
        if causal:
            lim = rows[:, None] + (1 if plant == 11 else 0)  # planted 11: one key past the diagonal
            s = np.where(np.arange(Skv)[None, :] > lim, -np.inf, s)
        s = s - s.max(axis=-1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=-1, keepdims=True)
        o = np.matmul(p, vh)
        return o.transpose(0, 2, 1, 3).reshape(N, len(rows), inner).astype(np.float32)

    # -- the Z-Image transformer (zimage.cpp:71-228) --
    def zimage_forward(self, weights, x, t, cap, heads, bf16_names=(), act_bf16=False, patch=2, eps=1e-5,
                       theta=256.0, t_scale=1000.0, axes=(32, 48, 48)):
        """float64 restatement of ZImageTransformer::forward. `weights` maps
        checkpoint names to float32 arrays (the values the loader produces);
        `bf16_names` are the weights held in BF16. With act_bf16 the input of
        every linear with a BF16 weight is rounded to bf16 first, as the
        device path does (backend_cuda.cu:466-479); without it the inputs stay
        exact, as the reference's CPU path keeps them fp32 (tensor.cpp:496-497).
        x [1, C, H, W], cap [1, L, cap_dim] -> [1, C, H, W]."""
        plant = getattr(self, "_plant_py", 0)
        f64 = np.float64
        Wd = {k: np.asarray(v, np.float32).astype(f64) for k, v in weights.items()}
        bf = set(bf16_names)

        def lin(name, h):  # modules.h:23-30, tensor.cpp:481-500
            if act_bf16 and name + ".weight" in bf:
                h = bf16_to_f32(f32_to_bf16(h.astype(np.float32))).astype(f64)
            y = h @ Wd[name + ".weight"].T
            b = Wd.get(name + ".bias")
            return y if b is None else y + b

        def rms(h, g, e):  # tensor.cpp:660-679
            return h / np.sqrt((h * h).mean(-1, keepdims=True) + e) * (Wd[g] if g else 1.0)

        def silu(h):
            return h / (1.0 + np.exp(-h))

        D = Wd["all_x_embedder.2-1.weight"].shape[0]
        hd = D // heads
        p = patch
        # 1. timestep embedding (zimage.cpp:148-163), the sinusoid in float as there
        F = Wd["t_embedder.mlp.0.weight"].shape[1]
        half = F // 2
        tt = np.float32(t) * np.float32(t_scale)
        fr = np.exp(-np.log(np.float32(10000.0)) * np.arange(half, dtype=np.float32) / np.float32(half)).astype(np.float32)
        freq = np.concatenate([np.cos(tt * fr), np.sin(tt * fr)]).astype(np.float32).astype(f64)[None, :]
        adaln = lin("t_embedder.mlp.2", silu(lin("t_embedder.mlp.0", freq)))
        # 2. image tokens: features ordered (ph, pw, c) (tensor.cpp:931-954)
        _, Cc, H, W = x.shape
        Ht, Wt = H // p, W // p
        tok = np.asarray(x, f64)[0].reshape(Cc, Ht, p, Wt, p).transpose(1, 3, 2, 4, 0).reshape(Ht * Wt, p * p * Cc)
        n_img = Ht * Wt
        pad32 = lambda n: (n + 31) // 32 * 32
        n_img_pad = pad32(n_img)
        img = lin("all_x_embedder.2-1", tok)
        img = np.concatenate([img, np.repeat(Wd["x_pad_token"].reshape(1, D), n_img_pad - n_img, 0)])
        # 3. text tokens
        n_cap = cap.shape[1]
        n_cap_pad = pad32(n_cap)
        ct = lin("cap_embedder.1", rms(np.asarray(cap, f64)[0], "cap_embedder.0.weight", eps))
        ct = np.concatenate([ct, np.repeat(Wd["cap_pad_token"].reshape(1, D), n_cap_pad - n_cap, 0)])
        # rotary positions (zimage.cpp:177-191) and tables (zimage.cpp:71-88, float angles)
        cap_pos = [(1 + i, 0, 0) for i in range(n_cap_pad)]
        img_pos = [(0, 0, 0)] * n_img_pad
        for hh in range(Ht):
            for ww in range(Wt):
                img_pos[hh * Wt + ww] = (n_cap_pad + 1, hh, ww) if plant != 13 else (n_cap_pad + 1, ww, hh)

        def tables(pos):
            cs = np.zeros((len(pos), hd), np.float32)
            sn = np.zeros((len(pos), hd), np.float32)
            off = 0
            for a in range(3):
                da = axes[a]
                fq = 1.0 / np.power(float(theta), (2.0 * np.arange(da // 2)) / da)
                for si, ps in enumerate(pos):
                    ang = (ps[a] * fq).astype(np.float32)
                    cs[si, off:off + da:2] = cs[si, off + 1:off + da:2] = np.cos(ang)
                    sn[si, off:off + da:2] = sn[si, off + 1:off + da:2] = np.sin(ang)
                off += da
            return cs.astype(f64), sn.astype(f64)

        def rope(h, cs, sn):  # interleaved pairs (tensor.cpp:698-730)
            S = h.shape[0]
            r = h.reshape(S, heads, hd // 2, 2)
            c = cs[:, 0::2][:, None, :]
            s_ = sn[:, 0::2][:, None, :]
            a, b = r[..., 0], r[..., 1]
            return np.stack([a * c - b * s_, b * c + a * s_], -1).reshape(S, D)

        def heads_norm(h, g):  # rms_norm_heads_ (tensor.cpp:681-696), eps 1e-5 (zimage.cpp:117-118)
            S = h.shape[0]
            r = h.reshape(S, heads, hd)
            return (r / np.sqrt((r * r).mean(-1, keepdims=True) + 1e-5) * Wd[g]).reshape(S, D)

        def block(pre, xs, cs, sn, modulated):  # zimage.cpp:90-136
            if modulated:
                m = lin(pre + ".adaLN_modulation.0", adaln).reshape(4, D)
                s_msa, g_msa, s_mlp, g_mlp = 1.0 + m[0], np.tanh(m[1]), 1.0 + m[2], np.tanh(m[3])
                if plant == 14:
                    s_msa, g_msa = g_msa, s_msa
            h = rms(xs, pre + ".attention_norm1.weight", eps)
            if modulated:
                h = h * s_msa
            q = rope(heads_norm(lin(pre + ".attention.to_q", h), pre + ".attention.norm_q.weight"), cs, sn)
            k = rope(heads_norm(lin(pre + ".attention.to_k", h), pre + ".attention.norm_k.weight"), cs, sn)
            v = lin(pre + ".attention.to_v", h)
            S = xs.shape[0]
            qh = q.reshape(S, heads, hd).transpose(1, 0, 2)
            kh = k.reshape(S, heads, hd).transpose(1, 0, 2)
            vh = v.reshape(S, heads, hd).transpose(1, 0, 2)
            sc = qh @ kh.transpose(0, 2, 1) * float(np.float32(1.0) / np.sqrt(np.float32(hd)))
            sc = np.exp(sc - sc.max(-1, keepdims=True))
            att = ((sc / sc.sum(-1, keepdims=True)) @ vh).transpose(1, 0, 2).reshape(S, D)
            a = rms(lin(pre + ".attention.to_out.0", att), pre + ".attention_norm2.weight", eps)
            xs = xs + (g_msa * a if modulated else a)
            h = rms(xs, pre + ".ffn_norm1.weight", eps)
            if modulated:
                h = h * s_mlp
            g, u = lin(pre + ".feed_forward.w1", h), lin(pre + ".feed_forward.w3", h)
            f = rms(lin(pre + ".feed_forward.w2", silu(g) * u), pre + ".ffn_norm2.weight", eps)
            return xs + (g_mlp * f if modulated else f)

        def count(prefix):
            i = 0
            while f"{prefix}.{i}.attention_norm1.weight" in Wd:
                i += 1
            return i

        ic, is_ = tables(img_pos)
        for i in range(count("noise_refiner")):
            img = block(f"noise_refiner.{i}", img, ic, is_, True)
        cc, cs_ = tables(cap_pos)
        for i in range(count("context_refiner")):
            ct = block(f"context_refiner.{i}", ct, cc, cs_, False)
        uni = np.concatenate([img, ct])
        uc, us = tables(img_pos + cap_pos)
        for i in range(count("layers")):
            uni = block(f"layers.{i}", uni, uc, us, True)
        # 5. final layer (zimage.cpp:218-227): LayerNorm without affine, eps 1e-6
        io = uni[:n_img]
        scale = 1.0 + lin("all_final_layer.2-1.adaLN_modulation.1", silu(adaln))
        mu = io.mean(-1, keepdims=True)
        io = (io - mu) / np.sqrt(((io - mu) ** 2).mean(-1, keepdims=True) + 1e-6) * scale
        ot = lin("all_final_layer.2-1.linear", io)
        out = ot.reshape(Ht, Wt, p, p, Cc).transpose(4, 0, 2, 1, 3).reshape(1, Cc, H, W)
        return out.astype(np.float32)

    # -- layout (tensor.cpp:931-1099) --
    def upsample_nearest2x(self, x):
        x = _f32(x)
        N, Cc, H, W = x.shape
        y = np.empty((N, Cc, 2 * H, 2 * W), np.float32)
        self.lib.orc_upsample_nearest2x(x, y, N * Cc, H, W)
        return y

    def concat_channels(self, a, b):
        a, b = _f32(a), _f32(b)
        N, Ca, Cb = a.shape[0], a.shape[1], b.shape[1]
        HW = a.size // (N * Ca) if Ca else b.size // (N * Cb)
        y = np.empty((N, Ca + Cb) + a.shape[2:], np.float32)
        self.lib.orc_concat_channels(a, b, y, N, Ca, Cb, HW)
        return y

    def nchw_to_nlc(self, x):
        x = _f32(x)
        N, Cc = x.shape[0], x.shape[1]
        HW = x.size // (N * Cc)
        y = np.empty((N, HW, Cc), np.float32)
        self.lib.orc_nchw_to_nlc(x, y, N, Cc, HW)
        return y

    def nlc_to_nchw(self, x, H, W):
        x = _f32(x)
        N, HW, Cc = x.shape
        assert HW == H * W
        y = np.empty((N, Cc, H, W), np.float32)
        self.lib.orc_nlc_to_nchw(x, y, N, Cc, HW)
        return y

    def patchify(self, x, p):
        """x [1, C, H, W] (or [C, H, W]) -> tokens [(H/p)(W/p), p*p*C]."""
        x = _f32(x)
        Cc, H, W = x.shape[-3:]
        y = np.empty(((H // p) * (W // p), p * p * Cc), np.float32)
        self.lib.orc_patchify(x, y, Cc, H, W, p)
        return y

    def unpatchify(self, tokens, Cc, H, W, p):
        """tokens [(H/p)(W/p), p*p*C] -> [1, C, H, W] (uncovered rows/columns 0)."""
        y = np.zeros((1, Cc, H, W), np.float32)
        self.lib.orc_unpatchify(_f32(tokens), y, Cc, H, W, p)
        return y


class Reference:
    """numpy-level wrapper of the compiled reference tensor library."""

    def __init__(self, path: str = REF_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} not built (run make -C oracle ref where /root/reference exists)")
        L = self.lib = C.CDLL(path)
        sig = {
            "ref_last_error": (C.c_char_p, []),
            "ref_set_threads": (None, [C.c_int]),
            "ref_num_threads": (C.c_int, []),
            "ref_tensor_new": (_vp, [C.POINTER(C.c_int64), C.c_int]),
            "ref_tensor_data": (C.POINTER(C.c_float), [_vp]),
            "ref_tensor_numel": (C.c_int64, [_vp]),
            "ref_tensor_free": (None, [_vp]),
            "ref_group_norm": (_vp, [_vp, C.c_int, _vp, _vp, _fl]),
            "ref_layer_norm": (_vp, [_vp, _vp, _vp, _fl]),
            "ref_rms_norm": (_vp, [_vp, _vp, _fl]),
            "ref_swiglu": (_vp, [_vp, _vp]),
            "ref_geglu": (_vp, [_vp]),
            "ref_rms_norm_heads_": (C.c_int, [_vp, _i64, _vp, _fl]),
            "ref_rope_": (C.c_int, [_vp, _i64, _vp, _vp, C.c_int]),
            "ref_softmax_rows_": (C.c_int, [_vp, _i64, _i64, _fl, C.c_int]),
            "ref_silu_": (C.c_int, [_vp]),
            "ref_tanh_": (C.c_int, [_vp]),
            "ref_gelu_": (C.c_int, [_vp]),
            "ref_quick_gelu_": (C.c_int, [_vp]),
            "ref_add_": (C.c_int, [_vp, _vp]),
            "ref_scale_": (C.c_int, [_vp, _fl]),
            "ref_affine_": (C.c_int, [_vp, _fl, _fl]),
            "ref_mul_rows_": (C.c_int, [_vp, _vp]),
            "ref_add_rows_scaled_": (C.c_int, [_vp, _vp, _vp]),
            "ref_add_channel_bias_": (C.c_int, [_vp, _vp]),
            "ref_tensor_to_bf16": (C.c_int, [_vp]),
            "ref_tensor_data16": (C.POINTER(C.c_uint16), [_vp]),
            "ref_linear": (_vp, [_vp, _vp, _vp]),
            "ref_attention": (_vp, [_vp, _vp, _vp, C.c_int, C.c_int, C.c_int]),
            "ref_conv2d": (_vp, [_vp, _vp, _vp, C.c_int, C.c_int]),
            "ref_zimage_forward": (C.c_int, [C.c_char_p, C.c_int, _i64, C.c_int, _f32p, _i64, _i64, _i64, _fl, _f32p,
                                             _i64, _i64, _f32p]),
            "ref_vae_decode": (C.c_int, [C.c_char_p, _fl, _fl, _f32p, _i64, _i64, _i64, _f32p, _i64,
                                         C.POINTER(C.c_int64)]),
            "ref_patchify2d": (_vp, [_vp, C.c_int]),
            "ref_unpatchify2d": (_vp, [_vp, _i64, _i64, _i64, C.c_int]),
            "ref_slice_rows": (_vp, [_vp, _i64, _i64]),
            "ref_upsample_nearest2x": (_vp, [_vp]),
            "ref_concat_channels": (_vp, [_vp, _vp]),
            "ref_concat_batch": (_vp, [_vp, _vp]),
            "ref_nchw_to_nlc": (_vp, [_vp]),
            "ref_nlc_to_nchw": (_vp, [_vp, _i64, _i64]),
            "ref_slice_batch": (_vp, [_vp, _i64]),
            "ref_repeat_batch": (_vp, [_vp, _i64]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args

    # -- handles --
    def new(self, shape, data=None):
        shp = (C.c_int64 * len(shape))(*[int(s) for s in shape])
        h = self.lib.ref_tensor_new(shp, len(shape))
        if not h:
            raise RuntimeError(self.lib.ref_last_error().decode())
        if data is not None:
            self.view(h)[...] = np.asarray(data, np.float32).reshape(-1)
        return h

    def view(self, h) -> np.ndarray:
        n = self.lib.ref_tensor_numel(h)
        return np.ctypeslib.as_array(self.lib.ref_tensor_data(h), shape=(n,))

    def take(self, h, shape) -> np.ndarray:
        out = self.view(h).copy().reshape(shape)
        self.lib.ref_tensor_free(h)
        return out

    def free(self, *hs):
        for h in hs:
            if h:
                self.lib.ref_tensor_free(h)

    def _chk(self, rc):
        if rc:
            raise RuntimeError(self.lib.ref_last_error().decode())

    def _ptr(self, h):
        if not h:
            raise RuntimeError(self.lib.ref_last_error().decode())
        return h

    # -- numpy-level ops (same meaning as Oracle's) --
    def group_norm(self, x, groups, gamma, beta, eps, silu=False):
        x = _f32(x)
        hx, hg, hb = self.new(x.shape, x), self.new(gamma.shape, gamma), self.new(beta.shape, beta)
        hy = self._ptr(self.lib.ref_group_norm(hx, groups, hg, hb, eps))
        if silu:
            self._chk(self.lib.ref_silu_(hy))
        self.free(hx, hg, hb)
        return self.take(hy, x.shape)

    def layer_norm(self, x, gamma, beta, eps):
        x = _f32(x)
        hx = self.new(x.shape, x)
        hg = self.new(gamma.shape, gamma) if gamma is not None else None
        hb = self.new(beta.shape, beta) if beta is not None else None
        hy = self._ptr(self.lib.ref_layer_norm(hx, hg, hb, eps))
        self.free(hx, hg, hb)
        return self.take(hy, x.shape)

    def rms_norm(self, x, gamma, eps):
        x = _f32(x)
        hx = self.new(x.shape, x)
        hg = self.new(gamma.shape, gamma) if gamma is not None else None
        hy = self._ptr(self.lib.ref_rms_norm(hx, hg, eps))
        self.free(hx, hg)
        return self.take(hy, x.shape)

    def rms_norm_heads(self, x, dim, gamma, eps):
        x = _f32(x)
        hx = self.new(x.shape, x)
        hg = self.new(gamma.shape, gamma) if gamma is not None else None
        self._chk(self.lib.ref_rms_norm_heads_(hx, dim, hg, eps))
        self.free(hg)
        return self.take(hx, x.shape)

    def rope(self, x, dim, cos_t, sin_t, interleaved):
        x = _f32(x)
        hx, hc, hs = self.new(x.shape, x), self.new(cos_t.shape, cos_t), self.new(sin_t.shape, sin_t)
        self._chk(self.lib.ref_rope_(hx, dim, hc, hs, int(bool(interleaved))))
        self.free(hc, hs)
        return self.take(hx, x.shape)

    def swiglu(self, g, u):
        g = _f32(g)
        hg, hu = self.new(g.shape, g), self.new(u.shape, u)
        hy = self._ptr(self.lib.ref_swiglu(hg, hu))
        self.free(hg, hu)
        return self.take(hy, g.shape)

    def geglu(self, x):
        x = _f32(x)
        hx = self.new(x.shape, x)
        hy = self._ptr(self.lib.ref_geglu(hx))
        self.free(hx)
        return self.take(hy, x.shape[:-1] + (x.shape[-1] // 2,))

    def _unary(self, fn, x):
        x = _f32(x)
        hx = self.new(x.shape, x)
        self._chk(fn(hx))
        return self.take(hx, x.shape)

    def silu(self, x):
        return self._unary(self.lib.ref_silu_, x)

    def tanh(self, x):
        return self._unary(self.lib.ref_tanh_, x)

    def gelu(self, x):
        return self._unary(self.lib.ref_gelu_, x)

    def quick_gelu(self, x):
        return self._unary(self.lib.ref_quick_gelu_, x)

    def softmax_rows(self, x, scale, causal=False):
        x = _f32(x)
        hx = self.new(x.shape, x)
        cols = x.shape[-1]
        self._chk(self.lib.ref_softmax_rows_(hx, x.size // cols, cols, scale, int(bool(causal))))
        return self.take(hx, x.shape)

    def add(self, a, b):
        a = _f32(a)
        ha, hb = self.new(a.shape, a), self.new(b.shape, b)
        self._chk(self.lib.ref_add_(ha, hb))
        self.free(hb)
        return self.take(ha, a.shape)

    def scale(self, x, s):
        x = _f32(x)
        hx = self.new(x.shape, x)
        self._chk(self.lib.ref_scale_(hx, s))
        return self.take(hx, x.shape)

    def affine(self, x, a, b):
        x = _f32(x)
        hx = self.new(x.shape, x)
        self._chk(self.lib.ref_affine_(hx, a, b))
        return self.take(hx, x.shape)

    def mul_rows(self, x, v):
        x = _f32(x)
        hx, hv = self.new(x.shape, x), self.new(v.shape, v)
        self._chk(self.lib.ref_mul_rows_(hx, hv))
        self.free(hv)
        return self.take(hx, x.shape)

    def add_rows_scaled(self, x, yv, g):
        x = _f32(x)
        hx, hy, hg = self.new(x.shape, x), self.new(yv.shape, yv), self.new(g.shape, g)
        self._chk(self.lib.ref_add_rows_scaled_(hx, hy, hg))
        self.free(hy, hg)
        return self.take(hx, x.shape)

    def add_channel_bias(self, x, b):
        x = _f32(x)
        hx, hb = self.new(x.shape, x), self.new(b.shape, b)
        self._chk(self.lib.ref_add_channel_bias_(hx, hb))
        self.free(hb)
        return self.take(hx, x.shape)

    # -- bf16 / linear --
    def to_bf16(self, a):
        """The reference's own Tensor::to_bf16 rounding of a float32 array."""
        a = _f32(a)
        h = self.new(a.shape, a)
        try:
            self._chk(self.lib.ref_tensor_to_bf16(h))
            return np.ctypeslib.as_array(self.lib.ref_tensor_data16(h), shape=(a.size,)).copy().reshape(a.shape)
        finally:
            self.free(h)

    def linear(self, x, W, b=None, bf16=True):
        """The reference's CPU linear. bf16: W converted to BF16 first
        (tensor.cpp:496-497: x stays fp32, W is rounded to bf16, products
        summed in fp32); otherwise the fp32 path (tensor.cpp:498, :354-406)."""
        x, W = _f32(x), _f32(W)
        hx, hw = self.new(x.shape, x), self.new(W.shape, W)
        hb = self.new(b.shape, b) if b is not None else None
        try:
            if bf16:
                self._chk(self.lib.ref_tensor_to_bf16(hw))
            h = self._ptr(self.lib.ref_linear(hx, hw, hb))
        finally:
            self.free(hx, hw, hb)
        return self.take(h, x.shape[:-1] + (W.shape[0],))

    def attention(self, q, k, v, heads, causal=False, kv_heads=0):
        """The reference's CPU attention (tensor.cpp:776-810): fp32 gemm_nt
        scores, softmax_rows_ with scale 1/sqrt(d), fp32 gemm_nt with v^T."""
        q, k, v = _f32(q), _f32(k), _f32(v)
        hq, hk, hv = self.new(q.shape, q), self.new(k.shape, k), self.new(v.shape, v)
        try:
            h = self._ptr(self.lib.ref_attention(hq, hk, hv, heads, int(bool(causal)), kv_heads))
        finally:
            self.free(hq, hk, hv)
        return self.take(h, q.shape)

    def conv2d(self, x, w, b=None, stride=1, pad=0):
        """The reference's CPU conv2d (tensor.cpp:520-560: im2col rows, then the
        fp32 GEMM seeded with the bias)."""
        x, w = _f32(x), _f32(w)
        hx, hw = self.new(x.shape, x), self.new(w.shape, w)
        hb = self.new(b.shape, _f32(b)) if b is not None else None
        try:
            h = self._ptr(self.lib.ref_conv2d(hx, hw, hb, stride, pad))
        finally:
            self.free(hx, hw, hb)
        N, _, H, W = x.shape
        Cout, _, kh, kw = w.shape
        return self.take(h, (N, Cout, (H + 2 * pad - kh) // stride + 1, (W + 2 * pad - kw) // stride + 1))

    def zimage_forward(self, path, x, t, cap, heads, keep_bf16=True, bf16_min_numel=1 << 20):
        """The reference's ZImageTransformer::forward on the CPU (zimage.cpp:
        138-228) with weights loaded by its own Weights::load_safetensors."""
        x, cap = _f32(x), _f32(cap)
        out = np.empty_like(x)
        self._chk(self.lib.ref_zimage_forward(str(path).encode(), int(bool(keep_bf16)), int(bf16_min_numel), int(heads),
                                              x, x.shape[1], x.shape[2], x.shape[3], float(t), cap, cap.shape[1],
                                              cap.shape[2], out))
        return out

    def vae_decode(self, path, z, scaling, shift):
        """The reference's VAEDecoder::decode on the CPU (vae.cpp:35-51) with
        F32 weights loaded by its own Weights::load_safetensors."""
        z = _f32(z)
        cap = 1024 * z.shape[2] * z.shape[3]  # up to 16 output channels at 8x per side
        out = np.empty(cap, np.float32)
        shape = (C.c_int64 * 4)()
        self._chk(self.lib.ref_vae_decode(str(path).encode(), float(scaling), float(shift), z, z.shape[1], z.shape[2],
                                          z.shape[3], out, cap, shape))
        n = int(np.prod(list(shape)))
        return out[:n].reshape(tuple(shape)).copy()

    # -- layout --
    def _new_op(self, fn, inputs, out_shape, *args):
        hs = [self.new(a.shape, a) for a in inputs]
        try:
            h = self._ptr(fn(*hs, *args))
        finally:
            self.free(*hs)
        return self.take(h, out_shape)

    def upsample_nearest2x(self, x):
        x = _f32(x)
        N, Cc, H, W = x.shape
        return self._new_op(self.lib.ref_upsample_nearest2x, [x], (N, Cc, 2 * H, 2 * W))

    def concat_channels(self, a, b):
        a, b = _f32(a), _f32(b)
        return self._new_op(self.lib.ref_concat_channels, [a, b], (a.shape[0], a.shape[1] + b.shape[1]) + a.shape[2:])

    def concat_batch(self, a, b):
        a, b = _f32(a), _f32(b)
        return self._new_op(self.lib.ref_concat_batch, [a, b], (a.shape[0] + b.shape[0],) + a.shape[1:])

    def nchw_to_nlc(self, x):
        x = _f32(x)
        N, Cc = x.shape[0], x.shape[1]
        return self._new_op(self.lib.ref_nchw_to_nlc, [x], (N, x.size // (N * Cc), Cc))

    def nlc_to_nchw(self, x, H, W):
        x = _f32(x)
        return self._new_op(self.lib.ref_nlc_to_nchw, [x], (x.shape[0], x.shape[2], H, W), H, W)

    def patchify(self, x, p):
        x = _f32(x)
        Cc, H, W = x.shape[-3:]
        return self._new_op(self.lib.ref_patchify2d, [x.reshape(1, Cc, H, W)], ((H // p) * (W // p), p * p * Cc), p)

    def unpatchify(self, tokens, Cc, H, W, p):
        return self._new_op(self.lib.ref_unpatchify2d, [_f32(tokens)], (1, Cc, H, W), Cc, H, W, p)

    def slice_rows(self, x, a, b):
        x = _f32(x)
        return self._new_op(self.lib.ref_slice_rows, [x], (b - a, x.shape[-1]), a, b)

    def slice_batch(self, x, i):
        x = _f32(x)
        return self._new_op(self.lib.ref_slice_batch, [x], (1,) + x.shape[1:], i)

    def repeat_batch(self, x, times):
        x = _f32(x)
        return self._new_op(self.lib.ref_repeat_batch, [x], (x.shape[0] * times,) + x.shape[1:], times)

    # -- compositions, exactly as the reference's callers chain the ops --
    def add_rms_norm(self, x, r, gamma, eps):
        s = self.add(x, r)
        return s, self.rms_norm(s, gamma, eps)

    def ln_modulate_gate(self, x, res, scale, shift, gate, eps):
        Cc = x.shape[-1]
        y = self.layer_norm(x, None, None, eps)
        s1 = self.affine(scale, 1.0, 1.0)
        tg = self.tanh(gate)
        y = self.mul_rows(y, s1)
        if shift is not None:
            y = self.add_rows_scaled(y, np.ones_like(y), shift)
        out = self.add_rows_scaled(res, y, tg)
        assert out.shape[-1] == Cc
        return out, y


def have_reference() -> bool:
    return os.path.exists(REF_SO)
