"""Python bindings of backend_hip's C ABI (include/sdh_backend.h), via ctypes.

This is a thin host-side mirror used by the parity tests and the benchmark:
``Backend`` loads ``libsdh.so`` (built in-tree by ``__graft_entry__.build()``)
and exposes every entry point with numpy-friendly helpers. Device memory comes
from the library's own arena (``DArray``); no other framework is involved.

There is deliberately no CPU fallback: if the library or the device is
missing, constructing ``Backend`` raises.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Optional, Sequence

import numpy as np

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_DIR, "libsdh.so")
STUB_PATH = os.path.join(PKG_DIR, "libsdh_stub.so")

SDH_OK = 0
SDH_ERR_UNAVAILABLE = 1
SDH_ERR_INVALID = 2
SDH_ERR_OOM = 3
SDH_ERR_HIP = 4

_STATUS = {1: "UNAVAILABLE", 2: "INVALID", 3: "OOM", 4: "HIP"}


class SdhError(RuntimeError):
    """A non-zero status from the C ABI, with the library's message."""

    def __init__(self, status: int, msg: str):
        super().__init__(f"[{_STATUS.get(status, status)}] {msg}")
        self.status = status


_i64, _fl, _vp, _int = C.c_int64, C.c_float, C.c_void_p, C.c_int

# name -> argtypes (all return int status unless listed in _RESTYPES)
SIGNATURES = {
    "sdh_last_error": [],
    "sdh_available": [],
    "sdh_device_name": [],
    "sdh_device_memory": [],
    "sdh_init": [C.c_size_t],
    "sdh_shutdown": [],
    "sdh_malloc": [C.c_size_t, C.POINTER(C.c_void_p)],
    "sdh_free": [_vp],
    "sdh_upload": [_vp, _vp, C.c_size_t],
    "sdh_download": [_vp, _vp, C.c_size_t],
    "sdh_copy": [_vp, _vp, C.c_size_t],
    "sdh_zero": [_vp, C.c_size_t],
    "sdh_synchronize": [],
    "sdh_register_external": [_vp, C.c_size_t],
    "sdh_unregister_external": [_vp],
    "sdh_memory_stats": [C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)],
    "sdh_group_norm": [_vp, _vp, _i64, _i64, _i64, _int, _vp, _vp, _fl],
    "sdh_layer_norm": [_vp, _vp, _i64, _i64, _vp, _vp, _fl],
    "sdh_rms_norm": [_vp, _vp, _i64, _i64, _vp, _fl],
    "sdh_rms_norm_heads": [_vp, _i64, _i64, _vp, _fl],
    "sdh_rope": [_vp, _i64, _i64, _i64, _i64, _vp, _vp, _int],
    "sdh_rope_qk": [_vp, _i64, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _int],
    "sdh_rope_qk_axes": [_vp, _i64, _vp, _i64, _i64, _i64, _i64, _vp, _int, _int, _int, _fl],
    "sdh_qknorm_rope": [_vp, _i64, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _fl, _vp, _vp, C.c_int],
    "sdh_softmax_rows": [_vp, _i64, _i64, _fl, _int],
    "sdh_softmax_rows_batched": [_vp, _i64, _i64, _fl, _int, _i64],
    "sdh_swiglu": [_vp, _vp, _vp, _i64],
    "sdh_geglu": [_vp, _vp, _i64, _i64],
    "sdh_silu": [_vp, _i64],
    "sdh_tanh": [_vp, _i64],
    "sdh_gelu": [_vp, _i64],
    "sdh_quick_gelu": [_vp, _i64],
    "sdh_add": [_vp, _vp, _i64],
    "sdh_scale": [_vp, _fl, _i64],
    "sdh_affine": [_vp, _fl, _fl, _i64],
    "sdh_modulation_rows": [_vp, _i64, _i64],
    "sdh_mul_rows": [_vp, _vp, _i64, _i64],
    "sdh_add_rows_scaled": [_vp, _vp, _vp, _i64, _i64],
    "sdh_add_channel_bias": [_vp, _vp, _i64, _i64, _i64],
    "sdh_add_rows": [_vp, _vp, _i64, _i64],
    "sdh_gemm_nt_bf16": [_i64, _i64, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, C.c_int],
    "sdh_linear_swiglu": [_vp, _vp, _vp, _vp, _i64, _i64, _i64],
    "sdh_gemm_nt_bf16_packed": [_i64, _i64, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, C.c_int],
    "sdh_rms_norm_modulate_bf16": [_vp, _vp, _i64, _i64, _vp, _vp, _fl],
    "sdh_rms_norm_gated_add": [_vp, _vp, _i64, _i64, _vp, _vp, _fl],
    "sdh_rms_norm_gated_add_modulate_bf16": [_vp, _vp, _vp, _i64, _i64, _vp, _vp, _vp, _vp, _fl, _fl],
    "sdh_swiglu_bf16": [_vp, _vp, _vp, _i64],
    "sdh_gemm_nt_f32": [_i64, _i64, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, C.c_int],
    "sdh_conv2d": [_vp, _i64, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _vp, C.c_int, C.c_int, _vp, _i64, _i64],
    "sdh_to_bf16": [_vp, _vp, _i64],
    "sdh_attention": [_vp, _vp, _vp, _vp, _i64, _i64, _i64, C.c_int, C.c_int, _i64, C.c_int],
    "sdh_attention_bf16": [_vp, _vp, _vp, _vp, _i64, _i64, _i64, C.c_int, C.c_int, _i64, C.c_int],
    "sdh_attention_fp16": [_vp, _vp, _vp, _vp, C.c_int, _i64, _i64, _i64, C.c_int, C.c_int, _i64, C.c_int],
    "sdh_qknorm_rope_attention": [_vp, _vp, _vp, _vp, C.c_int, _i64, _i64, C.c_int, _i64, _vp, _vp, _fl, _vp, _vp,
                                  C.c_int],
    "sdh_upsample_nearest2x": [_vp, _vp, _i64, _i64, _i64],
    "sdh_concat_channels": [_vp, _vp, _vp, _i64, _i64, _i64, _i64],
    "sdh_nchw_to_nlc": [_vp, _vp, _i64, _i64, _i64],
    "sdh_nlc_to_nchw": [_vp, _vp, _i64, _i64, _i64],
    "sdh_patchify": [_vp, _vp, _i64, _i64, _i64, C.c_int],
    "sdh_unpatchify": [_vp, _vp, _i64, _i64, _i64, C.c_int],
    "sdh_add_rms_norm": [_vp, _vp, _vp, _i64, _i64, _vp, _fl],
    "sdh_group_norm_silu": [_vp, _vp, _i64, _i64, _i64, _int, _vp, _vp, _fl],
    "sdh_group_norm_silu_noalloc": [_vp, _vp, _i64, _i64, _i64, _int, _vp, _vp, _fl],
    "sdh_ln_modulate_gate": [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _fl],
    "sdh_fill_normal": [_vp, _i64, C.c_uint64, _fl, _fl],
    "sdh_timer_record": [_int],
    "sdh_timer_elapsed": [_int, _int, C.POINTER(C.c_float)],
    "sdh_capture_begin": [],
    "sdh_capture_end": [C.POINTER(C.c_void_p)],
    "sdh_graph_launch": [_vp],
    "sdh_graph_destroy": [_vp],
}
_RESTYPES = {
    "sdh_last_error": C.c_char_p,
    "sdh_device_name": C.c_char_p,
    "sdh_device_memory": C.c_size_t,
}


def load_library(path: str = LIB_PATH) -> C.CDLL:
    """Loads a backend_hip shared library and declares every signature."""
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} is not built; run __graft_entry__.build() (or make -C "
                                f"stablediffusion-cpp_amd/csrc)")
    lib = C.CDLL(path)
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = _RESTYPES.get(name, C.c_int)
    return lib


def _p(x) -> Optional[int]:
    """Device address of a DArray (or None)."""
    if x is None:
        return None
    if isinstance(x, DArray):
        return x.ptr
    if isinstance(x, int):
        return x
    raise TypeError(f"expected DArray, int address or None, got {type(x).__name__}")


class DArray:
    """An array in the backend's device arena: float32 (activations) or
    uint16 (bf16 bit patterns, for weights)."""

    def __init__(self, backend: "Backend", shape: Sequence[int], ptr: Optional[int] = None, owned: bool = True,
                 dtype=np.float32):
        self.be = backend
        self.shape = tuple(int(s) for s in shape)
        self.size = int(np.prod(self.shape)) if self.shape else 1
        self.dtype = np.dtype(dtype)
        if self.dtype not in (np.dtype(np.float32), np.dtype(np.uint16)):
            raise TypeError("DArray holds float32 or uint16 (bf16) data")
        self.nbytes = self.size * self.dtype.itemsize
        self.owned = owned
        if ptr is None:
            ptr = backend.malloc(self.nbytes)
        self.ptr = ptr

    def upload(self, a: np.ndarray) -> "DArray":
        a = np.ascontiguousarray(a, dtype=self.dtype)
        if a.size != self.size:
            raise ValueError(f"upload size {a.size} != {self.size}")
        self.be.upload(self.ptr, a)
        return self

    def download(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        self.be.download(out, self.ptr)
        return out

    def free(self):
        if self.owned and self.ptr:
            self.be.free(self.ptr)
        self.ptr = 0

    def __del__(self):
        try:
            if self.owned and self.ptr:
                self.be.free(self.ptr)
        except Exception:
            pass


class Backend:
    """The loaded library plus numpy-level helpers for every entry point."""

    def __init__(self, path: str = LIB_PATH, require_device: bool = True, arena_bytes: int = 0):
        self.lib = load_library(path)
        self.path = path
        if require_device:
            if not self.lib.sdh_available():
                raise SdhError(SDH_ERR_UNAVAILABLE, "no HIP device visible to backend_hip")
            self.check(self.lib.sdh_init(arena_bytes))

    # -- plumbing --
    def last_error(self) -> str:
        return (self.lib.sdh_last_error() or b"").decode()

    def check(self, rc: int):
        if rc != SDH_OK:
            raise SdhError(rc, self.last_error())

    def call(self, name: str, *args):
        self.check(getattr(self.lib, name)(*args))

    def available(self) -> bool:
        return bool(self.lib.sdh_available())

    def device_name(self) -> str:
        return self.lib.sdh_device_name().decode()

    def malloc(self, nbytes: int) -> int:
        p = C.c_void_p()
        self.check(self.lib.sdh_malloc(nbytes, C.byref(p)))
        return p.value or 0

    def free(self, ptr: int):
        self.check(self.lib.sdh_free(ptr))

    def upload(self, ptr: int, a: np.ndarray):
        a = np.ascontiguousarray(a)
        self.check(self.lib.sdh_upload(ptr, a.ctypes.data, a.nbytes))

    def download(self, out: np.ndarray, ptr: int):
        assert out.flags.c_contiguous
        self.check(self.lib.sdh_download(out.ctypes.data, ptr, out.nbytes))

    def synchronize(self):
        self.check(self.lib.sdh_synchronize())

    def copy(self, dst, src, nbytes: int):
        """Device-to-device copy on the library stream (sdh_copy)."""
        self.check(self.lib.sdh_copy(_p(dst), _p(src), nbytes))

    def memory_stats(self):
        r, u = C.c_size_t(), C.c_size_t()
        self.check(self.lib.sdh_memory_stats(C.byref(r), C.byref(u)))
        return r.value, u.value

    def empty(self, shape) -> DArray:
        return DArray(self, shape)

    def array(self, a: np.ndarray) -> DArray:
        """float32 arrays stay float32; uint16 arrays are bf16 bit patterns."""
        dt = np.uint16 if np.asarray(a).dtype == np.uint16 else np.float32
        a = np.ascontiguousarray(a, dtype=dt)
        return DArray(self, a.shape, dtype=dt).upload(a)

    def randn(self, shape, seed: int, mean: float = 0.0, std: float = 1.0) -> DArray:
        d = DArray(self, shape)
        self.check(self.lib.sdh_fill_normal(d.ptr, d.size, seed, mean, std))
        return d

    def timer_record(self, slot: int):
        self.check(self.lib.sdh_timer_record(slot))

    def timer_elapsed(self, a: int, b: int) -> float:
        ms = C.c_float()
        self.check(self.lib.sdh_timer_elapsed(a, b, C.byref(ms)))
        return ms.value

    def capture_begin(self):
        """Starts recording the library stream into a graph (sdh_capture_begin)."""
        self.check(self.lib.sdh_capture_begin())

    def capture_end(self) -> int:
        """Ends the recording; returns the instantiated graph's handle."""
        g = C.c_void_p()
        self.check(self.lib.sdh_capture_end(C.byref(g)))
        return g.value

    def graph_launch(self, graph: int):
        self.check(self.lib.sdh_graph_launch(graph))

    def graph_destroy(self, graph: int):
        self.check(self.lib.sdh_graph_destroy(graph))

    # -- ops on DArrays (argument meaning as include/sdh_backend.h) --
    def group_norm(self, x, y, N, Cc, HW, groups, gamma, beta, eps, silu=False):
        self.call("sdh_group_norm_silu" if silu else "sdh_group_norm", _p(x), _p(y), N, Cc, HW, groups, _p(gamma),
                  _p(beta), eps)

    def layer_norm(self, x, y, rows, Cc, gamma, beta, eps):
        self.call("sdh_layer_norm", _p(x), _p(y), rows, Cc, _p(gamma), _p(beta), eps)

    def rms_norm(self, x, y, rows, Cc, gamma, eps):
        self.call("sdh_rms_norm", _p(x), _p(y), rows, Cc, _p(gamma), eps)

    def rope_qk_axes(self, q, inner_q, k, inner_k, N, S, dim, pos, axes, theta):
        """RoPE on q and k with the angles formed on the device from int32
        positions pos [S, 3] (a DArray of int32 bits), axes (d0, d1, d2)."""
        self.call("sdh_rope_qk_axes", _p(q), inner_q, _p(k), inner_k, N, S, dim, _p(pos), int(axes[0]),
                  int(axes[1]), int(axes[2]), float(theta))

    def rms_norm_heads(self, x, groups, dim, gamma, eps):
        self.call("sdh_rms_norm_heads", _p(x), groups, dim, _p(gamma), eps)

    def rope(self, x, N, S, inner, dim, cos_t, sin_t, interleaved):
        self.call("sdh_rope", _p(x), N, S, inner, dim, _p(cos_t), _p(sin_t), int(bool(interleaved)))

    def rope_qk(self, q, inner_q, k, inner_k, N, S, dim, cos_t, sin_t, interleaved):
        self.call("sdh_rope_qk", _p(q), inner_q, _p(k), inner_k, N, S, dim, _p(cos_t), _p(sin_t),
                  int(bool(interleaved)))

    def qknorm_rope(self, q, inner_q, k, inner_k, N, S, dim, gamma_q, gamma_k, eps, cos, sin, interleaved):
        self.call("sdh_qknorm_rope", _p(q), inner_q, _p(k), inner_k, N, S, dim, _p(gamma_q), _p(gamma_k), eps, _p(cos),
                  _p(sin), 1 if interleaved else 0)

    def softmax_rows(self, x, rows, cols, scale, causal=False, period=None):
        if period is None:
            self.call("sdh_softmax_rows", _p(x), rows, cols, scale, int(bool(causal)))
        else:
            self.call("sdh_softmax_rows_batched", _p(x), rows, cols, scale, int(bool(causal)), period)

    def attention(self, q, k, v, out, N, Sq, Skv, heads, kv_heads, d, causal=False):
        """out [N, Sq, heads*d] = softmax(q k^T / sqrt(d)) v per head (tensor.cpp:776-810)."""
        self.call("sdh_attention", _p(q), _p(k), _p(v), _p(out), N, Sq, Skv, heads, kv_heads, d, int(bool(causal)))

    def attention_bf16(self, q, k, v, out16, N, Sq, Skv, heads, kv_heads, d, causal=False):
        """As attention, out16 (uint16) holding the bf16 rounding of the result."""
        self.call("sdh_attention_bf16", _p(q), _p(k), _p(v), _p(out16), N, Sq, Skv, heads, kv_heads, d,
                  int(bool(causal)))

    def qknorm_rope_attention(self, q, k, v, out, N, S, heads, dim, gamma_q, gamma_k, eps, cos, sin, out_bf16=False,
                              fp16=False):
        """qknorm_rope (interleaved tables) of q and k, then self-attention; q is
        left normalised and rotated, k and v are read only."""
        self.call("sdh_qknorm_rope_attention", _p(q), _p(k), _p(v), _p(out), int(bool(out_bf16)), N, S, heads, dim,
                  _p(gamma_q), _p(gamma_k), eps, _p(cos), _p(sin), int(bool(fp16)))

    def attention_fp16(self, q, k, v, out, N, Sq, Skv, heads, kv_heads, d, causal=False, out_bf16=False):
        """Opt-in reduced precision attention (no reference counterpart): every
        product from block-scaled fp16 operands; out float32, or the bf16 bits
        (uint16) when out_bf16."""
        self.call("sdh_attention_fp16", _p(q), _p(k), _p(v), _p(out), int(bool(out_bf16)), N, Sq, Skv, heads,
                  kv_heads, d, int(bool(causal)))

    def swiglu(self, g, u, y, n):
        self.call("sdh_swiglu", _p(g), _p(u), _p(y), n)

    def geglu(self, x, y, rows, D):
        self.call("sdh_geglu", _p(x), _p(y), rows, D)

    def silu(self, x, n):
        self.call("sdh_silu", _p(x), n)

    def tanh(self, x, n):
        self.call("sdh_tanh", _p(x), n)

    def gelu(self, x, n):
        self.call("sdh_gelu", _p(x), n)

    def quick_gelu(self, x, n):
        self.call("sdh_quick_gelu", _p(x), n)

    def add(self, a, b, n):
        self.call("sdh_add", _p(a), _p(b), n)

    def scale(self, x, s, n):
        self.call("sdh_scale", _p(x), s, n)

    def affine(self, x, a, b, n):
        self.call("sdh_affine", _p(x), a, b, n)

    def modulation_rows(self, x, pairs, dim):
        """x [2 * pairs, dim] in place: rows 2p -> 1 + x, rows 2p + 1 -> tanh(x) (zimage.cpp:104-107)."""
        self.call("sdh_modulation_rows", _p(x), pairs, dim)

    def mul_rows(self, x, v, rows, dim):
        self.call("sdh_mul_rows", _p(x), _p(v), rows, dim)

    def add_rows_scaled(self, x, y, g, rows, dim):
        self.call("sdh_add_rows_scaled", _p(x), _p(y), _p(g), rows, dim)

    def add_rows(self, x, v, rows, dim):
        self.call("sdh_add_rows", _p(x), _p(v), rows, dim)

    def add_channel_bias(self, x, b, N, Cc, HW):
        self.call("sdh_add_channel_bias", _p(x), _p(b), N, Cc, HW)

    # GEMM (bf16 weights held in DArray buffers of uint16)
    def gemm_nt_bf16(self, M, N, K, A, lda, B, ldb, Cm, ldc, bias=None, accumulate=False):
        self.call("sdh_gemm_nt_bf16", M, N, K, _p(A), lda, _p(B), ldb, _p(Cm), ldc, _p(bias), 1 if accumulate else 0)

    def gemm_nt_bf16_packed(self, M, N, K, A16, lda, B, ldb, C, ldc, bias=None, accumulate=False):
        self.call("sdh_gemm_nt_bf16_packed", M, N, K, _p(A16), lda, _p(B), ldb, _p(C), ldc, _p(bias),
                  int(bool(accumulate)))

    def rms_norm_modulate_bf16(self, x, y16, rows, C, gamma, scale, eps):
        self.call("sdh_rms_norm_modulate_bf16", _p(x), _p(y16), rows, C, _p(gamma), _p(scale), eps)

    def rms_norm_gated_add(self, x, a, rows, C, gamma, gate, eps):
        self.call("sdh_rms_norm_gated_add", _p(x), _p(a), rows, C, _p(gamma), _p(gate), eps)

    def rms_norm_gated_add_modulate_bf16(self, x, a, y16, rows, C, gamma_out, gate, gamma_in, scale, eps_out,
                                         eps_in=None):
        self.call("sdh_rms_norm_gated_add_modulate_bf16", _p(x), _p(a), _p(y16), rows, C, _p(gamma_out), _p(gate),
                  _p(gamma_in), _p(scale), eps_out, eps_out if eps_in is None else eps_in)

    def swiglu_bf16(self, g, u, y16, n):
        self.call("sdh_swiglu_bf16", _p(g), _p(u), _p(y16), n)

    def gemm_nt_f32(self, M, N, K, A, lda, B, ldb, C, ldc, bias=None, accumulate=False):
        self.call("sdh_gemm_nt_f32", M, N, K, _p(A), lda, _p(B), ldb, _p(C), ldc, _p(bias), int(bool(accumulate)))

    def conv2d(self, x, N, Cin, H, W, w, Cout, kh, kw, bias, stride, pad, out, Ho, Wo):
        self.call("sdh_conv2d", _p(x), N, Cin, H, W, _p(w), Cout, kh, kw, _p(bias), stride, pad, _p(out), Ho, Wo)

    def to_bf16(self, x, y, n):
        self.call("sdh_to_bf16", _p(x), _p(y), n)

    def linear_swiglu(self, x, w1, w3, y, rows, inn, hidden):
        self.call("sdh_linear_swiglu", _p(x), _p(w1), _p(w3), _p(y), rows, inn, hidden)

    # layout (tensor.cpp:931-1099)
    def upsample_nearest2x(self, x, y, NC, H, W):
        self.call("sdh_upsample_nearest2x", _p(x), _p(y), NC, H, W)

    def concat_channels(self, a, b, y, N, Ca, Cb, HW):
        self.call("sdh_concat_channels", _p(a), _p(b), _p(y), N, Ca, Cb, HW)

    def nchw_to_nlc(self, x, y, N, Cc, HW):
        self.call("sdh_nchw_to_nlc", _p(x), _p(y), N, Cc, HW)

    def nlc_to_nchw(self, x, y, N, Cc, HW):
        self.call("sdh_nlc_to_nchw", _p(x), _p(y), N, Cc, HW)

    def patchify(self, x, y, Cc, H, W, p):
        self.call("sdh_patchify", _p(x), _p(y), Cc, H, W, p)

    def unpatchify(self, x, y, Cc, H, W, p):
        self.call("sdh_unpatchify", _p(x), _p(y), Cc, H, W, p)

    def add_rms_norm(self, x, r, y, rows, Cc, gamma, eps):
        self.call("sdh_add_rms_norm", _p(x), _p(r), _p(y), rows, Cc, _p(gamma), eps)

    def ln_modulate_gate(self, x, res, scale, shift, gate, y_out, rows, Cc, eps):
        self.call("sdh_ln_modulate_gate", _p(x), _p(res), _p(scale), _p(shift), _p(gate), _p(y_out), rows, Cc, eps)


# ---------------------------------------------------------------- the Z-Image transformer
TENSOR_LIB_PATH = os.path.join(PKG_DIR, "libsdh_tensor.so")
_MODEL_SIGNATURES = {
    "sdhm_zimage_load": ([C.c_char_p, _int, _i64, _int, C.POINTER(C.c_void_p)], _int),
    "sdhm_zimage_random": ([_i64, _int, _i64, _i64, _i64, _i64, _i64, _int, _int, _int, C.c_uint64,
                            C.POINTER(C.c_void_p)], _int),
    "sdhm_zimage_forward": ([C.c_void_p, _vp, _i64, _i64, _i64, _fl, _vp, _i64, _i64, _vp], _int),
    "sdhm_zimage_time": ([C.c_void_p, _i64, _i64, _i64, _i64, _int, _int, C.POINTER(C.c_double)], _int),
    "sdhm_zimage_set_fp16_attention": ([C.c_void_p, _int], _int),
    "sdhm_zimage_params": ([C.c_void_p], _i64),
    "sdhm_zimage_free": ([C.c_void_p], None),
    "sdhm_last_error": ([], C.c_char_p),
}
_tensor_lib = None


def _model_lib():
    """libsdh_tensor.so (the C++ host library: tensor.h API, weights loader,
    Z-Image transformer); it runs on the same libsdh.so as Backend."""
    global _tensor_lib
    if _tensor_lib is None:
        if not os.path.exists(TENSOR_LIB_PATH):
            raise FileNotFoundError(f"{TENSOR_LIB_PATH} is not built; run __graft_entry__.build()")
        lib = C.CDLL(TENSOR_LIB_PATH)
        for name, (args, res) in _MODEL_SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        _tensor_lib = lib
    return _tensor_lib


class ZImage:
    """ZImageTransformer (src/zimage.h:40-79) on the device: one denoising step
    per forward(). Load it from a .safetensors checkpoint, or build one of given
    shapes with seeded random weights (benchmarks)."""

    def __init__(self, handle):
        self.h = handle

    @staticmethod
    def _check(rc):
        if rc != 0:
            raise SdhError(SDH_ERR_INVALID, _model_lib().sdhm_last_error().decode())

    @classmethod
    def load(cls, path, heads=30, keep_bf16=True, bf16_min_numel=1 << 20):
        h = C.c_void_p()
        cls._check(_model_lib().sdhm_zimage_load(str(path).encode(), int(bool(keep_bf16)), int(bf16_min_numel),
                                                 int(heads), C.byref(h)))
        return cls(h)

    @classmethod
    def random(cls, dim=3840, heads=30, ffn=10240, in_channels=16, cap_dim=2560, t_hidden=1024, adaln_dim=256,
               noise_refiners=2, context_refiners=2, layers=30, seed=0):
        h = C.c_void_p()
        cls._check(_model_lib().sdhm_zimage_random(dim, heads, ffn, in_channels, cap_dim, t_hidden, adaln_dim,
                                                   noise_refiners, context_refiners, layers, seed, C.byref(h)))
        return cls(h)

    def forward(self, x, t, cap):
        x = np.ascontiguousarray(x, np.float32)
        cap = np.ascontiguousarray(cap, np.float32)
        out = np.empty_like(x)
        self._check(_model_lib().sdhm_zimage_forward(self.h, x.ctypes.data, x.shape[1], x.shape[2], x.shape[3],
                                                     float(t), cap.ctypes.data, cap.shape[1], cap.shape[2],
                                                     out.ctypes.data))
        return out

    def set_fp16_attention(self, on=True):
        """Opt-in (no reference counterpart): later forwards run attention from
        block-scaled fp16 operands (sdh_attention_fp16)."""
        self._check(_model_lib().sdhm_zimage_set_fp16_attention(self.h, int(bool(on))))

    def time(self, H, W, L, cap_dim, steps, warmup):
        ms = C.c_double()
        self._check(_model_lib().sdhm_zimage_time(self.h, H, W, L, cap_dim, steps, warmup, C.byref(ms)))
        return ms.value

    def params(self):
        return int(_model_lib().sdhm_zimage_params(self.h))

    def close(self):
        if self.h:
            _model_lib().sdhm_zimage_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
