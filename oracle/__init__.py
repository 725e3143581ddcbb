"""The oracle: ctypes access to oracle/liboracle.so, the plain-C restatement
of NaiveDiffusion's CPU layer math (Tensors/CpuMath.cs), its int8 block
quantiser (Tensors/BlockQuantizer.cs), the Transformer helpers
(Graph/Transformer.cs) and the DirectML operator semantics the graphs use.

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() as
the checker, and by bench.py for the CPU baseline. The product
(naivediffusion_amd) never imports it.

Every function takes and returns numpy float32 arrays (int8 / uint16 for
the quantiser) and names the reference member it follows in oracle.c.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")


def build() -> Path:
    """Compile liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", str(HERE), "liboracle.so"], check=True)
    return LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        c_int, c_float, c_double, c_i64, vp = ctypes.c_int, ctypes.c_float, ctypes.c_double, ctypes.c_int64, ctypes.c_void_p
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_f32_to_f16.argtypes = [c_float]
        L.orc_f16_to_f32.restype = c_float
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f32_to_bf16.restype = ctypes.c_uint16
        L.orc_f32_to_bf16.argtypes = [c_float]
        L.orc_dot.restype = c_float
        L.orc_dot.argtypes = [_f32p, _f32p, c_int]
        L.orc_linear.argtypes = [_f32p, c_int, c_int, _f32p, vp, vp, c_int]
        L.orc_layer_norm.argtypes = [_f32p, c_int, c_int, vp, vp, vp, c_float]
        L.orc_rms_norm.argtypes = [_f32p, c_int, c_int, vp, vp, c_float]
        L.orc_rope.argtypes = [vp, c_int, c_int, c_int, _f32p, _f32p]
        L.orc_rope_tables.argtypes = [c_int, c_int, c_double, _f32p, _f32p]
        L.orc_attention.argtypes = [_f32p, _f32p, _f32p, c_int, c_int, c_int, c_int, c_int, c_int, vp]
        L.orc_mha.argtypes = [_f32p, _f32p, _f32p, c_int, c_int, c_int, c_int, c_int, c_float, c_int, c_int, vp,
                              c_i64, c_i64, c_i64, c_i64, vp]
        for name in ("orc_silu", "orc_gelu", "orc_gelu_tanh", "orc_sigmoid", "orc_tanh"):
            getattr(L, name).argtypes = [vp, c_i64]
        L.orc_sinusoid.argtypes = [c_float, c_int, _f32p]
        L.orc_modulate.argtypes = [_f32p, c_int, c_int, vp, _f32p, c_float, vp]
        L.orc_group_norm.argtypes = [_f32p, c_int, c_int, c_int, c_int, vp, vp, c_float, c_int, vp]
        L.orc_conv2d.argtypes = [_f32p, c_int, c_int, c_int, c_int, _f32p, c_int, c_int, c_int, vp, c_int, c_int,
                                 c_int, vp]
        L.orc_upsample_nearest.argtypes = [_f32p, c_int, c_int, c_int, c_int, c_int, vp]
        L.orc_quantize.restype = c_int
        L.orc_quantize.argtypes = [_f32p, c_int, c_int, c_int, c_int, vp, vp]
        L.orc_quantization_loss.argtypes = [_f32p, c_int, c_int, c_int, ctypes.POINTER(c_double),
                                            ctypes.POINTER(c_double)]
        L.orc_qwen_rope_tables.argtypes = [c_int, c_int, c_int, c_int, _f32p, _f32p]
        L.orc_mmdit_rope_tables.argtypes = [c_int, c_int, c_int, _f32p, _f32p]
        L.orc_causal_table.argtypes = [c_int, c_int, _i32p]
        L.orc_mmdit_block.argtypes = [vp, c_int, vp, c_int, _f32p, c_int, c_int, c_int, c_int, vp, vp, _f32p, _f32p,
                                      c_int, c_float]
        _lib = L
    return _lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


# ---- narrow floats ---------------------------------------------------------

def f32_to_f16_bits(x) -> np.ndarray:
    x = _f32(x)
    f = lib().orc_f32_to_f16
    return np.array([f(float(v)) for v in x.ravel()], dtype=np.uint16).reshape(x.shape)


def f16_bits_to_f32(h) -> np.ndarray:
    h = np.asarray(h, dtype=np.uint16)
    f = lib().orc_f16_to_f32
    return np.array([f(int(v)) for v in h.ravel()], dtype=np.float32).reshape(h.shape)


def f32_to_bf16_bits(x) -> np.ndarray:
    x = _f32(x)
    f = lib().orc_f32_to_bf16
    return np.array([f(float(v)) for v in x.ravel()], dtype=np.uint16).reshape(x.shape)


# ---- CpuMath -----------------------------------------------------------------

def dot(a, b) -> float:
    a, b = _f32(a), _f32(b)
    return float(lib().orc_dot(a, b, a.size))


def linear(x, w, bias=None) -> np.ndarray:
    """CpuMath.Linear: x [..., K] times w [N, K]^T (+ bias)."""
    x, w = _f32(x), _f32(w)
    K = x.shape[-1]
    rows = x.size // K
    N = w.shape[0]
    b = None if bias is None else _f32(bias)
    y = np.empty(x.shape[:-1] + (N,), np.float32)
    lib().orc_linear(x, rows, K, w, _ptr(b), _ptr(y), N)
    return y


def layer_norm(x, weight=None, bias=None, eps=1e-6) -> np.ndarray:
    x = _f32(x)
    W = x.shape[-1]
    w = None if weight is None else _f32(weight)
    b = None if bias is None else _f32(bias)
    y = np.empty_like(x)
    lib().orc_layer_norm(x, x.size // W, W, _ptr(w), _ptr(b), _ptr(y), eps)
    return y


def rms_norm(x, weight=None, eps=1e-6) -> np.ndarray:
    x = _f32(x)
    W = x.shape[-1]
    w = None if weight is None else _f32(weight)
    y = np.empty_like(x)
    lib().orc_rms_norm(x, x.size // W, W, _ptr(w), _ptr(y), eps)
    return y


def rope(x, heads, cos, sin) -> np.ndarray:
    """CpuMath.Rope over [rows, heads*dim]; returns a rotated copy."""
    y = _f32(x).copy()
    rows = y.shape[-2] if y.ndim >= 2 else 1
    dim = y.shape[-1] // heads
    lib().orc_rope(_ptr(y), y.size // (heads * dim), heads, dim, _f32(cos), _f32(sin))
    return y


def rope_tables(rows, dim, theta):
    c = np.empty((rows, dim // 2), np.float32)
    s = np.empty((rows, dim // 2), np.float32)
    lib().orc_rope_tables(rows, dim, theta, c, s)
    return c, s


def attention(q, k, v, q_heads, k_heads, causal=False) -> np.ndarray:
    """CpuMath.Attention over q [rows, qh*d], k/v [keys, kh*d]."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    dim = q.shape[-1] // q_heads
    y = np.empty_like(q)
    lib().orc_attention(q, k, v, q.shape[0], k.shape[0], q_heads, k_heads, dim, int(causal), _ptr(y))
    return y


def mha(q, k, v, heads, scale=None, mask_kind=0, key_len=0, mask=None) -> np.ndarray:
    """DmlOps.MultiheadAttention semantics over [batch, tokens, heads*d]."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    if q.ndim == 2:
        q, k, v = q[None], k[None], v[None]
    B, T, W = q.shape
    S = k.shape[1]
    dim = W // heads
    scale = 1.0 / np.sqrt(np.float32(dim)) if scale is None else scale
    y = np.empty_like(q)
    strides = (0, 0, 0, 0)
    m = None
    if mask is not None:
        m = np.ascontiguousarray(mask, dtype=np.int32)
        m4 = m.reshape((1,) * (4 - m.ndim) + m.shape)
        strides = tuple(0 if m4.shape[i] == 1 else m4.strides[i] // 4 for i in range(4))
    lib().orc_mha(q, k, v, B, T, S, heads, dim, float(np.float32(scale)), mask_kind, key_len, _ptr(m), *strides, _ptr(y))
    return y


def _unary(name, x) -> np.ndarray:
    y = _f32(x).copy()
    getattr(lib(), name)(_ptr(y), y.size)
    return y


def silu(x): return _unary("orc_silu", x)
def gelu(x): return _unary("orc_gelu", x)
def gelu_tanh(x): return _unary("orc_gelu_tanh", x)
def sigmoid(x): return _unary("orc_sigmoid", x)
def tanh(x): return _unary("orc_tanh", x)


def sinusoid(time, width) -> np.ndarray:
    out = np.empty(width, np.float32)
    lib().orc_sinusoid(float(time), width, out)
    return out


def modulate(x, shift, scale, eps=1e-6) -> np.ndarray:
    x = _f32(x)
    W = x.shape[-1]
    sh = None if shift is None else _f32(shift)
    y = np.empty_like(x)
    lib().orc_modulate(x, x.size // W, W, _ptr(sh), _f32(scale), eps, _ptr(y))
    return y


def group_norm(x, groups, weight=None, bias=None, eps=1e-5, silu=False) -> np.ndarray:
    x = _f32(x)
    n, c = x.shape[0], x.shape[1]
    hw = x.size // (n * c)
    w = None if weight is None else _f32(weight)
    b = None if bias is None else _f32(bias)
    y = np.empty_like(x)
    lib().orc_group_norm(x, n, c, hw, groups, _ptr(w), _ptr(b), eps, int(silu), _ptr(y))
    return y


def conv2d(x, w, bias=None, stride=1, pad=1, pad_end=None) -> np.ndarray:
    x, w = _f32(x), _f32(w)
    pad_end = pad if pad_end is None else pad_end
    n, cin, h, wd = x.shape
    cout, _, kh, kw = w.shape
    ho = (h + pad + pad_end - kh) // stride + 1
    wo = (wd + pad + pad_end - kw) // stride + 1
    b = None if bias is None else _f32(bias)
    y = np.empty((n, cout, ho, wo), np.float32)
    lib().orc_conv2d(x, n, cin, h, wd, w, cout, kh, kw, _ptr(b), stride, pad, pad_end, _ptr(y))
    return y


def upsample_nearest(x, scale=2) -> np.ndarray:
    x = _f32(x)
    n, c, h, w = x.shape
    y = np.empty((n, c, h * scale, w * scale), np.float32)
    lib().orc_upsample_nearest(x, n, c, h, w, scale, _ptr(y))
    return y


# ---- BlockQuantizer ------------------------------------------------------------

def quantize(w, rows, block=32, fp16_scales=True):
    """BlockQuantizer.Quantize: returns (q int8 [rows, cols], scales uint16
    fp16 bits or float32 [rows, cols/block])."""
    w = _f32(w).reshape(rows, -1)
    cols = w.shape[1]
    q = np.empty((rows, cols), np.int8)
    s = np.empty((rows, cols // block), np.uint16 if fp16_scales else np.float32)
    rc = lib().orc_quantize(w, rows, cols, block, int(fp16_scales), _ptr(q), _ptr(s))
    if rc != 0:
        raise ValueError(f"{w.size} elements in {rows} rows do not split into blocks of {block}")
    return q, s


def quantization_loss(w, rows, block=32):
    w = _f32(w).reshape(rows, -1)
    e, g = ctypes.c_double(), ctypes.c_double()
    lib().orc_quantization_loss(w, rows, w.shape[1], block, ctypes.byref(e), ctypes.byref(g))
    return e.value, g.value


# ---- Qwen-Image inputs ------------------------------------------------------------

def qwen_rope_tables(rows, cols, text_length, context_rows):
    n = rows * cols + context_rows
    c = np.empty((n, 64), np.float32)
    s = np.empty((n, 64), np.float32)
    lib().orc_qwen_rope_tables(rows, cols, text_length, context_rows, c, s)
    return c, s


def mmdit_rope_tables(rows, cols, text_rows):
    n = rows * cols + text_rows
    c = np.empty((n, 64), np.float32)
    s = np.empty((n, 64), np.float32)
    lib().orc_mmdit_rope_tables(rows, cols, text_rows, c, s)
    return c, s


def causal_table(real, rows) -> np.ndarray:
    out = np.empty(rows * rows, np.int32)
    lib().orc_causal_table(real, rows, out)
    return out


# ---- the MMDiT block -------------------------------------------------------------

class _Stream(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in (
        "w_mod", "b_mod", "w_qkv", "b_qkv", "norm_q", "norm_k", "w_o", "b_o", "w_fc1", "b_fc1", "w_fc2", "b_fc2")]


STREAM_KEYS = ("w_mod", "b_mod", "w_qkv", "b_qkv", "norm_q", "norm_k", "w_o", "b_o", "w_fc1", "b_fc1", "w_fc2",
               "b_fc2")


def mmdit_block(x_img, x_txt, temb, img: dict, txt: dict, heads, cos, sin, key_len=-1, eps=1e-6):
    """The dual-stream joint block (oracle.c orc_mmdit_block). img and txt
    map STREAM_KEYS to fp32 arrays. Returns updated (x_img, x_txt)."""
    xi, xt = _f32(x_img).copy(), _f32(x_txt).copy()
    D = xi.shape[-1]
    F = img["w_fc1"].shape[0]
    keep = []

    def stream(p):
        arrs = {k: _f32(p[k]) for k in STREAM_KEYS}
        keep.append(arrs)
        return _Stream(*[arrs[k].ctypes.data for k in STREAM_KEYS])

    si, stx = stream(img), stream(txt)
    t = _f32(temb)
    lib().orc_mmdit_block(_ptr(xi), xi.shape[0], _ptr(xt), xt.shape[0], t, t.size, D, heads, F,
                          ctypes.byref(si), ctypes.byref(stx), _f32(cos), _f32(sin), key_len, eps)
    return xi, xt
