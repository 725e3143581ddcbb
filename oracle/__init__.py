"""The oracle: ctypes access to oracle/liboracle.so, the plain-C restatement
of NaiveDiffusion's CPU layer math (Tensors/CpuMath.cs), its int8 block
quantiser (Tensors/BlockQuantizer.cs), the Transformer helpers
(Graph/Transformer.cs) and the DirectML operator semantics the graphs use.

TEST INFRASTRUCTURE ONLY: imported by tests/ and by __graft_entry__.smoke()
to check the GPU's results against, and by bench.py for the CPU baseline. The
product (naivediffusion_amd) never imports it.

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
        L.orc_lora_merge.argtypes = [_f32p, c_i64, c_i64, _f32p, _f32p, c_int, c_float, c_i64, c_i64]
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
        L.orc_anima_rope_tables.argtypes = [c_int, c_int, c_int, _f32p, _f32p]
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


# ---- Anima (Models/Anima/AnimaDit.cs) ------------------------------------------------

def anima_rope_tables(rows, cols, head_dim=128):
    """AnimaDit.RopeTables (oracle.c orc_anima_rope_tables): [rows*cols, head_dim/2]."""
    c = np.empty((rows * cols, head_dim // 2), np.float32)
    s = np.empty((rows * cols, head_dim // 2), np.float32)
    lib().orc_anima_rope_tables(rows, cols, head_dim, c, s)
    return c, s


def anima_patchify(latent, patch=2):
    """AnimaDit.Patchify, AnimaDit.cs:193-219: [C, H, W] -> [tokens, C*p*p],
    patch (i, j) feature c*p*p + m*p + n = channel c at (p*i + m, p*j + n)."""
    x = _f32(latent)
    C, H, W = x.shape
    out = np.empty(((H // patch) * (W // patch), C * patch * patch), np.float32)
    for i in range(H // patch):
        for j in range(W // patch):
            for c in range(C):
                for m in range(patch):
                    for n in range(patch):
                        out[i * (W // patch) + j, c * patch * patch + m * patch + n] = x[c, i * patch + m, j * patch + n]
    return out


def anima_unpatchify(tokens, channels, height, width, patch=2):
    """AnimaDit.Unpatchify, AnimaDit.cs:223-247: feature (p1*p + p2)*C + c is
    channel c at (p*i + p1, p*j + p2)."""
    t = _f32(tokens)
    out = np.empty((channels, height, width), np.float32)
    cols = width // patch
    for i in range(height // patch):
        for j in range(cols):
            for p1 in range(patch):
                for p2 in range(patch):
                    for c in range(channels):
                        out[c, i * patch + p1, j * patch + p2] = t[i * cols + j, (p1 * patch + p2) * channels + c]
    return out


def anima_modulation(temb, lora, w1, w2, chunks, width):
    """AnimaDit.Modulation, AnimaDit.cs:270-291: Linear(Linear(SiLU(temb),
    W1), W2) + the shared term (its first chunks * width entries), cut into
    `chunks` rows of the model width."""
    h = silu(_f32(temb).reshape(1, -1))
    m = linear(linear(h, w1), w2)[0] + _f32(lora).reshape(-1)[: chunks * width]
    return [m[i * width:(i + 1) * width] for i in range(chunks)]


def anima_attention(x, source, w: dict, prefix, heads, cos=None, sin=None, eps=1e-6):
    """AnimaDit.Attention, AnimaDit.cs:295-323: q, k per-head RMS-normed
    (rotated when tables are given), v plain, Attend, the output projection.
    No biases."""
    D = x.shape[-1]
    d = D // heads
    q = linear(x, w[f"{prefix}.q_proj.weight"])
    k = linear(source, w[f"{prefix}.k_proj.weight"])
    v = linear(source, w[f"{prefix}.v_proj.weight"])
    q = rms_norm(q.reshape(-1, d), w[f"{prefix}.q_norm.weight"], eps).reshape(q.shape)
    k = rms_norm(k.reshape(-1, d), w[f"{prefix}.k_norm.weight"], eps).reshape(k.shape)
    if cos is not None:
        q = rope(q, heads, cos, sin)
        k = rope(k, heads, cos, sin)
    a = mha(q[None], k[None], v[None], heads)[0]
    return linear(a, w[f"{prefix}.output_proj.weight"])


def anima_block(x, temb, lora, context, w: dict, i, heads, cos, sin, eps=1e-6):
    """AnimaDit.Block, AnimaDit.cs:325-358, on the fp32 residual x [N, D]:
    self-attention with rotary positions, cross-attention into the context,
    exact-GELU MLP, each modulated and gated by its low-rank adaLN."""
    D = x.shape[-1]
    p = f"blocks.{i}"
    x = _f32(x).copy()
    mods = {}
    for part in ("self_attn", "cross_attn", "mlp"):
        q = f"{p}.adaln_modulation_{part}"
        mods[part] = anima_modulation(temb, lora, w[f"{q}.1.weight"], w[f"{q}.2.weight"], 3, D)
    sh, sc, g = mods["self_attn"]
    h = modulate(x, sh, sc, eps)
    x = x + g * anima_attention(h, h, w, f"{p}.self_attn", heads, cos, sin, eps)
    sh, sc, g = mods["cross_attn"]
    h = modulate(x, sh, sc, eps)
    x = x + g * anima_attention(h, _f32(context), w, f"{p}.cross_attn", heads, None, None, eps)
    sh, sc, g = mods["mlp"]
    h = modulate(x, sh, sc, eps)
    f = gelu(linear(h, w[f"{p}.mlp.layer1.weight"]))
    return x + g * linear(f, w[f"{p}.mlp.layer2.weight"])


def anima_step(latent, sigma, context, w: dict, blocks, heads, eps=1e-6, patch=2):
    """AnimaDit.Predict + Build, AnimaDit.cs:120-132 and :360-404: patchify,
    embed (the 16 real channels' columns), the time embedding (RMS-normed
    sinusoid; the shared adaLN term through t_embedder), the blocks, the
    final modulated projection, unpatchify. latent [C, H, W] -> flow [C, H, W]."""
    C, H, W = latent.shape
    D = w["x_embedder.proj.1.weight"].shape[0]
    kept = C * patch * patch
    tokens = anima_patchify(latent, patch)
    x = linear(tokens, np.ascontiguousarray(w["x_embedder.proj.1.weight"][:, :kept]))
    time = sinusoid(float(sigma), D).reshape(1, D)
    temb = rms_norm(time, w["t_embedding_norm.weight"], eps)
    lora = linear(silu(linear(time, w["t_embedder.1.linear_1.weight"])), w["t_embedder.1.linear_2.weight"])
    cos, sin = anima_rope_tables(H // patch, W // patch, D // heads)
    for i in range(blocks):
        x = anima_block(x, temb, lora, context, w, i, heads, cos, sin, eps)
    sh, sc = anima_modulation(temb, lora, w["final_layer.adaln_modulation.1.weight"],
                              w["final_layer.adaln_modulation.2.weight"], 2, D)
    out = linear(modulate(x, sh, sc, eps), w["final_layer.linear.weight"])
    return anima_unpatchify(out, C, H, W, patch)


# ---- SDXL's UNet (Models/Sdxl/UNetModel.cs, UNetLayers.cs) ----------------------------

def sdxl_resnet(x, silu_temb, w: dict, p: str, groups=32, eps=1e-5):
    """UNetModel.ResnetBlock, UNetModel.cs:230-254. x [B, C, H, W];
    silu_temb [B, T] (SiLU of the time embedding)."""
    x = _f32(x)
    h = group_norm(x, groups, w[f"{p}.norm1.weight"], w[f"{p}.norm1.bias"], eps, silu=True)
    h = conv2d(h, w[f"{p}.conv1.weight"], w[f"{p}.conv1.bias"], 1, 1)
    proj = linear(silu_temb, w[f"{p}.time_emb_proj.weight"], w[f"{p}.time_emb_proj.bias"])
    h = h + proj.reshape(h.shape[0], h.shape[1], 1, 1)
    h = group_norm(h, groups, w[f"{p}.norm2.weight"], w[f"{p}.norm2.bias"], eps, silu=True)
    h = conv2d(h, w[f"{p}.conv2.weight"], w[f"{p}.conv2.bias"], 1, 1)
    if f"{p}.conv_shortcut.weight" in w:
        x = conv2d(x, w[f"{p}.conv_shortcut.weight"], w[f"{p}.conv_shortcut.bias"], 1, 0)
    return x + h


def sdxl_transformer_block(x, context, w: dict, p: str, heads, eps=1e-5):
    """UNetModel.TransformerBlock, UNetModel.cs:258-276, with
    UNetLayers.DiffusersAttention (:14-26) and Geglu (:30-47). x [B, N, C],
    context [B, Nc, Cw]."""
    x = _f32(x)

    def attend(h, src, a):
        q = linear(h, w[f"{p}.{a}.to_q.weight"])
        k = linear(src, w[f"{p}.{a}.to_k.weight"])
        v = linear(src, w[f"{p}.{a}.to_v.weight"])
        return linear(mha(q, k, v, heads), w[f"{p}.{a}.to_out.0.weight"], w[f"{p}.{a}.to_out.0.bias"])

    h = layer_norm(x, w[f"{p}.norm1.weight"], w[f"{p}.norm1.bias"], eps)
    x = x + attend(h, h, "attn1")
    h = layer_norm(x, w[f"{p}.norm2.weight"], w[f"{p}.norm2.bias"], eps)
    x = x + attend(h, _f32(context), "attn2")
    h = layer_norm(x, w[f"{p}.norm3.weight"], w[f"{p}.norm3.bias"], eps)
    proj = linear(h, w[f"{p}.ff.net.0.proj.weight"], w[f"{p}.ff.net.0.proj.bias"])
    inner = proj.shape[-1] // 2
    gated = proj[..., :inner] * gelu(np.ascontiguousarray(proj[..., inner:]))
    return x + linear(gated, w[f"{p}.ff.net.2.weight"], w[f"{p}.ff.net.2.bias"])


def sdxl_transformer2d(x, context, w: dict, p: str, heads, layers, groups=32, eps=1e-6, ln_eps=1e-5):
    """UNetModel.Transformer2d, UNetModel.cs:279-301. x [B, C, H, W]."""
    x = _f32(x)
    B, C, H, W = x.shape
    n = group_norm(x, groups, w[f"{p}.norm.weight"], w[f"{p}.norm.bias"], eps)
    t = linear(n.reshape(B, C, H * W).transpose(0, 2, 1), w[f"{p}.proj_in.weight"], w[f"{p}.proj_in.bias"])
    for j in range(layers):
        t = sdxl_transformer_block(t, context, w, f"{p}.transformer_blocks.{j}", heads, ln_eps)
    t = linear(t, w[f"{p}.proj_out.weight"], w[f"{p}.proj_out.bias"])
    return t.transpose(0, 2, 1).reshape(B, C, H, W) + x


def sdxl_unet(sample, time, add, context, w: dict, cfg):
    """UNetModel.Build, UNetModel.cs:328-426, in fp32. sample [B, 4, h, w],
    time [B, c0], add [B, add_width], context [B, tokens, Cw]; cfg carries
    block_out, layers_per_block, transformer_layers, heads, groups, eps,
    transformer_eps, layer_norm_eps."""
    def mlp(x, prefix):
        h = silu(linear(x, w[f"{prefix}.linear_1.weight"], w[f"{prefix}.linear_1.bias"]))
        return linear(h, w[f"{prefix}.linear_2.weight"], w[f"{prefix}.linear_2.bias"])

    def unit(x, prefix, index, level):
        x = sdxl_resnet(x, st, w, f"{prefix}.resnets.{index}", cfg.groups, cfg.eps)
        if cfg.transformer_layers[level]:
            x = sdxl_transformer2d(x, context, w, f"{prefix}.attentions.{index}", cfg.heads[level],
                                   cfg.transformer_layers[level], cfg.groups, cfg.transformer_eps, cfg.layer_norm_eps)
        return x

    st = silu(mlp(time, "time_embedding") + mlp(add, "add_embedding"))
    skips = [conv2d(sample, w["conv_in.weight"], w["conv_in.bias"], 1, 1)]
    levels = len(cfg.block_out)
    for level in range(levels):
        prefix = f"down_blocks.{level}"
        for i in range(cfg.layers_per_block):
            skips.append(unit(skips[-1], prefix, i, level))
        if level != levels - 1:
            skips.append(conv2d(skips[-1], w[f"{prefix}.downsamplers.0.conv.weight"],
                                w[f"{prefix}.downsamplers.0.conv.bias"], 2, 1))
    x = sdxl_resnet(skips[-1], st, w, "mid_block.resnets.0", cfg.groups, cfg.eps)
    x = sdxl_transformer2d(x, context, w, "mid_block.attentions.0", cfg.heads[-1], cfg.transformer_layers[-1],
                           cfg.groups, cfg.transformer_eps, cfg.layer_norm_eps)
    x = sdxl_resnet(x, st, w, "mid_block.resnets.1", cfg.groups, cfg.eps)
    for i in range(levels):
        level = levels - 1 - i
        prefix = f"up_blocks.{i}"
        for j in range(cfg.layers_per_block + 1):
            x = np.concatenate([x, skips.pop()], axis=1)
            x = unit(x, prefix, j, level)
        if i != levels - 1:
            nxt = skips[-1].shape
            up = upsample_nearest(x, 2)[:, :, :nxt[2], :nxt[3]]
            x = conv2d(up, w[f"{prefix}.upsamplers.0.conv.weight"], w[f"{prefix}.upsamplers.0.conv.bias"], 1, 1)
    x = group_norm(x, cfg.groups, w["conv_norm_out.weight"], w["conv_norm_out.bias"], cfg.eps, silu=True)
    return conv2d(x, w["conv_out.weight"], w["conv_out.bias"], 1, 1)


# ---- Qwen-Image 2.1 (Models/QwenImage/QwenImageDit.cs) -------------------------------

def qwen_pairs_to_halves(w, head_dim):
    """QwenImageDit.PairsToHalves, QwenImageDit.cs:277-292, row by row: row r
    = (head, feature) takes source row head*d + 2f (f < d/2) or
    head*d + 2(f - d/2) + 1 (f >= d/2); a vector is one column."""
    w = _f32(w)
    rows = w.shape[0]
    half = head_dim // 2
    out = np.empty_like(w)
    for r in range(rows):
        head, f = divmod(r, head_dim)
        src = head * head_dim + (2 * f if f < half else 2 * (f - half) + 1)
        out[r] = w[src]
    return out


def qwen_block(x, mod, w: dict, i, heads, n_img, cos, sin, key_len, text_mask, eps=1e-6):
    """QwenImageDit.Block + Attention + FeedForward, QwenImageDit.cs:336-428,
    on the fp32 residual x [N, D] (image rows first). mod [2, 4D]: the
    shared modulation's noise-level and time-zero rows (scale1, tanh gate1,
    scale2, tanh gate2), read by the image and the text rows (Rows, :307-315).
    The query and key projections and norms go through PairsToHalves and are
    rotated in halves (Transformer.Rotate); the image rows attend over every
    key under the key length, the text rows over the text keys under the
    causal table; the feed-forward is SiLU(gate) * up of the fused gate_up
    (gate rows first)."""
    x = _f32(x).copy()
    mod = _f32(mod)
    D = x.shape[1]
    d = D // heads
    p = f"transformer_blocks.{i}"

    def mod_rows(c, t):
        return np.concatenate([modulate(t[:n_img], None, mod[0, c * D:(c + 1) * D], eps),
                               modulate(t[n_img:], None, mod[1, c * D:(c + 1) * D], eps)])

    def gate_rows(c):
        return np.concatenate([np.broadcast_to(mod[0, c * D:(c + 1) * D], (n_img, D)),
                               np.broadcast_to(mod[1, c * D:(c + 1) * D], (x.shape[0] - n_img, D))])

    h = mod_rows(0, x)
    q = linear(h, qwen_pairs_to_halves(w[f"{p}.attn.to_q.weight"], d))
    k = linear(h, qwen_pairs_to_halves(w[f"{p}.attn.to_k.weight"], d))
    v = linear(h, w[f"{p}.attn.to_v.weight"])
    q = rms_norm(q.reshape(-1, d), qwen_pairs_to_halves(w[f"{p}.attn.norm_q.weight"], d), eps).reshape(q.shape)
    k = rms_norm(k.reshape(-1, d), qwen_pairs_to_halves(w[f"{p}.attn.norm_k.weight"], d), eps).reshape(k.shape)
    q = rope(q, heads, cos, sin)
    k = rope(k, heads, cos, sin)
    image = mha(q[None, :n_img], k[None], v[None], heads, mask_kind=1, key_len=int(key_len))[0]
    text = mha(q[None, n_img:], k[None, n_img:], v[None, n_img:], heads, mask_kind=2,
               mask=np.asarray(text_mask, np.int32))[0]
    a = np.concatenate([image, text])
    x = x + gate_rows(1) * linear(a, w[f"{p}.attn.to_out.0.weight"])
    h = mod_rows(2, x)
    gu = linear(h, w[f"{p}.img_mlp.gate_up.weight"])
    F = gu.shape[1] // 2
    f = silu(gu[:, :F]) * gu[:, F:]
    return x + gate_rows(3) * linear(f, w[f"{p}.img_mlp.out.weight"])


def qwen_modulation(sigma, w: dict, time_dim, width):
    """The time path, QwenImageDit.cs:464-478 with Predict :152-166: temb [2,
    D] of Sinusoid(1000 sigma) and Sinusoid(0); the modulation [2, 4D] with
    chunks 1 and 3 through tanh."""
    time = np.stack([sinusoid(np.float32(sigma * 1000.0), time_dim), sinusoid(0.0, time_dim)])
    temb = linear(silu(linear(time, w["time_text_embed.timestep_embedder.linear_1.weight"])),
                  w["time_text_embed.timestep_embedder.linear_2.weight"])
    mod = linear(silu(temb), w["modulation.1.weight"])
    D = width
    mod[:, D:2 * D] = tanh(mod[:, D:2 * D])
    mod[:, 3 * D:4 * D] = tanh(mod[:, 3 * D:4 * D])
    return temb, mod


def qwen_step(latent, sigma, context, text_mask, key_len, w: dict, blocks, heads, cos, sin, time_dim=256, eps=1e-6):
    """QwenImageDit.Build + Predict, QwenImageDit.cs:152-166, 430-505: the
    latent's cells (ToTokens, patch 1) through img_in; the padded context
    through the zero-centred RMS norm (stored weight + 1) and in_layer,
    GELU-tanh, out_layer; the blocks; the final modulated projection of the
    image rows. latent [C, H, W] -> flow [C, H, W]."""
    C, H, W = latent.shape
    n_img = H * W
    D = w["img_in.weight"].shape[0]
    image = linear(_f32(latent).reshape(C, n_img).T, w["img_in.weight"])
    text = rms_norm(context, _f32(w["txt_in.text_norm.weight"]) + np.float32(1.0), eps)
    text = linear(gelu_tanh(linear(text, w["txt_in.in_layer.weight"])), w["txt_in.out_layer.weight"])
    x = np.concatenate([image, text])
    temb, mod = qwen_modulation(sigma, w, time_dim, D)
    for i in range(blocks):
        x = qwen_block(x, mod, w, i, heads, n_img, cos, sin, key_len, text_mask, eps)
    scale = linear(silu(temb[:1]), w["norm_out.linear.weight"])[0]
    out = linear(modulate(x[:n_img], None, scale, eps), w["proj_out.weight"])
    return out.T.reshape(C, H, W)


# ---- the sampler around the denoiser (Pipeline/, Sampling/) ----------------------------

def cfg_combine(uncond, cond, guidance):
    """ClassifierFreeGuidance.Combine, Pipeline/GuidanceStrategy.cs:34-44:
    uncond + g * (cond - uncond), every operation in float32."""
    u, c = _f32(uncond), _f32(cond)
    return (u + np.float32(guidance) * (c - u)).astype(np.float32)


def euler_step(sample, prediction, sigma, sigma_next):
    """EulerScheduler.Step, Sampling/Schedulers.cs:270-279, with the flow
    prediction's derivative (the model output, Prediction.cs:83-84): sample +
    derivative * (sigma_next - sigma), the difference taken in float32 as the
    float[] sigmas give it."""
    delta = np.float32(np.float32(sigma_next) - np.float32(sigma))
    return (_f32(sample) + _f32(prediction) * delta).astype(np.float32)


def mmdit_step(latent, text, t, w: dict, blocks, heads, cos, sin, patch=2, eps=1e-6):
    """The dual-stream MMDiT denoiser step composed from the primitives above
    in the order of QwenImageDit's Build (QwenImageDit.cs:430-505): 2x2
    patchify and img_in, the RMS-normed text through txt_in, the time MLP on
    Sinusoid(1000 t), the blocks, the final layer (scale, shift) and
    unpatchify. latent [1, C, H, W], text [Nt, text_dim]; weights by the
    build's names (blocks.{i}.{img,txt}_*)."""
    _, C, H, W = latent.shape
    D = w["img_in.weight"].shape[0]
    p = patch
    tokens = _f32(latent)[0].reshape(C, H // p, p, W // p, p).transpose(1, 3, 0, 2, 4).reshape(-1, C * p * p)
    x_img = linear(tokens, w["img_in.weight"], w["img_in.bias"])
    x_txt = linear(rms_norm(_f32(text).reshape(-1, w["txt_in.weight"].shape[1]), w["txt_norm.weight"], eps),
                   w["txt_in.weight"], w["txt_in.bias"])
    ts = sinusoid(np.float32(t * 1000.0), w["time.linear_1.weight"].shape[1])
    temb = linear(silu(linear(ts, w["time.linear_1.weight"], w["time.linear_1.bias"])), w["time.linear_2.weight"],
                  w["time.linear_2.bias"])

    def stream(i, s):
        q = f"blocks.{i}.{s}"
        return dict(w_mod=w[f"{q}_mod.weight"], b_mod=w[f"{q}_mod.bias"], w_qkv=w[f"{q}_qkv.weight"],
                    b_qkv=w[f"{q}_qkv.bias"], norm_q=w[f"{q}_norm_q.weight"], norm_k=w[f"{q}_norm_k.weight"],
                    w_o=w[f"{q}_out.weight"], b_o=w[f"{q}_out.bias"], w_fc1=w[f"{q}_fc1.weight"],
                    b_fc1=w[f"{q}_fc1.bias"], w_fc2=w[f"{q}_fc2.weight"], b_fc2=w[f"{q}_fc2.bias"])

    for i in range(blocks):
        x_img, x_txt = mmdit_block(x_img, x_txt, temb, stream(i, "img"), stream(i, "txt"), heads, cos, sin, -1, eps)
    mod = linear(silu(temb), w["norm_out.weight"], w["norm_out.bias"])
    y = modulate(x_img, mod[D:], mod[:D], eps)
    out = linear(y, w["proj_out.weight"], w["proj_out.bias"])
    return out.reshape(H // p, W // p, C, p, p).transpose(2, 0, 3, 1, 4).reshape(1, C, H, W)


def lora_scale(weight, alpha, rank) -> float:
    """The pair's factor weight * (alpha or rank) / rank in float32, left to
    right (LoraPatchSet.Prepare, Weights/LoraFile.cs:492)."""
    a = np.float32(rank if alpha is None else alpha)
    return float(np.float32(np.float32(np.float32(weight) * a) / np.float32(rank)))


def lora_merge(weight, patches):
    """LoraMerge.Merge (Weights/LoraFile.cs:362-420) through orc_lora_merge:
    weight is float32 values (a float16 / bfloat16 weight widened exactly),
    patches a list of (down [rank, cols], up [count, rank], scale, first_row).
    Returns the merged rows in float32 before narrowing; narrow with
    f32_to_f16_bits / f32_to_bf16_bits as the reference's width asks."""
    w = np.array(weight, np.float32, copy=True)
    rows = w.shape[0]
    flat = np.ascontiguousarray(w.reshape(rows, -1))
    cols = flat.shape[1]
    for down, up, scale, first in patches:
        down = _f32(np.asarray(down).reshape(-1, cols))
        rank = down.shape[0]
        up = _f32(np.asarray(up).reshape(-1, rank))
        lib().orc_lora_merge(flat, rows, cols, down, up, rank, float(np.float32(scale)), int(first), up.shape[0])
    return flat.reshape(w.shape)


# ---- AutoencoderKL (Vae/AutoencoderKl.cs) ------------------------------------------

def vae_resnet(x, w: dict, p: str, groups=32, eps=1e-6):
    """AutoencoderKl.ResnetBlock (:16-35): GroupNorm-SiLU-conv twice, plus the
    input (1x1-projected when the width changes)."""
    x = _f32(x)
    h = conv2d(group_norm(x, groups, w[f"{p}.norm1.weight"], w[f"{p}.norm1.bias"], eps, silu=True),
               w[f"{p}.conv1.weight"], w[f"{p}.conv1.bias"], 1, 1)
    h = conv2d(group_norm(h, groups, w[f"{p}.norm2.weight"], w[f"{p}.norm2.bias"], eps, silu=True),
               w[f"{p}.conv2.weight"], w[f"{p}.conv2.bias"], 1, 1)
    if f"{p}.conv_shortcut.weight" in w:
        x = conv2d(x, w[f"{p}.conv_shortcut.weight"], w[f"{p}.conv_shortcut.bias"], 1, 0)
    return x + h


def vae_attention(x, w: dict, p: str, groups=32, eps=1e-6):
    """AutoencoderKl.AttentionBlock (:40-63): single-head self-attention over
    every pixel, softmax(q k^T / sqrt(C)) v, projected, plus the input."""
    x = _f32(x)
    n, c, h, wd = x.shape
    t = group_norm(x, groups, w[f"{p}.group_norm.weight"], w[f"{p}.group_norm.bias"], eps)
    t = np.ascontiguousarray(t.reshape(n, c, h * wd).transpose(0, 2, 1))
    q = linear(t, w[f"{p}.to_q.weight"], w[f"{p}.to_q.bias"])
    k = linear(t, w[f"{p}.to_k.weight"], w[f"{p}.to_k.bias"])
    v = linear(t, w[f"{p}.to_v.weight"], w[f"{p}.to_v.bias"])
    a = mha(q, k, v, 1, scale=float(np.float32(1.0) / np.sqrt(np.float32(c))))
    o = linear(a, w[f"{p}.to_out.0.weight"], w[f"{p}.to_out.0.bias"])
    return o.transpose(0, 2, 1).reshape(n, c, h, wd) + x


def vae_decoder(latent, w: dict, block_out, layers_per_block=2, groups=32, eps=1e-6):
    """AutoencoderKl.Decoder (:72-112) in fp32: latent [1, C, h, w] already
    in the VAE's scale (LatentSpace.FromModelScale done) -> image [1, 3, H, W]."""
    h = conv2d(latent, w["post_quant_conv.weight"], w["post_quant_conv.bias"], 1, 0)
    h = conv2d(h, w["decoder.conv_in.weight"], w["decoder.conv_in.bias"], 1, 1)
    h = vae_resnet(h, w, "decoder.mid_block.resnets.0", groups, eps)
    h = vae_attention(h, w, "decoder.mid_block.attentions.0", groups, eps)
    h = vae_resnet(h, w, "decoder.mid_block.resnets.1", groups, eps)
    for i in range(len(block_out)):
        p = f"decoder.up_blocks.{i}"
        for j in range(layers_per_block + 1):
            h = vae_resnet(h, w, f"{p}.resnets.{j}", groups, eps)
        if f"{p}.upsamplers.0.conv.weight" in w:
            h = conv2d(upsample_nearest(h), w[f"{p}.upsamplers.0.conv.weight"], w[f"{p}.upsamplers.0.conv.bias"], 1, 1)
    h = group_norm(h, groups, w["decoder.conv_norm_out.weight"], w["decoder.conv_norm_out.bias"], eps, silu=True)
    return conv2d(h, w["decoder.conv_out.weight"], w["decoder.conv_out.bias"], 1, 1)


# ---- Wan 2.2's VAE on one frame (Vae/Wan22Vae.cs, Vae/WanVae.cs) ------------------------------

def wan_channel_rms(x, gamma):
    """WanVae.ChannelRmsNorm (:103-113): per pixel, x / sqrt(mean over the
    channels of x^2 + 1e-24 / C) * gamma. x [1, C, H, W]."""
    x = _f32(x)
    n, c, h, w = x.shape
    t = np.ascontiguousarray(x.reshape(c, h * w).T)
    y = rms_norm(t, gamma, float(np.float32(1e-24 / c)))
    return np.ascontiguousarray(y.T.reshape(n, c, h, w))


def wan_residual(x, w: dict, p: str):
    """WanVae.ResidualBlock (:121-132)."""
    x = _f32(x)
    h = conv2d(silu(wan_channel_rms(x, w[f"{p}.residual.0.gamma"])), w[f"{p}.residual.2.weight"],
               w[f"{p}.residual.2.bias"], 1, 1)
    h = conv2d(silu(wan_channel_rms(h, w[f"{p}.residual.3.gamma"])), w[f"{p}.residual.6.weight"],
               w[f"{p}.residual.6.bias"], 1, 1)
    if f"{p}.shortcut.weight" in w:
        x = conv2d(x, w[f"{p}.shortcut.weight"], w[f"{p}.shortcut.bias"], 1, 0)
    return x + h


def wan_attention(x, w: dict, p: str):
    """WanVae.AttentionBlock (:134-151): one head of C features over every
    pixel; the 1x1 projections as products over the pixels' rows."""
    x = _f32(x)
    n, c, h, wd = x.shape
    t = np.ascontiguousarray(wan_channel_rms(x, w[f"{p}.norm.gamma"]).reshape(c, h * wd).T)
    qkv = linear(t, np.asarray(w[f"{p}.to_qkv.weight"]).reshape(3 * c, c), w[f"{p}.to_qkv.bias"])
    q, k, v = (np.ascontiguousarray(qkv[:, i * c:(i + 1) * c]) for i in range(3))
    a = mha(q, k, v, 1, scale=float(np.float32(1.0) / np.sqrt(np.float32(c))))
    o = linear(a, np.asarray(w[f"{p}.proj.weight"]).reshape(c, c), w[f"{p}.proj.bias"])
    return np.ascontiguousarray(o.reshape(h * wd, c).T.reshape(n, c, h, wd)) + x


def wan_up_shortcut(x, out_channels, temporal):
    """Wan22Vae.UpShortcut (:153-189) by indexing: the same width is a
    nearest upsample; half the width is the odd channels upsampled (a level
    that doubled time), else out[o, 2y + r, 2x + s] = x[2o + r, y, x]."""
    x = _f32(x)
    n, c, h, w = x.shape
    if c == out_channels:
        return upsample_nearest(x)
    if temporal:
        return upsample_nearest(np.ascontiguousarray(x[:, 1::2]))
    out = np.empty((n, out_channels, 2 * h, 2 * w), np.float32)
    for r in range(2):
        out[:, :, r::2, :] = np.repeat(x[:, r::2], 2, axis=3)
    return out


def wan22_decoder(z, w: dict, temporal=(False, True, True, True)):
    """Wan22Vae.Decoder (:191-238) in fp32: z [1, 64, h, w] already on the
    VAE's scale -> RGB [1, 3, 16h, 16w]."""
    h = conv2d(z, w["conv2.weight"], w["conv2.bias"], 1, 0)
    h = conv2d(h, w["decoder.conv1.weight"], w["decoder.conv1.bias"], 1, 1)
    h = wan_residual(h, w, "decoder.middle.0")
    h = wan_attention(h, w, "decoder.middle.1")
    h = wan_residual(h, w, "decoder.middle.2")
    levels = 0
    while f"decoder.upsamples.{levels}.upsamples.0.residual.0.gamma" in w:
        levels += 1
    for level in range(levels):
        p = f"decoder.upsamples.{level}.upsamples"
        level_in = h
        i = 0
        while f"{p}.{i}.residual.0.gamma" in w:
            h = wan_residual(h, w, f"{p}.{i}")
            i += 1
        if level != levels - 1:
            h = conv2d(upsample_nearest(h), w[f"{p}.{i}.resample.1.weight"], w[f"{p}.{i}.resample.1.bias"], 1, 1)
            h = h + wan_up_shortcut(level_in, h.shape[1], temporal[levels - 2 - level])
    h = silu(wan_channel_rms(h, w["decoder.head.0.gamma"]))
    return conv2d(h, w["decoder.head.2.weight"], w["decoder.head.2.bias"], 1, 1)[:, :3]
