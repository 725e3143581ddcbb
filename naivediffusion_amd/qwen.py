"""Qwen-Image 2.1's denoiser, the reference's own single-stream DiT
(Models/QwenImage/QwenImageDit.cs): the latent's cells (one token per cell,
patch 1) and the projected text in one sequence, image first, through blocks
of self-attention with three-axis rotary positions and a SwiGLU feed-forward,
modulated and gated by one modulation the whole model shares.

What each block does, as QwenImageDit.cs:336-428 builds it:
- Modulate without a shift; the scale and gate rows are the noise level's row
  for the image tokens and the time-zero row for the text tokens
  (QwenImageDit.Rows, :307-315). Rows() is written as the reference writes it
  (a join of two row broadcasts); the library reads such a join in place.
- Q, K, V projections (one stacked GEMM), Q and K per-head RMS-normed and
  rotated (rotate-half, with the projection rows and norm weights permuted
  from adjacent pairs to halves once, PairsToHalves :277-292).
- The image rows' queries over every key under the count of real keys; the
  text rows' queries over the text keys under the causal table
  (QwenImageConditioner.cs); the two joined and projected out. The reference
  cuts the image queries into 1024-row chunks because a DirectML graph's
  scratch is the sum of its intermediates; one flash-attention launch takes
  them all here.
- SwiGLU (:390-406) as one GEMM whose epilogue forms SiLU(gate) * up from the
  interleaved gate and up rows.
- Both residual adds gated by tanh'd modulation chunks, in fp32.

Precision as the reference's (:41-45): the blocks at the compute type, the
residual stream, norms, rotary positions, embeddings, time path and final
layer fp32.
"""

from __future__ import annotations

import dataclasses
import math
from typing import Dict

import numpy as np

from . import rng
from .graph import CompiledModel, Graph, MaskType, ModelBuilder, Ops
from .layers import Layers, Transformer
from .tensors import Device, DeviceTensor, HostDataType, HostTensor, bf16_to_f32, f32_to_bf16

# QwenImageCheckpoint's names for the feed-forward's first projection
# (Models/QwenImage/QwenImageCheckpoint.cs:32-34).
FUSED_GATE_UP = "img_mlp.gate_up.weight"
GATE_PROJECTION = "img_mlp.gate_layer.weight"
UP_PROJECTION = "img_mlp.proj.weight"

ROPE_AXES = (16, 56, 56)
ROPE_THETA = 10000.0
F32 = HostDataType.Float32


@dataclasses.dataclass(frozen=True)
class QwenImageConfig:
    width: int = 4096            # D
    heads: int = 32              # 32 x 128
    mlp: int = 12288             # F, SwiGLU
    blocks: int = 32
    latent_channels: int = 64    # Wan 2.2's latent, patch 1
    context_width: int = 4096    # Qwen3-VL-8B's hidden width
    time_dim: int = 256
    eps: float = 1e-6

    @property
    def head_dim(self) -> int:
        return self.width // self.heads


def block_weight_shapes(cfg: QwenImageConfig, i: int) -> Dict[str, tuple]:
    D, F, d = cfg.width, cfg.mlp, cfg.head_dim
    p = f"transformer_blocks.{i}"
    return {
        f"{p}.attn.to_q.weight": (D, D), f"{p}.attn.to_k.weight": (D, D), f"{p}.attn.to_v.weight": (D, D),
        f"{p}.attn.norm_q.weight": (d,), f"{p}.attn.norm_k.weight": (d,), f"{p}.attn.to_out.0.weight": (D, D),
        # Fused as Comfy-Org saves it (QwenImageCheckpoint.FusedGateUp): gate rows first, then up.
        f"{p}.img_mlp.gate_up.weight": (2 * F, D), f"{p}.img_mlp.out.weight": (D, F),
    }


def weight_shapes(cfg: QwenImageConfig) -> Dict[str, tuple]:
    """The checkpoint's names (Tests/Fixtures/FakeSafetensors.cs QwenImageDit;
    QwenImageDit.cs:430-505). No linear carries a bias."""
    D, C, T, Cw = cfg.width, cfg.latent_channels, cfg.time_dim, cfg.context_width
    out = {
        "img_in.weight": (D, C),
        "txt_in.text_norm.weight": (Cw,),
        "txt_in.in_layer.weight": (D, Cw),
        "txt_in.out_layer.weight": (D, D),
        "time_text_embed.timestep_embedder.linear_1.weight": (D, T),
        "time_text_embed.timestep_embedder.linear_2.weight": (D, D),
        "modulation.1.weight": (4 * D, D),
        "norm_out.linear.weight": (D, D),
        "proj_out.weight": (C, D),
    }
    for i in range(cfg.blocks):
        out.update(block_weight_shapes(cfg, i))
    return out


def _is_norm(name: str) -> bool:
    return name.endswith("norm_q.weight") or name.endswith("norm_k.weight") or name == "txt_in.text_norm.weight"


def synthetic_weights(cfg: QwenImageConfig, seed: int, names=None, norm_spread: float = 0.0) -> Dict[str, np.ndarray]:
    """Host weights: N(0, 0.02) rounded to bf16; the head norms 1 (+ N(0,
    norm_spread)); the text norm is stored zero-centred (the weight less one,
    QwenImageDit.cs:450-455), so 0 (+ N(0, norm_spread))."""
    shapes = weight_shapes(cfg)
    out = {}
    for name in (names or shapes):
        shape = shapes[name]
        if _is_norm(name):
            v = np.full(shape, 0.0 if name.startswith("txt_in") else 1.0, np.float32)
            if norm_spread:
                v = v + rng.normal(rng.tensor_seed(seed, name), shape, 0.0, norm_spread)
        else:
            v = rng.normal(rng.tensor_seed(seed, name), shape, 0.0, 0.02)
        out[name] = bf16_to_f32(f32_to_bf16(v)).reshape(shape)
    return out


def device_weights(device: Device, cfg: QwenImageConfig, seed: int, dtype: HostDataType = HostDataType.BFloat16,
                   names=None) -> Dict[str, DeviceTensor]:
    """The synthetic weights made on the GPU (norms as synthetic_weights
    makes them with no spread)."""
    shapes = weight_shapes(cfg)
    out = {}
    for name in (names or shapes):
        shape = shapes[name]
        if _is_norm(name):
            v = np.full(shape, 0.0 if name.startswith("txt_in") else 1.0, np.float32)
            out[name] = device.Upload(HostTensor.FromFloats(v).ConvertTo(dtype))
        else:
            out[name] = device.Normal(dtype, shape, rng.tensor_seed(seed, name), 0.0, 0.02)
    return out


# ---- host-side inputs (QwenImageDit.cs:176-240; QwenImageConditioner.cs) ------------------

def time_embedding(time: float, width: int) -> np.ndarray:
    """QwenImageDit.TimeEmbedding (:176-177): Sinusoid(1000 t)."""
    return Transformer.Sinusoid(float(np.float32(time * 1000.0)), width)


def rope_tables(rows: int, cols: int, text_length: int, context_rows: int):
    """QwenImageDit.RopeTables (:189-240): [rows*cols + context_rows, 64]; an
    image cell (i, j) at (text_length, i - ceil(rows/2), j - ceil(cols/2)),
    text row p at (p, p, p), on the {16, 56, 56} axes at theta 10000."""
    freqs = []
    for axis in ROPE_AXES:
        for k in range(axis // 2):
            freqs.append(1.0 / ROPE_THETA ** (2.0 * k / axis))
    freqs = np.array(freqs, np.float64)
    splits = np.cumsum([a // 2 for a in ROPE_AXES])[:-1]
    r0, c0 = rows - rows // 2, cols - cols // 2
    ii, jj = np.meshgrid(np.arange(rows) - r0, np.arange(cols) - c0, indexing="ij")
    n = rows * cols + context_rows
    pos = np.zeros((n, 64), np.float64)
    pos[: rows * cols, : splits[0]] = text_length
    pos[: rows * cols, splits[0]:splits[1]] = ii.reshape(-1, 1)
    pos[: rows * cols, splits[1]:] = jj.reshape(-1, 1)
    pos[rows * cols:, :] = np.arange(context_rows).reshape(-1, 1)
    ang = pos * freqs
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def causal_table(real: int, rows: int) -> np.ndarray:
    """QwenImageConditioning.CausalTable: row i may read key j when j <= i
    and j < real (the triangle closed over the padding)."""
    i, j = np.meshgrid(np.arange(rows), np.arange(rows), indexing="ij")
    return ((j <= i) & (j < real)).astype(np.int32)


def conditioning(context: np.ndarray, rows: int, latent_rows: int, latent_cols: int) -> dict:
    """One branch of QwenImageConditioning: the context padded to `rows`, the
    causal text table, the count of real keys (image tokens + real text
    rows) and the rotary tables with the image at the branch's own text
    length."""
    real, width = context.shape
    padded = np.zeros((rows, width), np.float32)
    padded[:real] = context
    cos, sin = rope_tables(latent_rows, latent_cols, real, rows)
    return {"context": padded, "text_mask": causal_table(real, rows),
            "key_length": np.array([latent_rows * latent_cols + real], np.int32), "cos": cos, "sin": sin}


# ---- weight preparation -------------------------------------------------------------

def _device_view_copy(device: Device, t: DeviceTensor, sizes, strides, out_shape) -> DeviceTensor:
    """A packed copy of a strided view of a device tensor (one small compiled
    copy at build time)."""
    g = Graph(device)
    x = g.Input(t.DataType, list(t.Shape))
    y = Ops.Reinterpret(Ops.Identity(Ops.Reinterpret(x, sizes, strides)), out_shape)
    model = CompiledModel(g, [y], device)
    (res,) = model.DispatchOnDevice([t])
    model.Dispose()
    g.Dispose()
    return res


def pairs_to_halves(w, head_dim: int):
    """QwenImageDit.PairsToHalves (:277-292): within each head, feature rows
    from adjacent pairs (2i, 2i+1) to halves (i, half + i). A [D, K]
    projection or a [d] norm; host array or device tensor."""
    half = head_dim // 2
    if isinstance(w, DeviceTensor):
        return _pairs_device(w, head_dim)
    a = np.asarray(w, np.float32)
    if a.ndim == 1:
        return np.ascontiguousarray(a.reshape(half, 2).T.reshape(-1))
    heads = a.shape[0] // head_dim
    return np.ascontiguousarray(a.reshape(heads, half, 2, -1).transpose(0, 2, 1, 3).reshape(a.shape))


def _pairs_device(w: DeviceTensor, head_dim: int) -> DeviceTensor:
    half = head_dim // 2
    shape = list(w.Shape)
    cols = shape[1] if len(shape) == 2 else 1
    heads = shape[0] // head_dim
    # View [heads, 2, half, cols] of the [heads, half, 2, cols] layout.
    return _device_view_copy(w.Device, w, [heads, 2, half, cols], [head_dim * cols, cols, 2 * cols, 1], shape)


def _gate_up(weights, p: str):
    """The block's [gate; up] projection: the fused matrix as Comfy-Org saves
    it, or diffusers' two matrices stacked (QwenImageDit.FeedForward,
    :390-406)."""
    fused = f"{p}.{FUSED_GATE_UP}"
    if fused in weights:
        return weights[fused]
    return _stack([weights[f"{p}.{GATE_PROJECTION}"], weights[f"{p}.{UP_PROJECTION}"]])


def interleave_gate_up(w):
    """The fused [2F, D] gate-then-up projection with its rows interleaved
    (row 2j the gate's j, row 2j + 1 the up's j): what the SwiGLU epilogue
    reads."""
    if isinstance(w, DeviceTensor):
        F2, D = w.Shape
        F = F2 // 2
        return _device_view_copy(w.Device, w, [F, 2, D], [D, F * D, 1], [F2, D])
    a = np.asarray(w, np.float32)
    F = a.shape[0] // 2
    return np.ascontiguousarray(a.reshape(2, F, -1).transpose(1, 0, 2).reshape(a.shape))


def _stack(ws):
    if all(isinstance(w, DeviceTensor) for w in ws):
        from .weights import device_stack
        return device_stack(ws[0].Device, ws)
    return np.concatenate([np.asarray(w, np.float32) for w in ws], 0)


class _Weights:
    """The model's weights registered once: host arrays or device tensors
    (device tensors handed to the builder are taken over by it)."""

    def __init__(self, model: ModelBuilder, weights: dict, compute: HostDataType):
        self.model, self.weights, self.compute = model, weights, compute
        self.cache = {}
        self.made = []

    def _register(self, key, w, kind):
        m = self.model
        if isinstance(w, DeviceTensor):
            if kind == "weight":
                e = m.WeightOnDevice(w, w.Shape[0])
            else:
                dt = F32 if kind == "wide" else self.compute
                if w.DataType == dt:
                    e = m.ConstantOnDevice(w)
                else:
                    e = m.Constant(w.Download().ConvertTo(dt), [int(np.prod(w.Shape))], dt)
        else:
            arr = np.asarray(w, np.float32)
            if kind == "weight":
                e = m.Weight(HostTensor.FromFloats(arr), arr.shape, arr.shape[0])
            else:
                dt = F32 if kind == "wide" else self.compute
                e = m.Constant(HostTensor.FromFloats(arr), [arr.size], dt)
        self.cache[key] = e
        return e

    def __call__(self, name, kind="weight"):
        if name in self.cache:
            return self.cache[name]
        return self._register(name, self.weights[name], kind)

    def derived(self, key, make, kind="weight"):
        if key in self.cache:
            return self.cache[key]
        w = make()
        if isinstance(w, DeviceTensor):
            self.made.append(w)
        return self._register(key, w, kind)

    def release(self):
        for t in self.made:
            t.Dispose()
        self.made = []


# ---- the graph -----------------------------------------------------------------------

def rows(modulation, chunk: int, D: int, n_img: int, n_txt: int):
    """QwenImageDit.Rows (:307-315): chunk `chunk` of the modulation's noise
    level row over the image tokens, of its time-zero row over the text
    tokens."""
    def row(r, n):
        return Layers.Broadcast(Ops.Slice(modulation, [0, 0, r, chunk * D], [1, 1, 1, D]), [1, 1, n, D])
    return Ops.Join([row(0, n_img), row(1, n_txt)], 2)


def build_block(model: ModelBuilder, W: _Weights, i: int, cfg: QwenImageConfig, x, modulation, cos, sin, key_length,
                text_mask, n_img: int, n_txt: int, compute: HostDataType):
    """One block (QwenImageDit.Block, :411-428) on the fp32 residual x [1, 1,
    N, D]; returns the updated x."""
    D, H, d, eps = cfg.width, cfg.heads, cfg.head_dim, cfg.eps
    N = n_img + n_txt
    p = f"transformer_blocks.{i}"
    normed = Transformer.Modulate(x, rows(modulation, 0, D, n_img, n_txt), eps, compute)
    qkv = Layers.Linear(model, normed, W.derived(f"{p}.qkv", lambda: _stack(
        [pairs_to_halves(W.weights[f"{p}.attn.to_q.weight"], d), pairs_to_halves(W.weights[f"{p}.attn.to_k.weight"], d),
         W.weights[f"{p}.attn.to_v.weight"]])))
    nq = W.derived(f"{p}.norm_q", lambda: pairs_to_halves(W.weights[f"{p}.attn.norm_q.weight"], d), "norm")
    nk = W.derived(f"{p}.norm_k", lambda: pairs_to_halves(W.weights[f"{p}.attn.norm_k.weight"], d), "norm")
    q = Transformer.HeadNormRotate(model, Ops.Slice(qkv, [0, 0, 0, 0], [1, 1, N, D]), nq, H, eps, cos, sin, compute)
    k = Transformer.HeadNormRotate(model, Ops.Slice(qkv, [0, 0, 0, D], [1, 1, N, D]), nk, H, eps, cos, sin, compute)
    v = Ops.Slice(qkv, [0, 0, 0, 2 * D], [1, 1, N, D])
    image = Layers.Attend(Ops.Slice(q, [0, 0, 0, 0], [1, 1, n_img, D]), k, v, H, key_length,
                          MaskType.KeySequenceLength)
    text = Layers.Attend(Ops.Slice(q, [0, 0, n_img, 0], [1, 1, n_txt, D]), Ops.Slice(k, [0, 0, n_img, 0], [1, 1, n_txt, D]),
                         Ops.Slice(v, [0, 0, n_img, 0], [1, 1, n_txt, D]), H,
                         Layers.Broadcast(text_mask, [1, H, n_txt, n_txt]), MaskType.Boolean)
    attended = Ops.Join([image, text], 2)
    x = Layers.Linear(model, attended, W(f"{p}.attn.to_out.0.weight"), gate=rows(modulation, 1, D, n_img, n_txt),
                      residual=x)
    normed = Transformer.Modulate(x, rows(modulation, 2, D, n_img, n_txt), eps, compute)
    f = Layers.Linear(model, normed, W.derived(f"{p}.gate_up", lambda: interleave_gate_up(_gate_up(W.weights, p))),
                      activation="swiglu")
    return Layers.Linear(model, f, W(f"{p}.img_mlp.out.weight"), gate=rows(modulation, 3, D, n_img, n_txt),
                         residual=x)


def _modulation(model: ModelBuilder, W: _Weights, cfg: QwenImageConfig, time):
    """The time path (QwenImageDit.cs:464-478): temb [1, 1, 2, D] of the
    noise level's and time zero's sinusoids, and the shared modulation [1, 1,
    2, 4D] = (scale1, tanh(gate1), scale2, tanh(gate2)), fp32."""
    D = cfg.width
    temb = Layers.Linear(model, Layers.Silu(Layers.Linear(model, time, W(
        "time_text_embed.timestep_embedder.linear_1.weight"))), W("time_text_embed.timestep_embedder.linear_2.weight"))
    mod = Layers.Linear(model, Layers.Silu(temb), W("modulation.1.weight"))

    def chunk(c):
        return Ops.Slice(mod, [0, 0, 0, c * D], [1, 1, 2, D])
    return temb, Ops.Join([chunk(0), Ops.ActivationTanh(chunk(1)), chunk(2), Ops.ActivationTanh(chunk(3))], 3)


def build_block_model(device: Device, cfg: QwenImageConfig, weights: dict, n_img: int, n_txt: int,
                      compute: HostDataType, int8: bool = False, block: int = 0):
    """One block as a compiled model. Inputs: x [1, 1, N, D] fp32, time [1, 1,
    2, time_dim] (the two sinusoids), text_mask [1, 1, Nt, Nt] I32, key_length
    [1, 1, 1, 1] I32, cos, sin [1, N, 1, 64] fp32. Output: x fp32."""
    store = compute if compute != F32 else HostDataType.Float16
    model = ModelBuilder(device, store, int8)
    W = _Weights(model, weights, compute)
    N = n_img + n_txt
    x = model.Placeholder([1, 1, N, cfg.width], F32)
    time = model.Placeholder([1, 1, 2, cfg.time_dim], F32)
    mask = model.Placeholder([1, 1, n_txt, n_txt], HostDataType.Int32)
    key_length = model.Placeholder([1, 1, 1, 1], HostDataType.Int32)
    cos = model.Placeholder([1, N, 1, cfg.head_dim // 2], F32)
    sin = model.Placeholder([1, N, 1, cfg.head_dim // 2], F32)
    _, mod = _modulation(model, W, cfg, time)
    y = build_block(model, W, block, cfg, x, mod, cos, sin, key_length, mask, n_img, n_txt, compute)
    model.Compile([y])
    W.release()
    return model


def build_step_model(device: Device, cfg: QwenImageConfig, weights: dict, latent_h: int, latent_w: int, n_txt: int,
                     compute: HostDataType, int8: bool = False):
    """The whole step (QwenImageDit.Build, :430-505) as one compiled model.
    Inputs: latent [1, C, H, W], time [1, 1, 2, time_dim], context [1, 1, Nt,
    context_width], text_mask [1, 1, Nt, Nt] I32, key_length [1, 1, 1, 1]
    I32, cos, sin [1, N, 1, 64]; all float inputs fp32. Output: the flow [1,
    C, H, W] fp32."""
    store = compute if compute != F32 else HostDataType.Float16
    model = ModelBuilder(device, store, int8)
    W = _Weights(model, weights, compute)
    C, D = cfg.latent_channels, cfg.width
    n_img = latent_h * latent_w
    N = n_img + n_txt
    latent = model.Placeholder([1, C, latent_h, latent_w], F32)
    time = model.Placeholder([1, 1, 2, cfg.time_dim], F32)
    context = model.Placeholder([1, 1, n_txt, cfg.context_width], F32)
    mask = model.Placeholder([1, 1, n_txt, n_txt], HostDataType.Int32)
    key_length = model.Placeholder([1, 1, 1, 1], HostDataType.Int32)
    cos = model.Placeholder([1, N, 1, cfg.head_dim // 2], F32)
    sin = model.Placeholder([1, N, 1, cfg.head_dim // 2], F32)

    # Embeddings, wide: the cells through img_in; the text through its
    # zero-centred RMS norm (stored weight + 1) and the GELU-tanh MLP.
    image = Layers.Linear(model, Ops.Patchify(latent, 1), W("img_in.weight"))
    text_scale = W.derived("txt_in.text_norm+1", lambda: _plus_one(W.weights["txt_in.text_norm.weight"]), "wide")
    text = Layers.RmsNorm(model, context, text_scale, cfg.eps)
    text = Layers.Linear(model, Layers.Linear(model, text, W("txt_in.in_layer.weight"), activation="gelu_tanh"),
                         W("txt_in.out_layer.weight"))
    x = Ops.Join([image, text], 2)
    temb, mod = _modulation(model, W, cfg, time)
    for i in range(cfg.blocks):
        x = build_block(model, W, i, cfg, x, mod, cos, sin, key_length, mask, n_img, n_txt, compute)
    # The final layer reads the image rows, scaled from the noise level's
    # row of the time embedding (:482-496).
    scale = Layers.Linear(model, Layers.Silu(Ops.Slice(temb, [0, 0, 0, 0], [1, 1, 1, D])), W("norm_out.linear.weight"))
    y = Transformer.Modulate(Ops.Slice(x, [0, 0, 0, 0], [1, 1, n_img, D]), scale, cfg.eps, F32)
    out = Layers.Linear(model, y, W("proj_out.weight"))
    model.Compile([Ops.Unpatchify(out, 1, C, latent_h, latent_w)])
    W.release()
    return model


def _plus_one(w):
    if isinstance(w, DeviceTensor):
        return HostTensor.FromFloats(w.Download().ToFloats() + 1.0).ToFloats()
    return np.asarray(w, np.float32) + 1.0


class QwenImageDit:
    """IDenoiser over the compiled step (QwenImageDit.Predict, :152-166):
    Predict(latent [64, H, W], timestep, sigma, conditioning) -> flow, with
    one branch of conditioning() (context, text_mask, key_length, cos, sin)."""

    def __init__(self, device: Device, cfg: QwenImageConfig, weights: dict, height: int, width: int,
                 context_rows: int, compute: HostDataType = HostDataType.BFloat16, int8: bool = False,
                 scale_factor: int = 16):
        if height % scale_factor or width % scale_factor:
            raise ValueError(f"{width}x{height} does not divide into {scale_factor}-pixel cells")
        self.cfg, self.device = cfg, device
        self.latent_h, self.latent_w = height // scale_factor, width // scale_factor
        self.context_rows = context_rows
        self.model = build_step_model(device, cfg, weights, self.latent_h, self.latent_w, context_rows, compute, int8)

    @property
    def Tokens(self) -> int:
        return self.latent_h * self.latent_w

    def Predict(self, latent: HostTensor, timestep: float, sigma: float, conditioning: dict) -> HostTensor:
        cfg = self.cfg
        n = self.Tokens + self.context_rows
        time = np.stack([time_embedding(sigma, cfg.time_dim), time_embedding(0.0, cfg.time_dim)])
        ins = [latent.ConvertTo(F32).Reshape(1, cfg.latent_channels, self.latent_h, self.latent_w),
               HostTensor.FromFloats(time.reshape(1, 1, 2, -1)),
               HostTensor.FromFloats(np.asarray(conditioning["context"], np.float32).reshape(1, 1, self.context_rows, -1)),
               HostTensor.FromInt32(np.asarray(conditioning["text_mask"], np.int32), 1, 1, self.context_rows,
                                    self.context_rows),
               HostTensor.FromInt32(np.asarray(conditioning["key_length"], np.int32), 1, 1, 1, 1),
               HostTensor.FromFloats(np.asarray(conditioning["cos"], np.float32).reshape(1, n, 1, -1)),
               HostTensor.FromFloats(np.asarray(conditioning["sin"], np.float32).reshape(1, n, 1, -1))]
        return self.model.Run(*ins)[0]

    def Dispose(self):
        self.model.Dispose()


# ---- checkpoints and LoRAs (QwenImageCheckpoint.cs, QwenImageLoras.cs, QwenImageWeights.cs) ---

DIT_PREFIXES = ("", "model.diffusion_model.")
# The tensors that together mark Qwen-Image 2.1's transformer
# (QwenImageCheckpoint.cs:24-28).
DIT_MARKERS = ("txt_in.text_norm.weight", "modulation.1.weight", "transformer_blocks.0.attn.norm_q.weight",
               "img_in.weight", "proj_out.weight")


def dit_prefix(file) -> "str | None":
    """QwenImageCheckpoint.DitPrefix (:38-50): the prefix the transformer
    sits under in a SafetensorsFile, or None for another file."""
    keys = set(file.Keys)
    for prefix in DIT_PREFIXES:
        if all(prefix + m in keys for m in DIT_MARKERS) and (
                f"{prefix}transformer_blocks.0.{FUSED_GATE_UP}" in keys
                or f"{prefix}transformer_blocks.0.{GATE_PROJECTION}" in keys):
            return prefix
    return None


def config_from_shapes(shapes: Dict[str, tuple]) -> QwenImageConfig:
    """The model's widths from its weights' shapes, as the reference's
    constructor reads them (QwenImageDit.cs:119-144): width and latent
    channels from img_in, the head from the query norm, the feed-forward
    from the gate rows, the time width from linear_1, the blocks by count and
    the context width from the text norm (QwenImageDit.ContextWidth)."""
    from .safetensors import InvalidDataError
    emb = tuple(shapes["img_in.weight"])
    if len(emb) != 2:
        raise InvalidDataError(f"img_in.weight is [{', '.join(map(str, emb))}], not [width, channels]")
    width, channels = emb
    head = shapes["transformer_blocks.0.attn.norm_q.weight"][0]
    if head != sum(ROPE_AXES) or width % head:
        raise InvalidDataError(f"a head of {head} features does not take the rotary axes")
    fused = f"transformer_blocks.0.{FUSED_GATE_UP}"
    mlp = shapes[fused][0] // 2 if fused in shapes else shapes[f"transformer_blocks.0.{GATE_PROJECTION}"][0]
    blocks = 0
    while f"transformer_blocks.{blocks}.attn.to_q.weight" in shapes:
        blocks += 1
    norm = tuple(shapes["txt_in.text_norm.weight"])
    if len(norm) != 1:
        raise InvalidDataError("the text norm has an unexpected shape")
    return QwenImageConfig(width=width, heads=width // head, mlp=mlp, blocks=blocks, latent_channels=channels,
                           context_width=norm[0],
                           time_dim=shapes["time_text_embed.timestep_embedder.linear_1.weight"][1])


LORA_DIT = "dit"
LORA_TEXT_ENCODER = "te"


def lora_layout():
    """QwenImageLoras.Layout (QwenImageLoras.cs:19-33): the transformer as
    kohya's lora_unet_..., diffusion_model..., transformer... or bare names,
    the Qwen3-VL text encoder as lora_te_... or text_encoders...; SDXL's two
    text towers refused on their names."""
    from .lora import LoraLayout, LoraTower
    sdxl = "was trained for SDXL, whose text encoders are two CLIP towers where Qwen-Image has Qwen3-VL"
    return LoraLayout("Qwen-Image 2.1",
                      [LoraTower(LORA_DIT, "transformer", "unet", "diffusion_model", ("transformer", "")),
                       LoraTower(LORA_TEXT_ENCODER, "Qwen3-VL text encoder", "te", "text_encoders")],
                      {"te1": sdxl, "te2": sdxl})


def fused_halves(key: str, rows: int):
    """QwenImageLoras.FusedHalves (:39-49): the names a LoRA has for the two
    halves of the fused gate/up matrix."""
    from .lora import LoraRows
    if not key.endswith("." + FUSED_GATE_UP):
        return []
    block = key[: -len(FUSED_GATE_UP)]
    return [LoraRows(block + GATE_PROJECTION, 0, rows // 2), LoraRows(block + UP_PROJECTION, rows // 2, rows // 2)]


def load_dit(file, device: Device, loras=(), dtype: HostDataType = HostDataType.BFloat16):
    """QwenImageWeights.LoadDit (QwenImageWeights.cs:26-34) for the device:
    the transformer's tensors under their bare names, each read from the
    mapping into HBM when the builder asks for it, narrowed there to dtype,
    with the LoRAs' deltas folded in on the device. A LoRA that fits nothing
    is refused here, before the build starts. Returns (config, weights)."""
    from .lora import LazyWeights, LoraPatchSet
    from .safetensors import InvalidDataError
    prefix = dit_prefix(file)
    if prefix is None:
        raise InvalidDataError("not a Qwen-Image 2.1 checkpoint")
    shapes = {k[len(prefix):]: file.TryGetInfo(k)[2] for k in file.Keys if k.startswith(prefix)}
    patches = (LoraPatchSet.Prepare(shapes, lora_layout(), LORA_DIT, list(loras),
                                    parts=lambda key: fused_halves(key, shapes[key][0]))
               if loras else None)
    return config_from_shapes(shapes), LazyWeights(file, prefix, patches, dtype, device)
