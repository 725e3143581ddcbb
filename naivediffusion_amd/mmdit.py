"""The Qwen-Image-shaped MMDiT denoiser: dual-stream joint blocks (separate
image and text weights, joint attention over the image-first sequence) and
the full step around them.

The reference has no dual-stream block (its Qwen-Image 2.1 is single
stream, Models/QwenImage/QwenImageDit.cs:9-16); this one is composed from
the reference's own per-layer primitives exactly as its Qwen-Image block
uses them (QwenImageDit.cs:336-428): Layers.Linear, Transformer.Modulate,
Transformer.HeadNorm + Rotate, Layers.Attend over the joined sequence,
GELU-tanh (QwenImageDit.cs:510-515) and the gated residuals. Mixed
precision follows QwenImageDit.cs:41-45: at half/bf16 compute the products
and the attention run narrow while the residual stream, the norms, the
rotary positions, the embeddings and the final layer stay fp32.
"""

from __future__ import annotations

import dataclasses
import math
from typing import Dict, Optional

import numpy as np

from . import rng
from .graph import ModelBuilder, Ops
from .layers import Layers, Transformer
from .tensors import Device, DeviceTensor, HostDataType, HostTensor, f32_to_bf16, bf16_to_f32

ROPE_AXES = (16, 56, 56)
ROPE_THETA = 10000.0


@dataclasses.dataclass(frozen=True)
class MmditConfig:
    width: int = 3072          # D
    heads: int = 24            # H (head size D / H = 128)
    mlp: int = 12288           # F, GELU-tanh
    blocks: int = 60
    latent_channels: int = 16
    patch: int = 2
    text_dim: int = 4096
    time_dim: int = 256        # the sinusoid's width
    eps: float = 1e-6

    @property
    def head_dim(self) -> int:
        return self.width // self.heads


STREAMS = ("img", "txt")


def block_weight_shapes(cfg: MmditConfig, i: int) -> Dict[str, tuple]:
    D, F, d = cfg.width, cfg.mlp, cfg.head_dim
    out = {}
    for s in STREAMS:
        p = f"blocks.{i}.{s}"
        out[f"{p}_mod.weight"] = (6 * D, D)
        out[f"{p}_mod.bias"] = (6 * D,)
        out[f"{p}_qkv.weight"] = (3 * D, D)
        out[f"{p}_qkv.bias"] = (3 * D,)
        out[f"{p}_norm_q.weight"] = (d,)
        out[f"{p}_norm_k.weight"] = (d,)
        out[f"{p}_out.weight"] = (D, D)
        out[f"{p}_out.bias"] = (D,)
        out[f"{p}_fc1.weight"] = (F, D)
        out[f"{p}_fc1.bias"] = (F,)
        out[f"{p}_fc2.weight"] = (D, F)
        out[f"{p}_fc2.bias"] = (D,)
    return out


def weight_shapes(cfg: MmditConfig) -> Dict[str, tuple]:
    D = cfg.width
    pd = cfg.latent_channels * cfg.patch * cfg.patch
    out = {
        "img_in.weight": (D, pd), "img_in.bias": (D,),
        "txt_norm.weight": (cfg.text_dim,),
        "txt_in.weight": (D, cfg.text_dim), "txt_in.bias": (D,),
        "time.linear_1.weight": (D, cfg.time_dim), "time.linear_1.bias": (D,),
        "time.linear_2.weight": (D, D), "time.linear_2.bias": (D,),
        "norm_out.weight": (2 * D, D), "norm_out.bias": (2 * D,),
        "proj_out.weight": (pd, D), "proj_out.bias": (pd,),
    }
    for i in range(cfg.blocks):
        out.update(block_weight_shapes(cfg, i))
    return out


def _is_norm(name: str) -> bool:
    return "norm_q" in name or "norm_k" in name or name == "txt_norm.weight"


def synthetic_weights(cfg: MmditConfig, seed: int, names=None, norm_spread: float = 0.0) -> Dict[str, np.ndarray]:
    """Host weights: N(0, 0.02) rounded to bf16 (returned as the fp32 values
    of those bf16 numbers); norm weights 1 (+ N(0, norm_spread))."""
    shapes = weight_shapes(cfg)
    out = {}
    for name in (names or shapes):
        shape = shapes[name]
        if _is_norm(name):
            v = np.ones(shape, np.float32)
            if norm_spread:
                v = v + rng.normal(rng.tensor_seed(seed, name), shape, 0.0, norm_spread)
        else:
            v = rng.normal(rng.tensor_seed(seed, name), shape, 0.0, 0.02)
        out[name] = bf16_to_f32(f32_to_bf16(v)).reshape(shape)
    return out


def device_weights(device: Device, cfg: MmditConfig, seed: int, names=None,
                   norm_spread: float = 0.0) -> Dict[str, DeviceTensor]:
    """The same weights made on the GPU in bf16 (norm weights 1, + N(0,
    norm_spread) made on the host as synthetic_weights makes them): the
    synthetic model of the benchmark, never passing through host memory."""
    shapes = weight_shapes(cfg)
    out = {}
    for name in (names or shapes):
        shape = shapes[name]
        if _is_norm(name):
            v = np.ones(shape, np.float32)
            if norm_spread:
                v = v + rng.normal(rng.tensor_seed(seed, name), shape, 0.0, norm_spread)
            out[name] = device.Upload(HostTensor(HostDataType.BFloat16, shape, f32_to_bf16(v)))
        else:
            out[name] = device.Normal(HostDataType.BFloat16, shape, rng.tensor_seed(seed, name), 0.0, 0.02)
    return out


def rope_tables(rows: int, cols: int, text_rows: int):
    """The joint sequence's rotary tables [tokens, 64]: image cell (i, j) at
    (0, i - ceil(h/2), j - ceil(w/2)) on the {16, 56, 56} axes
    (QwenImageDit.RopeTables, QwenImageDit.cs:189-240, with the frame at 0),
    text rows unrotated (cos 1, sin 0)."""
    freqs = []
    for axis in ROPE_AXES:
        for k in range(axis // 2):
            freqs.append(1.0 / ROPE_THETA ** (2.0 * k / axis))
    freqs = np.array(freqs, np.float64)
    r0, c0 = rows - rows // 2, cols - cols // 2
    ii, jj = np.meshgrid(np.arange(rows) - r0, np.arange(cols) - c0, indexing="ij")
    pos = np.zeros((rows * cols, 64), np.float64)
    pos[:, 8:36] = ii.reshape(-1, 1)
    pos[:, 36:64] = jj.reshape(-1, 1)
    ang = pos * freqs
    cos = np.concatenate([np.cos(ang), np.ones((text_rows, 64))]).astype(np.float32)
    sin = np.concatenate([np.sin(ang), np.zeros((text_rows, 64))]).astype(np.float32)
    return cos, sin


def time_embedding(t: float, width: int) -> np.ndarray:
    """Flux/Qwen's sinusoid of 1000 t (QwenImageDit.TimeEmbedding, :176-177)."""
    return Transformer.Sinusoid(float(t * 1000.0), width)


class _W:
    """Registers each named weight once in a builder. With per_channel the
    matrices are quantised to int8 on the device with one fp32 scale per
    output row (block = the row) and handed over pre-quantised."""

    def __init__(self, model: ModelBuilder, weights: dict, compute: HostDataType, per_channel: bool = False):
        self.model, self.weights, self.compute = model, weights, compute
        self.per_channel = per_channel
        self.cache = {}
        self.owned = []  # device tensors made here (stacks), released after the builder has what it needs

    def __call__(self, name: str, kind: str = "weight"):
        if name in self.cache:
            return self.cache[name]
        return self._register(name, self.weights[name], kind)

    def stacked(self, names, kind: str = "weight"):
        """The named tensors stacked along their first axis into one weight
        (matrices: rows one after another; vectors: end to end). Device
        tensors are stacked on the device; the stack is freed once the
        builder holds it."""
        key = ("stack", kind) + tuple(names)
        if key in self.cache:
            return self.cache[key]
        ws = [self.weights[n] for n in names]
        if all(isinstance(w, DeviceTensor) for w in ws):
            from .weights import device_stack
            w = device_stack(self.model.Device, ws)
            self.owned.append(w)
        else:
            w = np.concatenate([np.asarray(x, np.float32) for x in ws], 0)
        return self._register(key, w, kind)

    def release(self):
        for t in self.owned:
            t.Dispose()
        self.owned = []

    def _register(self, name, w, kind):
        m = self.model
        if isinstance(w, DeviceTensor):
            shape = w.Shape
            if kind == "weight" and len(shape) == 2 and self.per_channel and shape[0] * shape[1] >= (1 << 16):
                q, sc = m.Device.QuantizeInt8(w, shape[1], HostDataType.Float32)
                e = m.WeightInt8(q, sc, shape[1])
            elif kind == "weight" and len(shape) == 2:
                e = m.WeightOnDevice(w, shape[0])
            else:
                e = m.ConstantOnDevice(w)
        else:
            arr = np.asarray(w, np.float32)
            if kind == "weight" and arr.ndim == 2:
                e = m.Weight(HostTensor.FromFloats(arr), arr.shape, arr.shape[0])
            else:
                dt = HostDataType.Float32 if kind == "wide" else self.compute
                e = m.Constant(HostTensor.FromFloats(arr), [arr.size], dt)
        self.cache[name] = e
        return e


def _chunk(mod, i: int, D: int):
    s = mod.Shape
    return Ops.Slice(mod, [0, 0, 0, i * D], [s[0], s[1], s[2], D])


def adaln_projections(model: ModelBuilder, W: _W, cfg: MmditConfig, silu_temb, blocks: int):
    """Every block's adaLN projection (QwenImageDit.cs:466-478 per stream:
    Linear(SiLU(temb)) -> 6 x D) as one weight-streaming GEMV per stream over
    the blocks' stacked weights, launched once at the start of the step: the
    projections depend only on the time embedding, and one launch over 6.8 GB
    of weights streams them at the GEMV's full rate instead of 60 short
    launches beside the other stream's products. Returns, per stream, the
    blocks' [B, 1, 1, 6D] views of the result."""
    D = cfg.width
    B = silu_temb.Shape[0]
    out = {}
    for s in STREAMS:
        w = W.stacked([f"blocks.{i}.{s}_mod.weight" for i in range(blocks)])
        b = W.stacked([f"blocks.{i}.{s}_mod.bias" for i in range(blocks)], "wide")
        every = Layers.Linear(model, silu_temb, w, b)
        out[s] = [Ops.Slice(every, [0, 0, 0, i * 6 * D], [B, 1, 1, 6 * D]) for i in range(blocks)]
    return out


def build_block(model: ModelBuilder, W: _W, i: int, cfg: MmditConfig, x_img, x_txt, silu_temb, cos, sin,
                compute: HostDataType, key_len=None, two_streams: bool = True, mods=None):
    """One dual-stream joint block. x_img [B, 1, Ni, D] and x_txt [B, 1, Nt,
    D] are the fp32 residual streams; silu_temb [B, 1, 1, T]; cos/sin [1, N,
    1, 64]. Returns the updated (x_img, x_txt). With two_streams the text
    stream's operations run on the second stream, beside the image stream's
    (they meet at the joint attention). mods: the block's adaLN projections
    per stream when they were made elsewhere (adaln_projections)."""
    D, H, eps = cfg.width, cfg.heads, cfg.eps
    B, _, n_img, _ = x_img.Shape
    n_txt = x_txt.Shape[2]
    x = {"img": x_img, "txt": x_txt}
    rows = {"img": (0, n_img), "txt": (n_img, n_txt)}
    p = {s: f"blocks.{i}.{s}" for s in STREAMS}
    g = model.Graph

    def lane(s):
        return g.Stream(1 if (two_streams and s == "txt") else 0)

    mod, h, q, k, v = {}, {}, {}, {}, {}
    for s in STREAMS:
        with lane(s):
            # (shift1, scale1, gate1, shift2, scale2, gate2), fp32 like the
            # reference's time path.
            if mods is not None:
                mod[s] = mods[s]
            else:
                mod[s] = Layers.Linear(model, silu_temb, W(f"{p[s]}_mod.weight"), W(f"{p[s]}_mod.bias", "wide"))
            h[s] = Transformer.Modulate(x[s], _chunk(mod[s], 0, D), _chunk(mod[s], 1, D), eps, compute)
            qkv = Layers.Linear(model, h[s], W(f"{p[s]}_qkv.weight"), W(f"{p[s]}_qkv.bias", "bias"))
            r0, nr = rows[s]
            c = Ops.Slice(cos, [0, r0, 0, 0], [1, nr, 1, 64])
            sn = Ops.Slice(sin, [0, r0, 0, 0], [1, nr, 1, 64])
            q[s] = Transformer.HeadNormRotate(model, Ops.Slice(qkv, [0, 0, 0, 0], [B, 1, nr, D]),
                                              W(f"{p[s]}_norm_q.weight", "bias"), H, eps, c, sn, compute)
            k[s] = Transformer.HeadNormRotate(model, Ops.Slice(qkv, [0, 0, 0, D], [B, 1, nr, D]),
                                              W(f"{p[s]}_norm_k.weight", "bias"), H, eps, c, sn, compute)
            v[s] = Ops.Slice(qkv, [0, 0, 0, 2 * D], [B, 1, nr, D])
    joint = [Ops.Join([t["img"], t["txt"]], 2) for t in (q, k, v)]
    if key_len is None:
        a = Layers.Attend(*joint, H)
    else:
        from .graph import MaskType
        a = Layers.Attend(*joint, H, key_len, MaskType.KeySequenceLength)
    for s in STREAMS:
        with lane(s):
            r0, nr = rows[s]
            a_s = Ops.Slice(a, [0, 0, r0, 0], [B, 1, nr, D])
            x[s] = Layers.Linear(model, a_s, W(f"{p[s]}_out.weight"), W(f"{p[s]}_out.bias", "bias"),
                                 gate=_chunk(mod[s], 2, D), residual=x[s])
            h[s] = Transformer.Modulate(x[s], _chunk(mod[s], 3, D), _chunk(mod[s], 4, D), eps, compute)
            f = Layers.Linear(model, h[s], W(f"{p[s]}_fc1.weight"), W(f"{p[s]}_fc1.bias", "bias"),
                              activation="gelu_tanh")
            x[s] = Layers.Linear(model, f, W(f"{p[s]}_fc2.weight"), W(f"{p[s]}_fc2.bias", "bias"),
                                 gate=_chunk(mod[s], 5, D), residual=x[s])
    return x["img"], x["txt"]


def build_block_model(device: Device, cfg: MmditConfig, weights: dict, batch: int, n_img: int, n_txt: int,
                      compute: HostDataType, int8=False, block: int = 0, key_len: bool = False,
                      two_streams: bool = True):
    """A compiled single-block model. Inputs in order: x_img [B,1,Ni,D],
    x_txt [B,1,Nt,D], temb [B,1,1,D] (the time embedding before SiLU), cos,
    sin [1,N,1,64] (and the key length [1,1,1,1] when key_len). Outputs the
    updated x_img, x_txt (fp32). int8 as in build_step_model ("channel"
    needs the weights as device tensors)."""
    D = cfg.width
    per_channel = int8 == "channel"
    model = ModelBuilder(device, compute, bool(int8) and not per_channel)
    W = _W(model, weights, compute, per_channel)
    xi = model.Placeholder([batch, 1, n_img, D], HostDataType.Float32)
    xt = model.Placeholder([batch, 1, n_txt, D], HostDataType.Float32)
    temb = model.Placeholder([batch, 1, 1, D], HostDataType.Float32)
    cos = model.Placeholder([1, n_img + n_txt, 1, 64], HostDataType.Float32)
    sin = model.Placeholder([1, n_img + n_txt, 1, 64], HostDataType.Float32)
    kl = model.Placeholder([1, 1, 1, 1], HostDataType.Int32) if key_len else None
    yi, yt = build_block(model, W, block, cfg, xi, xt, Layers.Silu(temb), cos, sin, compute, kl, two_streams)
    return model.Compile([yi, yt])


def build_step_model(device: Device, cfg: MmditConfig, weights: dict, batch: int, n_txt: int, latent_h: int,
                     latent_w: int, compute: HostDataType, int8=False, two_streams: bool = True,
                     stack_adaln: bool = True):
    """The full denoiser step as one compiled model (every GraphChain cut of
    the reference is a no-op here: everything is resident). Inputs: latent
    [B, C, H, W] fp32, text [B, 1, Nt, text_dim] fp32, the time sinusoid
    [B, 1, 1, time_dim] fp32, cos, sin [1, N, 1, 64]. Output: the flow
    [B, C, H, W] fp32."""
    D, C, p = cfg.width, cfg.latent_channels, cfg.patch
    n_img = (latent_h // p) * (latent_w // p)
    # int8: False, True / "block32" (the reference's BlockQuantizer format,
    # quantised by the builder) or "channel" (one fp32 scale per output row).
    per_channel = int8 == "channel"
    model = ModelBuilder(device, compute, bool(int8) and not per_channel)
    W = _W(model, weights, compute, per_channel)
    latent = model.Placeholder([batch, C, latent_h, latent_w], HostDataType.Float32)
    text = model.Placeholder([batch, 1, n_txt, cfg.text_dim], HostDataType.Float32)
    tsin = model.Placeholder([batch, 1, 1, cfg.time_dim], HostDataType.Float32)
    cos = model.Placeholder([1, n_img + n_txt, 1, 64], HostDataType.Float32)
    sin = model.Placeholder([1, n_img + n_txt, 1, 64], HostDataType.Float32)

    # Embeddings, kept wide (QwenImageDit.cs:445-462).
    x_img = Layers.Linear(model, Ops.Patchify(latent, p), W("img_in.weight"), W("img_in.bias", "wide"))
    normed = Layers.RmsNorm(model, text, W("txt_norm.weight", "wide"), cfg.eps)
    x_txt = Layers.Linear(model, normed, W("txt_in.weight"), W("txt_in.bias", "wide"))
    temb = Layers.Linear(model, Layers.Silu(Layers.Linear(model, tsin, W("time.linear_1.weight"),
                                                          W("time.linear_1.bias", "wide"))),
                         W("time.linear_2.weight"), W("time.linear_2.bias", "wide"))
    silu_temb = Layers.Silu(temb)
    mods = adaln_projections(model, W, cfg, silu_temb, cfg.blocks) if stack_adaln else None
    for i in range(cfg.blocks):
        x_img, x_txt = build_block(model, W, i, cfg, x_img, x_txt, silu_temb, cos, sin, compute,
                                   two_streams=two_streams,
                                   mods=None if mods is None else {s: mods[s][i] for s in STREAMS})
    # Final layer: modulated LayerNorm (scale, shift) then the projection,
    # wide (QwenImageDit.cs:488-496).
    mod = Layers.Linear(model, silu_temb, W("norm_out.weight"), W("norm_out.bias", "wide"))
    y = Transformer.Modulate(x_img, _chunk(mod, 1, D), _chunk(mod, 0, D), cfg.eps, HostDataType.Float32)
    out = Layers.Linear(model, y, W("proj_out.weight"), W("proj_out.bias", "wide"))
    flow = Ops.Unpatchify(out, p, C, latent_h, latent_w)
    compiled = model.Compile([flow])
    W.release()
    return compiled


class QwenImageMmdit:
    """IDenoiser over the compiled step (Pipeline/IDenoiser.cs:16-17):
    Predict(latent, timestep, sigma, conditioning) -> flow, host tensors in
    and out. conditioning holds 'context' [Nt, text_dim] rows."""

    def __init__(self, device: Device, cfg: MmditConfig, weights: dict, latent_h: int, latent_w: int, n_txt: int,
                 compute: HostDataType = HostDataType.BFloat16, int8: bool = False):
        self.cfg, self.device = cfg, device
        self.latent_h, self.latent_w, self.n_txt = latent_h, latent_w, n_txt
        self.model = build_step_model(device, cfg, weights, 1, n_txt, latent_h, latent_w, compute, int8)
        p = cfg.patch
        self.cos, self.sin = rope_tables(latent_h // p, latent_w // p, n_txt)

    @property
    def ResidentBytes(self) -> int:
        return self.model.PersistentBytes

    @property
    def StreamedBytes(self) -> int:
        return 0

    def Predict(self, latent: HostTensor, timestep: float, sigma: float, conditioning: dict) -> HostTensor:
        cfg = self.cfg
        n = self.cos.shape[0]
        ctx = np.asarray(conditioning["context"], np.float32).reshape(1, 1, self.n_txt, cfg.text_dim)
        t = time_embedding(sigma, cfg.time_dim).reshape(1, 1, 1, cfg.time_dim)
        ins = [latent.ConvertTo(HostDataType.Float32).Reshape(1, cfg.latent_channels, self.latent_h, self.latent_w),
               HostTensor.FromFloats(ctx), HostTensor.FromFloats(t),
               HostTensor.FromFloats(self.cos.reshape(1, n, 1, 64)), HostTensor.FromFloats(self.sin.reshape(1, n, 1, 64))]
        return self.model.Run(*ins)[0]
