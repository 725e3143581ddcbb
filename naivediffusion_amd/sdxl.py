"""SDXL's UNet on the device: Models/Sdxl/UNetModel.cs and UNetLayers.cs.

A noisy latent, a timestep and the text conditioning in, the predicted
noise out: the input convolution, three levels down (resnets, then at
levels 1 and 2 a Transformer2d per resnet; a stride-2 convolution between
levels), the mid block, three levels up (each unit first joins the newest
skip connection onto the running value along the channels; a nearest 2x
upsample cropped to the next skip's extent and a convolution between
levels), the output norm and convolution.

Built from the reference's per-layer primitives with the MI355X path's
fused forms: GroupNorm and its SiLU as one kernel, the resnet's x + h in
the second convolution's epilogue, the residual adds of the transformer
block in the epilogues of its output projections, the self-attention's q,
k, v as one GEMM over stacked weights (k, v likewise for the
cross-attention), and the 3x3 / 1x1 convolutions as implicit GEMMs on
MFMA. The reference runs the UNet at fp16 throughout (UNetModel.cs:61-67);
fp16 is the default here, bf16 and fp32 are accepted.
"""

from __future__ import annotations

import dataclasses
import math
from typing import Dict, Sequence

import numpy as np

from . import rng
from .graph import ModelBuilder, Ops
from .layers import Layers
from .tensors import Device, DeviceTensor, HostDataType, HostTensor
from .weights import WeightSet


@dataclasses.dataclass(frozen=True)
class SdxlConfig:
    """UNetModel.cs:22-39."""
    block_out: tuple = (320, 640, 1280)
    layers_per_block: int = 2
    transformer_layers: tuple = (0, 2, 10)
    heads: tuple = (5, 10, 20)
    in_channels: int = 4
    context_width: int = 2048
    time_embed: int = 1280
    add_time_dim: int = 256
    pooled_width: int = 1280
    groups: int = 32
    eps: float = 1e-5              # the resnets' GroupNorm
    transformer_eps: float = 1e-6  # Transformer2DModel's GroupNorm
    layer_norm_eps: float = 1e-5

    @property
    def add_width(self) -> int:
        return self.pooled_width + 6 * self.add_time_dim


def _resnet_shapes(out: dict, p: str, cin: int, cout: int, temb: int):
    out[f"{p}.norm1.weight"] = (cin,)
    out[f"{p}.norm1.bias"] = (cin,)
    out[f"{p}.conv1.weight"] = (cout, cin, 3, 3)
    out[f"{p}.conv1.bias"] = (cout,)
    out[f"{p}.time_emb_proj.weight"] = (cout, temb)
    out[f"{p}.time_emb_proj.bias"] = (cout,)
    out[f"{p}.norm2.weight"] = (cout,)
    out[f"{p}.norm2.bias"] = (cout,)
    out[f"{p}.conv2.weight"] = (cout, cout, 3, 3)
    out[f"{p}.conv2.bias"] = (cout,)
    if cin != cout:
        out[f"{p}.conv_shortcut.weight"] = (cout, cin, 1, 1)
        out[f"{p}.conv_shortcut.bias"] = (cout,)


def _transformer_shapes(out: dict, p: str, c: int, layers: int, ctx: int):
    inner = 4 * c
    out[f"{p}.norm.weight"] = (c,)
    out[f"{p}.norm.bias"] = (c,)
    out[f"{p}.proj_in.weight"] = (c, c)
    out[f"{p}.proj_in.bias"] = (c,)
    for j in range(layers):
        q = f"{p}.transformer_blocks.{j}"
        for n in (1, 2, 3):
            out[f"{q}.norm{n}.weight"] = (c,)
            out[f"{q}.norm{n}.bias"] = (c,)
        for a, src in (("attn1", c), ("attn2", ctx)):
            out[f"{q}.{a}.to_q.weight"] = (c, c)
            out[f"{q}.{a}.to_k.weight"] = (c, src)
            out[f"{q}.{a}.to_v.weight"] = (c, src)
            out[f"{q}.{a}.to_out.0.weight"] = (c, c)
            out[f"{q}.{a}.to_out.0.bias"] = (c,)
        out[f"{q}.ff.net.0.proj.weight"] = (2 * inner, c)
        out[f"{q}.ff.net.0.proj.bias"] = (2 * inner,)
        out[f"{q}.ff.net.2.weight"] = (c, inner)
        out[f"{q}.ff.net.2.bias"] = (c,)
    out[f"{p}.proj_out.weight"] = (c, c)
    out[f"{p}.proj_out.bias"] = (c,)


def weight_shapes(cfg: SdxlConfig) -> Dict[str, tuple]:
    """diffusers' UNet2DConditionModel names and shapes, walked the way
    UNetModel.Build (:328-426) consumes them."""
    c0, T = cfg.block_out[0], cfg.time_embed
    out = {
        "conv_in.weight": (c0, cfg.in_channels, 3, 3), "conv_in.bias": (c0,),
        "time_embedding.linear_1.weight": (T, c0), "time_embedding.linear_1.bias": (T,),
        "time_embedding.linear_2.weight": (T, T), "time_embedding.linear_2.bias": (T,),
        "add_embedding.linear_1.weight": (T, cfg.add_width), "add_embedding.linear_1.bias": (T,),
        "add_embedding.linear_2.weight": (T, T), "add_embedding.linear_2.bias": (T,),
    }
    levels = len(cfg.block_out)
    ch = c0
    skips = [ch]
    for level in range(levels):
        cout = cfg.block_out[level]
        for i in range(cfg.layers_per_block):
            _resnet_shapes(out, f"down_blocks.{level}.resnets.{i}", ch, cout, T)
            ch = cout
            if cfg.transformer_layers[level]:
                _transformer_shapes(out, f"down_blocks.{level}.attentions.{i}", ch, cfg.transformer_layers[level],
                                    cfg.context_width)
            skips.append(ch)
        if level != levels - 1:
            out[f"down_blocks.{level}.downsamplers.0.conv.weight"] = (ch, ch, 3, 3)
            out[f"down_blocks.{level}.downsamplers.0.conv.bias"] = (ch,)
            skips.append(ch)
    _resnet_shapes(out, "mid_block.resnets.0", ch, ch, T)
    _transformer_shapes(out, "mid_block.attentions.0", ch, cfg.transformer_layers[-1], cfg.context_width)
    _resnet_shapes(out, "mid_block.resnets.1", ch, ch, T)
    for i in range(levels):
        level = levels - 1 - i
        cout = cfg.block_out[level]
        for j in range(cfg.layers_per_block + 1):
            skip = skips.pop()
            _resnet_shapes(out, f"up_blocks.{i}.resnets.{j}", ch + skip, cout, T)
            ch = cout
            if cfg.transformer_layers[level]:
                _transformer_shapes(out, f"up_blocks.{i}.attentions.{j}", ch, cfg.transformer_layers[level],
                                    cfg.context_width)
        if i != levels - 1:
            out[f"up_blocks.{i}.upsamplers.0.conv.weight"] = (ch, ch, 3, 3)
            out[f"up_blocks.{i}.upsamplers.0.conv.bias"] = (ch,)
    out["conv_norm_out.weight"] = (ch,)
    out["conv_norm_out.bias"] = (ch,)
    out["conv_out.weight"] = (cfg.in_channels, ch, 3, 3)
    out["conv_out.bias"] = (cfg.in_channels,)
    return out


def _init(name: str, shape: tuple, seed: int):
    """Synthetic values: norm weights 1 and norm biases 0 (+ a small seeded
    spread); matrices and filters N(0, 1/fan_in) so activations keep their
    scale through the depth; biases N(0, 0.02)."""
    if ".norm" in name or name.startswith("conv_norm_out"):
        base = 1.0 if name.endswith("weight") else 0.0
        return base + rng.normal(rng.tensor_seed(seed, name), shape, 0.0, 0.05)
    if len(shape) == 1:
        return rng.normal(rng.tensor_seed(seed, name), shape, 0.0, 0.02)
    fan_in = int(np.prod(shape[1:]))
    return rng.normal(rng.tensor_seed(seed, name), shape, 0.0, 1.0 / math.sqrt(fan_in))


def synthetic_weights(cfg: SdxlConfig, seed: int, dtype: HostDataType = HostDataType.Float16) -> Dict[str, np.ndarray]:
    """Host weights (fp32 arrays holding values exact at `dtype`)."""
    out = {}
    for name, shape in weight_shapes(cfg).items():
        v = np.asarray(_init(name, shape, seed), np.float32)
        out[name] = HostTensor.FromFloats(v).ConvertTo(dtype).ToFloats().reshape(shape)
    return out


def device_weights(device: Device, cfg: SdxlConfig, seed: int, dtype: HostDataType = HostDataType.Float16) -> dict:
    """Synthetic weights made on the GPU at `dtype`: N(0, 0.02) everywhere
    but the norm weights, which are 1."""
    out = {}
    for name, shape in weight_shapes(cfg).items():
        if (".norm" in name or name.startswith("conv_norm_out")) and name.endswith("weight"):
            out[name] = device.Upload(HostTensor.FromFloats(np.ones(shape, np.float32)).ConvertTo(dtype))
        else:
            out[name] = device.Normal(dtype, shape, rng.tensor_seed(seed, name), 0.0, 0.02)
    return out


def timestep_embedding(timesteps: Sequence[float], dim: int, max_period: float = 10000.0) -> np.ndarray:
    """UNetModel.TimestepEmbedding (:150-169): per timestep, cosines of
    t * exp(-ln(max_period) i / half) then sines (flip_sin_to_cos), computed
    in double and stored as float."""
    half = dim // 2
    out = np.empty((len(timesteps), dim), np.float32)
    i = np.arange(half, dtype=np.float64)
    freq = np.exp(-math.log(max_period) * i / half)
    for r, t in enumerate(timesteps):
        ang = float(t) * freq
        out[r, :half] = np.cos(ang)
        out[r, half:] = np.sin(ang)
    return out


def add_conditioning(pooled: np.ndarray, original=(1024, 1024), crop=(0, 0), target=(1024, 1024),
                     add_time_dim: int = 256) -> np.ndarray:
    """UNetModel.AddConditioning (:180-197): the pooled text embedding, then
    the sinusoids of (original h, w, crop top, left, target h, w)."""
    ids = [original[0], original[1], crop[0], crop[1], target[0], target[1]]
    return np.concatenate([np.asarray(pooled, np.float32).ravel(),
                           timestep_embedding(ids, add_time_dim).ravel()]).astype(np.float32)


# ---- graph construction ----------------------------------------------------------------

def embedding_mlp(model: ModelBuilder, W: WeightSet, x, prefix: str):
    """UNetModel.EmbeddingMlp (:220-227): Linear, SiLU, Linear."""
    h = Layers.Linear(model, x, W(f"{prefix}.linear_1.weight"), W(f"{prefix}.linear_1.bias", "norm"),
                      activation="silu")
    return Layers.Linear(model, h, W(f"{prefix}.linear_2.weight"), W(f"{prefix}.linear_2.bias", "norm"))


def resnet_block(model: ModelBuilder, W: WeightSet, cfg: SdxlConfig, x, silu_temb, p: str):
    """UNetModel.ResnetBlock (:230-254): GroupNorm-SiLU-conv, plus the time
    projection per channel, GroupNorm-SiLU-conv, plus the (1x1-projected
    when the width changes) input, fused into the second convolution."""
    v = lambda n: W(f"{p}.{n}", "norm")
    h = Layers.GroupNorm(model, x, v("norm1.weight"), v("norm1.bias"), cfg.groups, cfg.eps, silu=True)
    h = Layers.Conv2d(model, h, W(f"{p}.conv1.weight"), v("conv1.bias"))
    projected = Layers.Linear(model, silu_temb, W(f"{p}.time_emb_proj.weight"), v("time_emb_proj.bias"))
    h = h + Layers.Broadcast(Layers.ToChannels(projected), h.Shape)
    h = Layers.GroupNorm(model, h, v("norm2.weight"), v("norm2.bias"), cfg.groups, cfg.eps, silu=True)
    if W.has(f"{p}.conv_shortcut.weight"):
        x = Layers.Conv2d(model, x, W(f"{p}.conv_shortcut.weight"), v("conv_shortcut.bias"), padding=0)
    return Layers.Conv2d(model, h, W(f"{p}.conv2.weight"), v("conv2.bias"), residual=x)


def context_kv(model: ModelBuilder, W: WeightSet, context):
    """The cross-attention keys and values of the context for every
    transformer block at once: the context is the same for all of them, so
    their to_k / to_v projections (UNetLayers.DiffusersAttention, :14-26)
    stack into one product over the context's rows instead of one small
    product per block. Returns {block prefix: (k, v)}, views of the result."""
    blocks = sorted(n[: -len(".attn2.to_k.weight")] for n in W.weights if n.endswith(".attn2.to_k.weight"))
    if not blocks:
        return {}
    names = [f"{b}.attn2.{t}.weight" for b in blocks for t in ("to_k", "to_v")]
    kv = Layers.Linear(model, context, W.stacked(names))
    b_, _, nc, _ = kv.Shape
    out, col = {}, 0
    for blk in blocks:
        w = W.weights[f"{blk}.attn2.to_k.weight"]
        c = w.Shape[0] if isinstance(w, DeviceTensor) else len(w)
        out[blk] = (Ops.Slice(kv, [0, 0, 0, col], [b_, 1, nc, c]), Ops.Slice(kv, [0, 0, 0, col + c], [b_, 1, nc, c]))
        col += 2 * c
    return out


def transformer_block(model: ModelBuilder, W: WeightSet, cfg: SdxlConfig, x, context, p: str, heads: int,
                      kv_all=None):
    """UNetModel.TransformerBlock (:258-276) with UNetLayers.DiffusersAttention
    (:14-26) and Geglu (:30-47): self-attention, cross-attention into the
    context, the gated feed-forward, each on a LayerNorm of x and added back.
    kv_all: the context's keys and values made for every block at once
    (context_kv); without it the block projects the context itself."""
    v = lambda n: W(f"{p}.{n}", "norm")
    b, _, n, c = x.Shape
    eps = cfg.layer_norm_eps

    h = Layers.LayerNorm(model, x, v("norm1.weight"), v("norm1.bias"), eps)
    a = f"{p}.attn1"
    qkv = Layers.Linear(model, h, W.stacked([f"{a}.to_q.weight", f"{a}.to_k.weight", f"{a}.to_v.weight"]))
    q, k, val = (Ops.Slice(qkv, [0, 0, 0, i * c], [b, 1, n, c]) for i in range(3))
    x = Layers.Linear(model, Layers.Attend(q, k, val, heads), W(f"{a}.to_out.0.weight"), v("attn1.to_out.0.bias"),
                      residual=x)

    h = Layers.LayerNorm(model, x, v("norm2.weight"), v("norm2.bias"), eps)
    a = f"{p}.attn2"
    q = Layers.Linear(model, h, W(f"{a}.to_q.weight"))
    if kv_all and p in kv_all:
        k, val = kv_all[p]
    else:
        nc = context.Shape[2]
        kv = Layers.Linear(model, context, W.stacked([f"{a}.to_k.weight", f"{a}.to_v.weight"]))
        k = Ops.Slice(kv, [0, 0, 0, 0], [b, 1, nc, c])
        val = Ops.Slice(kv, [0, 0, 0, c], [b, 1, nc, c])
    x = Layers.Linear(model, Layers.Attend(q, k, val, heads), W(f"{a}.to_out.0.weight"), v("attn2.to_out.0.bias"),
                      residual=x)

    h = Layers.LayerNorm(model, x, v("norm3.weight"), v("norm3.bias"), eps)
    proj = Layers.Linear(model, h, W(f"{p}.ff.net.0.proj.weight"), v("ff.net.0.proj.bias"))
    inner = proj.Shape[3] // 2
    gated = Ops.Slice(proj, [0, 0, 0, 0], [b, 1, n, inner]) * \
        Ops.ActivationGelu(Ops.Slice(proj, [0, 0, 0, inner], [b, 1, n, inner]))
    return Layers.Linear(model, gated, W(f"{p}.ff.net.2.weight"), v("ff.net.2.bias"), residual=x)


def transformer2d(model: ModelBuilder, W: WeightSet, cfg: SdxlConfig, x, context, p: str, heads: int, layers: int,
                  kv_all=None):
    """UNetModel.Transformer2d (:279-301): GroupNorm, to tokens, proj_in, the
    blocks, proj_out, back to the image, plus the input."""
    _, _, height, width = x.Shape
    v = lambda n: W(f"{p}.{n}", "norm")
    normed = Layers.GroupNorm(model, x, v("norm.weight"), v("norm.bias"), cfg.groups, cfg.transformer_eps)
    tokens = Layers.Linear(model, Layers.ToTokens(normed), W(f"{p}.proj_in.weight"), v("proj_in.bias"))
    for j in range(layers):
        tokens = transformer_block(model, W, cfg, tokens, context, f"{p}.transformer_blocks.{j}", heads, kv_all)
    tokens = Layers.Linear(model, tokens, W(f"{p}.proj_out.weight"), v("proj_out.bias"))
    return Layers.ToImage(tokens, height, width) + x


def unit(model: ModelBuilder, W: WeightSet, cfg: SdxlConfig, x, silu_temb, context, prefix: str, index: int,
         level: int, kv_all=None):
    """UNetModel.Unit (:306-318): a resnet, then the level's transformers."""
    x = resnet_block(model, W, cfg, x, silu_temb, f"{prefix}.resnets.{index}")
    layers = cfg.transformer_layers[level]
    if layers:
        x = transformer2d(model, W, cfg, x, context, f"{prefix}.attentions.{index}", cfg.heads[level], layers, kv_all)
    return x


def build_unet(device: Device, cfg: SdxlConfig, weights: dict, batch: int, latent_h: int, latent_w: int,
               tokens: int = 77, compute: HostDataType = HostDataType.Float16, int8: bool = False) -> ModelBuilder:
    """UNetModel.Build (:328-426) as one compiled model (every GraphChain cut
    is a no-op: the whole UNet stays resident). Inputs at the compute type:
    sample [B, 4, h, w], time [B, 1, 1, c0] (timestep_embedding), add [B,
    1, 1, add_width] (add_conditioning), context [B, 1, tokens, 2048].
    Output: the predicted noise [B, 4, h, w]."""
    model = ModelBuilder(device, compute, int8)
    W = WeightSet(model, weights, compute, device)
    sample = model.Placeholder([batch, cfg.in_channels, latent_h, latent_w], compute)
    time = model.Placeholder([batch, 1, 1, cfg.block_out[0]], compute)
    add = model.Placeholder([batch, 1, 1, cfg.add_width], compute)
    context = model.Placeholder([batch, 1, tokens, cfg.context_width], compute)

    kv_all = context_kv(model, W, context)
    temb = embedding_mlp(model, W, time, "time_embedding") + embedding_mlp(model, W, add, "add_embedding")
    silu_temb = Layers.Silu(temb)
    skips = [Layers.Conv2d(model, sample, W("conv_in.weight"), W("conv_in.bias", "norm"))]
    levels = len(cfg.block_out)
    for level in range(levels):
        prefix = f"down_blocks.{level}"
        for i in range(cfg.layers_per_block):
            skips.append(unit(model, W, cfg, skips[-1], silu_temb, context, prefix, i, level, kv_all))
        if level != levels - 1:
            skips.append(Layers.Conv2d(model, skips[-1], W(f"{prefix}.downsamplers.0.conv.weight"),
                                       W(f"{prefix}.downsamplers.0.conv.bias", "norm"), stride=2, padding=1))

    x = resnet_block(model, W, cfg, skips[-1], silu_temb, "mid_block.resnets.0")
    x = transformer2d(model, W, cfg, x, context, "mid_block.attentions.0", cfg.heads[-1], cfg.transformer_layers[-1],
                      kv_all)
    x = resnet_block(model, W, cfg, x, silu_temb, "mid_block.resnets.1")

    for i in range(levels):
        level = levels - 1 - i
        prefix = f"up_blocks.{i}"
        for j in range(cfg.layers_per_block + 1):
            x = Ops.Join([x, skips.pop()], 1)
            x = unit(model, W, cfg, x, silu_temb, context, prefix, j, level, kv_all)
        if i != levels - 1:
            nxt = skips[-1].Shape
            x = Layers.Conv2d(model, Layers.CropTo(Layers.UpsampleNearest(x), nxt[2], nxt[3]),
                              W(f"{prefix}.upsamplers.0.conv.weight"), W(f"{prefix}.upsamplers.0.conv.bias", "norm"))

    x = Layers.GroupNorm(model, x, W("conv_norm_out.weight", "norm"), W("conv_norm_out.bias", "norm"), cfg.groups,
                         cfg.eps, silu=True)
    noise = Layers.Conv2d(model, x, W("conv_out.weight"), W("conv_out.bias", "norm"))
    model.Compile([noise])
    W.release()
    return model


class UNetModel:
    """IDenoiser over the compiled UNet (Pipeline/IDenoiser.cs:16-17;
    UNetModel.Predict, :86-107): Predict(latent, timestep, sigma,
    conditioning) -> noise, host tensors in and out; conditioning holds
    'add' [add_width] and 'context' [tokens, 2048]."""

    def __init__(self, device: Device, cfg: SdxlConfig, weights: dict, height: int, width: int, tokens: int = 77,
                 batch: int = 1, compute: HostDataType = HostDataType.Float16, int8: bool = False):
        self.cfg, self.batch, self.tokens, self.compute = cfg, batch, tokens, compute
        self.latent_h, self.latent_w = height // 8, width // 8
        self.model = build_unet(device, cfg, weights, batch, self.latent_h, self.latent_w, tokens, compute, int8)

    def Predict(self, latent: HostTensor, timestep: float, sigma: float, conditioning: dict) -> HostTensor:
        cfg, B = self.cfg, self.batch
        t = np.tile(timestep_embedding([timestep], cfg.block_out[0]), (B, 1)).reshape(B, 1, 1, -1)
        add = np.asarray(conditioning["add"], np.float32).reshape(-1, cfg.add_width)
        add = np.broadcast_to(add, (B, cfg.add_width)).reshape(B, 1, 1, cfg.add_width)
        ctx = np.asarray(conditioning["context"], np.float32).reshape(-1, self.tokens, cfg.context_width)
        ctx = np.broadcast_to(ctx, (B, self.tokens, cfg.context_width)).reshape(B, 1, self.tokens, cfg.context_width)
        c = self.compute
        ins = [latent.ConvertTo(c).Reshape(B, cfg.in_channels, self.latent_h, self.latent_w),
               HostTensor.FromFloats(np.ascontiguousarray(t)).ConvertTo(c),
               HostTensor.FromFloats(np.ascontiguousarray(add)).ConvertTo(c),
               HostTensor.FromFloats(np.ascontiguousarray(ctx)).ConvertTo(c)]
        return self.model.Run(*ins)[0]

    def Dispose(self):
        self.model.Dispose()


# ---- LoRAs (Models/Sdxl/SdxlLoras.cs) ------------------------------------------------------

LORA_UNET, LORA_TEXT_ENCODER, LORA_TEXT_ENCODER_2 = "unet", "te1", "te2"


def lora_layout():
    """SdxlLoras.Layout (SdxlLoras.cs:11-28): the UNet and the two CLIP
    towers; a kohya lora_te_ file (one text tower) is refused as SD 1.x/2.x."""
    from .lora import LoraLayout, LoraTower
    return LoraLayout("SDXL", [LoraTower(LORA_UNET, "UNet", "unet", "unet"),
                               LoraTower(LORA_TEXT_ENCODER, "CLIP-L", "te1", "text_encoder"),
                               LoraTower(LORA_TEXT_ENCODER_2, "CLIP-G", "te2", "text_encoder_2")],
                      {"te": "was trained for Stable Diffusion 1.x or 2.x, which has one text tower where SDXL has two"})
