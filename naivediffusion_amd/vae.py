"""The latent-diffusion VAE's decoder (AutoencoderKL, Vae/AutoencoderKl.cs) on
the denoiser's kernels: the implicit-GEMM convolutions, the split-statistics
GroupNorm with SiLU fused, nearest upsampling, and the mid block's
single-head attention over every pixel.

The reference builds the decoder as one DirectML graph at float32
(ModelBuilder's default width) and, where DirectML's scratch would not fit,
decodes in overlapping 64-cell tiles blended together (Vae/TiledVae.cs). On
MI355X the whole image fits with room to spare (a 1024x1024 decode at bf16
holds about 3 GB of temporaries), so the decoder runs untiled, as one
compiled model, at the compute width the caller picks.

The attention is the reference's: q k^T, softmax of it scaled by 1/sqrt(C),
times v (AutoencoderKl.AttentionBlock, :40-63) with its head of C = 512
features. It runs as two MFMA products with the [tokens, tokens] scores
between them (0.5 GB at bf16 for a 1024x1024 image) and a row softmax that
applies the scale; v is transposed once so both products read their operands
in rows.
"""

from __future__ import annotations

import dataclasses
import math
from typing import Dict, Sequence, Tuple

import numpy as np

from . import rng
from .graph import ModelBuilder, Ops
from .layers import Layers
from .tensors import Device, DeviceTensor, HostDataType, HostTensor
from .weights import WeightSet

F32 = HostDataType.Float32


@dataclasses.dataclass(frozen=True)
class VaeConfig:
    """VaeConfig (Vae/VaeConfig.cs) with its LatentSpace (Vae/LatentSpace.cs):
    widths per level (highest resolution first), resnets per encoder level
    (the decoder has one more), the GroupNorm groups and epsilon, the latent's
    channels, pixels per cell and its scaling/shift."""
    block_out: Tuple[int, ...] = (128, 256, 512, 512)
    layers_per_block: int = 2
    groups: int = 32
    eps: float = 1e-6
    latent_channels: int = 4
    scale_factor: int = 8
    scaling_factor: float = 0.13025
    shift_factor: float = 0.0
    image_channels: int = 3


# SdxlVae.Config and SdxlVae.Latent (Models/Sdxl/SdxlVae.cs:11-31).
SDXL = VaeConfig()


def _resnet_shapes(out: dict, p: str, cin: int, cout: int):
    out.update({f"{p}.norm1.weight": (cin,), f"{p}.norm1.bias": (cin,),
                f"{p}.conv1.weight": (cout, cin, 3, 3), f"{p}.conv1.bias": (cout,),
                f"{p}.norm2.weight": (cout,), f"{p}.norm2.bias": (cout,),
                f"{p}.conv2.weight": (cout, cout, 3, 3), f"{p}.conv2.bias": (cout,)})
    if cin != cout:
        out.update({f"{p}.conv_shortcut.weight": (cout, cin, 1, 1), f"{p}.conv_shortcut.bias": (cout,)})


def decoder_weight_shapes(cfg: VaeConfig) -> Dict[str, tuple]:
    """The decoder's tensors under diffusers' names, as AutoencoderKl.Decoder
    reads them (:72-112)."""
    lc = cfg.latent_channels
    widths = list(reversed(cfg.block_out))
    top = widths[0]
    out = {"post_quant_conv.weight": (lc, lc, 1, 1), "post_quant_conv.bias": (lc,),
           "decoder.conv_in.weight": (top, lc, 3, 3), "decoder.conv_in.bias": (top,)}
    _resnet_shapes(out, "decoder.mid_block.resnets.0", top, top)
    a = "decoder.mid_block.attentions.0"
    out.update({f"{a}.group_norm.weight": (top,), f"{a}.group_norm.bias": (top,)})
    for n in ("to_q", "to_k", "to_v", "to_out.0"):
        out.update({f"{a}.{n}.weight": (top, top), f"{a}.{n}.bias": (top,)})
    _resnet_shapes(out, "decoder.mid_block.resnets.1", top, top)
    cin = top
    for i, c in enumerate(widths):
        for j in range(cfg.layers_per_block + 1):
            _resnet_shapes(out, f"decoder.up_blocks.{i}.resnets.{j}", cin, c)
            cin = c
        if i != len(widths) - 1:
            out.update({f"decoder.up_blocks.{i}.upsamplers.0.conv.weight": (c, c, 3, 3),
                        f"decoder.up_blocks.{i}.upsamplers.0.conv.bias": (c,)})
    out.update({"decoder.conv_norm_out.weight": (cin,), "decoder.conv_norm_out.bias": (cin,),
                "decoder.conv_out.weight": (cfg.image_channels, cin, 3, 3),
                "decoder.conv_out.bias": (cfg.image_channels,)})
    return out


def _is_norm(name: str) -> bool:
    return ".norm" in name or ".group_norm" in name or "conv_norm_out" in name


def synthetic_weights(cfg: VaeConfig, seed: int, dtype: HostDataType = F32) -> Dict[str, np.ndarray]:
    """Host weights (fp32 arrays holding values exact at dtype): norm weights
    1 and biases 0 plus a small seeded spread; filters and matrices
    N(0, 1/fan_in), so activations keep their scale through the depth;
    biases N(0, 0.02)."""
    out = {}
    for name, shape in decoder_weight_shapes(cfg).items():
        s = rng.tensor_seed(seed, name)
        if _is_norm(name):
            v = (1.0 if name.endswith("weight") else 0.0) + rng.normal(s, shape, 0.0, 0.05)
        elif len(shape) == 1:
            v = rng.normal(s, shape, 0.0, 0.02)
        else:
            v = rng.normal(s, shape, 0.0, 1.0 / math.sqrt(int(np.prod(shape[1:]))))
        out[name] = HostTensor.FromFloats(np.asarray(v, np.float32)).ConvertTo(dtype).ToFloats().reshape(shape)
    return out


def device_weights(device: Device, cfg: VaeConfig, seed: int, dtype: HostDataType = HostDataType.BFloat16) -> dict:
    """Synthetic weights made on the GPU at dtype: filters and matrices
    N(0, 1/fan_in), biases N(0, 0.02), norm weights 1, norm biases 0."""
    out = {}
    for name, shape in decoder_weight_shapes(cfg).items():
        if _is_norm(name):
            v = np.full(shape, 1.0 if name.endswith("weight") else 0.0, np.float32)
            out[name] = device.Upload(HostTensor.FromFloats(v).ConvertTo(dtype))
        else:
            std = 0.02 if len(shape) == 1 else 1.0 / math.sqrt(int(np.prod(shape[1:])))
            out[name] = device.Normal(dtype, shape, rng.tensor_seed(seed, name), 0.0, std)
    return out


def resnet_block(model: ModelBuilder, W: WeightSet, cfg: VaeConfig, x, p: str):
    """AutoencoderKl.ResnetBlock (:16-35): the SiLU fused into each
    GroupNorm, the residual (1x1-projected when the width changes) into the
    second convolution's epilogue."""
    v = lambda n: W(f"{p}.{n}", "norm")
    h = Layers.GroupNorm(model, x, v("norm1.weight"), v("norm1.bias"), cfg.groups, cfg.eps, silu=True)
    h = Layers.Conv2d(model, h, W(f"{p}.conv1.weight"), v("conv1.bias"))
    h = Layers.GroupNorm(model, h, v("norm2.weight"), v("norm2.bias"), cfg.groups, cfg.eps, silu=True)
    if W.has(f"{p}.conv_shortcut.weight"):
        x = Layers.Conv2d(model, x, W(f"{p}.conv_shortcut.weight"), v("conv_shortcut.bias"), padding=0)
    return Layers.Conv2d(model, h, W(f"{p}.conv2.weight"), v("conv2.bias"), residual=x)


def attention_block(model: ModelBuilder, W: WeightSet, cfg: VaeConfig, x, p: str):
    """AutoencoderKl.AttentionBlock (:40-63): GroupNorm, to tokens, the q/k/v
    projections as one stacked GEMM, softmax(q k^T / sqrt(C)) v as two
    products around a row softmax, the output projection, back to the image
    plus the input."""
    _, c, height, width = x.Shape
    n = height * width
    v = lambda name: W(f"{p}.{name}", "norm")
    normed = Layers.GroupNorm(model, x, v("group_norm.weight"), v("group_norm.bias"), cfg.groups, cfg.eps)
    tokens = Layers.ToTokens(normed)
    qkv = Layers.Linear(model, tokens, W.stacked([f"{p}.to_q.weight", f"{p}.to_k.weight", f"{p}.to_v.weight"]),
                        W.stacked([f"{p}.to_q.bias", f"{p}.to_k.bias", f"{p}.to_v.bias"], "norm"))
    q, k, val = (Ops.Slice(qkv, [0, 0, 0, i * c], [1, 1, n, c]) for i in range(3))
    scores = Layers.Linear(model, q, k)                       # q k^T: the keys are the product's weight rows
    probs = Ops.ActivationSoftmax(scores, 1.0 / math.sqrt(c))
    # v^T packed: [C, tokens] rows, so the second product also reads rows
    vt = Ops.Identity(Ops.Reinterpret(val, [1, 1, c, n], [n * 3 * c, n * 3 * c, 1, 3 * c]))
    attended = Layers.Linear(model, probs, vt)
    projected = Layers.Linear(model, attended, W(f"{p}.to_out.0.weight"), v("to_out.0.bias"))
    return Layers.ToImage(projected, height, width) + x


def build_decoder(device: Device, cfg: VaeConfig, weights: dict, height: int, width: int,
                  compute: HostDataType = HostDataType.BFloat16) -> ModelBuilder:
    """AutoencoderKl.Decoder (:72-112) as one compiled model, with
    LatentSpace.FromModelScale (Vae/LatentSpace.cs:30-46) at its start.
    Input: the sampler's latent [1, C, height/8, width/8] in float32, in the
    model's scale. Output: the image [1, 3, height, width] at the compute
    width, roughly in [-1, 1]."""
    f = cfg.scale_factor
    if height % f or width % f:
        raise ValueError(f"{width}x{height} does not divide into {f}-pixel cells")
    model = ModelBuilder(device, compute)
    W = WeightSet(model, weights, compute, device)
    latent = model.Placeholder([1, cfg.latent_channels, height // f, width // f], F32)
    # FromModelScale: latent / scaling + shift, in float32 as the host loop does it
    scaling = model.Constant(HostTensor.FromFloats(np.full(1, cfg.scaling_factor, np.float32)), [1, 1, 1, 1], F32)
    z = latent / Layers.Broadcast(scaling, latent.Shape)
    if cfg.shift_factor:
        z = z + float(np.float32(cfg.shift_factor))
    z = Layers.Cast(z, compute)
    v = lambda n: W(n, "norm")
    h = Layers.Conv2d(model, z, W("post_quant_conv.weight"), v("post_quant_conv.bias"), padding=0)
    h = Layers.Conv2d(model, h, W("decoder.conv_in.weight"), v("decoder.conv_in.bias"))
    h = resnet_block(model, W, cfg, h, "decoder.mid_block.resnets.0")
    h = attention_block(model, W, cfg, h, "decoder.mid_block.attentions.0")
    h = resnet_block(model, W, cfg, h, "decoder.mid_block.resnets.1")
    for i in range(len(cfg.block_out)):
        p = f"decoder.up_blocks.{i}"
        for j in range(cfg.layers_per_block + 1):
            h = resnet_block(model, W, cfg, h, f"{p}.resnets.{j}")
        if W.has(f"{p}.upsamplers.0.conv.weight"):
            h = Layers.Conv2d(model, Layers.UpsampleNearest(h), W(f"{p}.upsamplers.0.conv.weight"),
                              v(f"{p}.upsamplers.0.conv.bias"))
    h = Layers.GroupNorm(model, h, v("decoder.conv_norm_out.weight"), v("decoder.conv_norm_out.bias"), cfg.groups,
                         cfg.eps, silu=True)
    image = Layers.Conv2d(model, h, W("decoder.conv_out.weight"), v("decoder.conv_out.bias"))
    model.Compile([image])
    W.release()
    return model


def decoder_flops(cfg: VaeConfig, height: int, width: int) -> float:
    """Algorithmic flops of one decode: 2 per multiply-add of every
    convolution, linear and attention product."""
    total = 0.0
    shapes = decoder_weight_shapes(cfg)
    h, w = height // cfg.scale_factor, width // cfg.scale_factor
    levels = list(reversed(cfg.block_out))

    def conv(name, hh, ww):
        co, ci, kh, kw = shapes[name]
        return 2.0 * co * ci * kh * kw * hh * ww

    total += conv("post_quant_conv.weight", h, w) + conv("decoder.conv_in.weight", h, w)

    def resnet(p, hh, ww):
        t = conv(f"{p}.conv1.weight", hh, ww) + conv(f"{p}.conv2.weight", hh, ww)
        if f"{p}.conv_shortcut.weight" in shapes:
            t += conv(f"{p}.conv_shortcut.weight", hh, ww)
        return t

    c, n = levels[0], h * w
    total += resnet("decoder.mid_block.resnets.0", h, w) + resnet("decoder.mid_block.resnets.1", h, w)
    total += 2.0 * n * c * c * 4 + 2.0 * 2 * n * n * c
    for i in range(len(levels)):
        p = f"decoder.up_blocks.{i}"
        for j in range(cfg.layers_per_block + 1):
            total += resnet(f"{p}.resnets.{j}", h, w)
        if f"{p}.upsamplers.0.conv.weight" in shapes:
            h, w = 2 * h, 2 * w
            total += conv(f"{p}.upsamplers.0.conv.weight", h, w)
    total += conv("decoder.conv_out.weight", h, w)
    return total


class AutoencoderKlDecoder:
    """ILatentDecoder (VaeLatentCodec.Decoder, Vae/VaeLatentCodec.cs:142-157)
    over the compiled decoder: Decode(latent in the model's scale) -> image
    [1, 3, H, W]; DecodeOnDevice keeps the latent and the image in HBM."""

    def __init__(self, device: Device, cfg: VaeConfig, weights: dict, height: int, width: int,
                 compute: HostDataType = HostDataType.BFloat16):
        self.cfg, self.height, self.width = cfg, height, width
        self.model = build_decoder(device, cfg, weights, height, width, compute)

    @property
    def TemporaryBytes(self) -> int:
        return self.model.TemporarySize

    def Decode(self, latent) -> np.ndarray:
        f = self.cfg.scale_factor
        x = HostTensor.FromFloats(np.asarray(latent, np.float32).reshape(
            1, self.cfg.latent_channels, self.height // f, self.width // f))
        return self.model.Run(x)[0].ToFloats()

    def DecodeOnDevice(self, latent: DeviceTensor) -> DeviceTensor:
        (out,) = self.model.RunOnDevice(latent)
        return out

    def Dispose(self):
        self.model.Dispose()
