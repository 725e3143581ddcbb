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


# ---- Wan 2.2's VAE on one frame: Qwen-Image 2.1's decoder (Vae/Wan22Vae.cs, Vae/WanVae.cs) -------------

# Wan22Vae.Latent (Vae/Wan22Vae.cs:43-101): Qwen-Image 2.1's 64-channel latent, 16 pixels a cell,
# standardised channel by channel (StandardizedLatentSpace, Vae/LatentSpace.cs:95-128).
WAN22_MEANS = (
    0.5126, 0.7721, -0.0631, 1.3506, -0.7855, -2.1025, -0.3458, 1.3722,
    1.8873, -1.7177, -0.6510, 0.2732, 0.7562, -0.6163, -1.0277, 3.8363,
    2.0210, 0.0472, 0.9320, 2.0087, 2.4954, -0.1391, -1.4249, 1.8464,
    -0.5236, 1.2826, 3.7046, -1.3035, 2.7286, -1.4518, -1.9036, -1.9955,
    -0.0342, -1.0265, -0.7636, 3.0555, 0.0746, -3.0751, -0.1076, 1.7376,
    -1.0914, -1.9435, -0.2784, -1.3680, 0.4809, -0.4433, 0.3764, 0.5729,
    -2.0595, 1.0960, -1.3260, -2.0211, -5.0179, 0.5275, 4.0162, 1.8505,
    0.3026, 1.9373, 1.4937, 0.2632, 0.5547, -1.7121, -0.1562, 0.0304)
WAN22_DEVIATIONS = (
    3.2001, 3.2936, 3.4321, 3.0091, 3.1061, 4.0379, 4.0705, 3.7910,
    3.0785, 3.6500, 3.9308, 3.0904, 2.8778, 3.7675, 3.7320, 5.0756,
    3.2864, 4.0397, 3.1317, 4.0443, 2.9249, 3.9454, 3.0988, 4.2489,
    3.4896, 3.8513, 3.9323, 3.4719, 3.7498, 4.2830, 3.5694, 4.2467,
    3.9037, 3.2947, 5.0770, 3.5075, 3.2700, 3.4767, 2.8063, 5.1125,
    3.5327, 4.7833, 3.1286, 4.1819, 3.8527, 3.8312, 3.5605, 4.3875,
    3.9624, 4.0168, 3.5643, 4.0550, 5.5614, 4.2963, 4.4080, 3.4959,
    3.8747, 3.7608, 3.5735, 3.1490, 3.7662, 3.6746, 3.4563, 3.8161)
# Which of the image-side levels also halved time in the video model
# (Wan22Vae.TemporalLevels, :37); the decoder's level L mirrors entry
# levels - 2 - L.
WAN22_TEMPORAL = (False, True, True, True)


@dataclasses.dataclass(frozen=True)
class Wan22Config:
    """The decoder's shape: the latent's channels, the width of each level
    from the latent (the last one's is the head's input), resnets per level
    (three in the decoder) and the image channels the head makes (four:
    RGB and an alpha the decoder cuts)."""
    latent_channels: int = 64
    widths: Tuple[int, ...] = (1152, 1152, 576, 288, 144)
    resnets: int = 3
    image_channels: int = 4
    scale_factor: int = 16


WAN22 = Wan22Config()


def _wan_residual_shapes(out: dict, p: str, cin: int, cout: int):
    out.update({f"{p}.residual.0.gamma": (cin,), f"{p}.residual.2.weight": (cout, cin, 3, 3),
                f"{p}.residual.2.bias": (cout,), f"{p}.residual.3.gamma": (cout,),
                f"{p}.residual.6.weight": (cout, cout, 3, 3), f"{p}.residual.6.bias": (cout,)})
    if cin != cout:
        out.update({f"{p}.shortcut.weight": (cout, cin, 1, 1), f"{p}.shortcut.bias": (cout,)})


def wan22_decoder_shapes(cfg: Wan22Config = WAN22) -> Dict[str, tuple]:
    """The single-frame decoder's tensors (WanVae.SingleFrame's names: the
    temporal taps cut, gammas flat) as Wan22Vae.Decoder reads them
    (:191-238). Each level: the first resnet takes the level's input width
    to its own, the resample convolution after the upsample keeps it."""
    lc, w = cfg.latent_channels, cfg.widths
    out = {"conv2.weight": (lc, lc, 1, 1), "conv2.bias": (lc,),
           "decoder.conv1.weight": (w[0], lc, 3, 3), "decoder.conv1.bias": (w[0],)}
    _wan_residual_shapes(out, "decoder.middle.0", w[0], w[0])
    out.update({"decoder.middle.1.norm.gamma": (w[0],), "decoder.middle.1.to_qkv.weight": (3 * w[0], w[0], 1, 1),
                "decoder.middle.1.to_qkv.bias": (3 * w[0],), "decoder.middle.1.proj.weight": (w[0], w[0], 1, 1),
                "decoder.middle.1.proj.bias": (w[0],)})
    _wan_residual_shapes(out, "decoder.middle.2", w[0], w[0])
    cin = w[0]
    for level, c in enumerate(w):
        p = f"decoder.upsamples.{level}.upsamples"
        for i in range(cfg.resnets):
            _wan_residual_shapes(out, f"{p}.{i}", cin if i == 0 else c, c)
        if level != len(w) - 1:
            out.update({f"{p}.{cfg.resnets}.resample.1.weight": (c, c, 3, 3),
                        f"{p}.{cfg.resnets}.resample.1.bias": (c,)})
        cin = c
    out.update({"decoder.head.0.gamma": (cin,), "decoder.head.2.weight": (cfg.image_channels, cin, 3, 3),
                "decoder.head.2.bias": (cfg.image_channels,)})
    return out


def wan22_synthetic_weights(cfg: Wan22Config, seed: int, dtype: HostDataType = F32) -> Dict[str, np.ndarray]:
    """Host weights exact at dtype: gammas 1 plus a small seeded spread,
    filters N(0, 1/fan_in), biases N(0, 0.02)."""
    out = {}
    for name, shape in wan22_decoder_shapes(cfg).items():
        s = rng.tensor_seed(seed, name)
        if name.endswith(".gamma"):
            v = 1.0 + rng.normal(s, shape, 0.0, 0.05)
        elif len(shape) == 1:
            v = rng.normal(s, shape, 0.0, 0.02)
        else:
            v = rng.normal(s, shape, 0.0, 1.0 / math.sqrt(int(np.prod(shape[1:]))))
        out[name] = HostTensor.FromFloats(np.asarray(v, np.float32)).ConvertTo(dtype).ToFloats().reshape(shape)
    return out


def wan22_device_weights(device: Device, cfg: Wan22Config, seed: int,
                         dtype: HostDataType = HostDataType.BFloat16) -> dict:
    out = {}
    for name, shape in wan22_decoder_shapes(cfg).items():
        if name.endswith(".gamma"):
            out[name] = device.Upload(HostTensor.FromFloats(np.ones(shape, np.float32)).ConvertTo(dtype))
        else:
            std = 0.02 if len(shape) == 1 else 1.0 / math.sqrt(int(np.prod(shape[1:])))
            out[name] = device.Normal(dtype, shape, rng.tensor_seed(seed, name), 0.0, std)
    return out


def single_frame(raw: Dict[str, np.ndarray]) -> Dict[str, np.ndarray]:
    """WanVae.SingleFrame (Vae/WanVae.cs:48-99) for host arrays: the
    temporal-resampling convolutions dropped, gammas flattened to [C], 3-D
    kernels [out, in, t, kh, kw] cut to their last temporal tap (the only
    one that sees the frame through a causal convolution)."""
    out = {}
    for name, t in raw.items():
        if ".time_conv." in name:
            continue
        a = np.asarray(t)
        if name.endswith(".gamma"):
            out[name] = a.reshape(a.shape[0])
        elif a.ndim == 5:
            out[name] = np.ascontiguousarray(a[:, :, -1])
        else:
            out[name] = a
    return out


def _channel_rms_tokens(model: ModelBuilder, W: WeightSet, x, gamma: str):
    """WanVae.ChannelRmsNorm (Vae/WanVae.cs:103-113): x / sqrt(mean over
    channels of x^2 + 1e-24 / C) * gamma, as a row RMSNorm of the tokens
    [1, 1, H*W, C]; the result is packed tokens (NHWC)."""
    c = x.Shape[1]
    return Ops.MeanVarianceNormalization2(Layers.ToTokens(x), [3], False, 1e-24 / c, W(gamma, "norm"))


def _tokens_to_image(t, height: int, width: int):
    return Layers.ToImage(t, height, width)


def wan_residual_block(model: ModelBuilder, W: WeightSet, x, p: str):
    """WanVae.ResidualBlock (:121-132): RMS norm over channels, SiLU, 3x3
    convolution, twice, plus the input (1x1-projected when the width
    changes), the sum fused into the second convolution's epilogue."""
    _, _, h, w = x.Shape
    v = lambda n: W(f"{p}.{n}", "norm")
    t = Layers.Silu(_channel_rms_tokens(model, W, x, f"{p}.residual.0.gamma"))
    y = Layers.Conv2d(model, _tokens_to_image(t, h, w), W(f"{p}.residual.2.weight"), v("residual.2.bias"))
    t = Layers.Silu(_channel_rms_tokens(model, W, y, f"{p}.residual.3.gamma"))
    if W.has(f"{p}.shortcut.weight"):
        x = Layers.Conv2d(model, x, W(f"{p}.shortcut.weight"), v("shortcut.bias"), padding=0)
    return Layers.Conv2d(model, _tokens_to_image(t, h, w), W(f"{p}.residual.6.weight"), v("residual.6.bias"),
                         residual=x)


def _as_matrix(W: WeightSet, name: str):
    """A 1x1 convolution's [out, in, 1, 1] filter as the [out, in] weight of
    a linear over tokens (the same product)."""
    w = W(name)
    o, i = w.Shape[0], w.Shape[1]
    return Ops.Reinterpret(w, [1, 1, o, i])


def wan_attention_block(model: ModelBuilder, W: WeightSet, x, p: str):
    """WanVae.AttentionBlock (:134-151): RMS norm over channels, the 1x1
    q/k/v projection (as a linear over the tokens), softmax(q k^T / sqrt(C))
    v with one head of C features (two MFMA products around the row
    softmax), the 1x1 output projection, plus the input."""
    _, c, height, width = x.Shape
    n = height * width
    v = lambda name: W(f"{p}.{name}", "norm")
    t = _channel_rms_tokens(model, W, x, f"{p}.norm.gamma")
    qkv = Layers.Linear(model, t, _as_matrix(W, f"{p}.to_qkv.weight"), v("to_qkv.bias"))
    q, k, val = (Ops.Slice(qkv, [0, 0, 0, i * c], [1, 1, n, c]) for i in range(3))
    probs = Ops.ActivationSoftmax(Layers.Linear(model, q, k), 1.0 / math.sqrt(c))
    vt = Ops.Identity(Ops.Reinterpret(val, [1, 1, c, n], [n * 3 * c, n * 3 * c, 1, 3 * c]))
    attended = Layers.Linear(model, probs, vt)
    projected = Layers.Linear(model, attended, _as_matrix(W, f"{p}.proj.weight"), v("proj.bias"))
    return Layers.ToImage(projected, height, width) + x


def up_shortcut(x, out_channels: int, temporal: bool):
    """Wan22Vae.UpShortcut (:153-189), DupUp3D on one frame: the same width
    is a nearest upsample; half the width is the odd input channels
    upsampled on a level that doubled time, and otherwise output channel o
    takes its even rows from input channel 2o and its odd rows from 2o + 1,
    each pixel repeated across. x is packed [1, C, H, W]; the interleave is
    two strided copies."""
    _, c, h, w = x.Shape
    if c == out_channels:
        return Layers.UpsampleNearest(x)
    if c != 2 * out_channels:
        raise ValueError(f"an up level halves its channels at most, not {c} to {out_channels}")
    if temporal:
        return Layers.UpsampleNearest(Ops.Slice(x, [0, 1, 0, 0], [1, c - 1, h, w], [1, 2, 1, 1]))
    o = out_channels
    # (o, y, r, x) <- channel 2o + r, row y: packed, this is [o, 2h, w]
    rows = Ops.Identity(Ops.Reinterpret(x, [o, h, 2, w], [2 * h * w, w, h * w, 1]))
    # every pixel twice across: [o * 2h, w, 2] with the last axis a repeat
    wide = Ops.Identity(Ops.Reinterpret(rows, [1, o * 2 * h, w, 2], [o * 2 * h * w, w, 1, 0]))
    return Ops.Reinterpret(wide, [1, o, 2 * h, 2 * w])


def build_wan22_decoder(device: Device, cfg: Wan22Config, weights: dict, height: int, width: int,
                        compute: HostDataType = HostDataType.BFloat16) -> ModelBuilder:
    """Wan22Vae.Decoder (Vae/Wan22Vae.cs:191-238) as one compiled model,
    with StandardizedLatentSpace.FromModelScale (latent * deviation + mean
    per channel, Vae/LatentSpace.cs:113-126) at its start. Input: the
    sampler's latent [1, 64, height/16, width/16] in float32. Output: the
    RGB image [1, 3, height, width] at the compute width (the head's fourth,
    alpha, channel cut as the reference cuts it). Widths are read from the
    weights, as the reference reads them."""
    f = cfg.scale_factor
    if height % f or width % f:
        raise ValueError(f"{width}x{height} does not divide into {f}-pixel cells")
    lc = cfg.latent_channels
    model = ModelBuilder(device, compute)
    W = WeightSet(model, weights, compute, device)
    latent = model.Placeholder([1, lc, height // f, width // f], F32)
    dev = model.Constant(HostTensor.FromFloats(np.asarray(WAN22_DEVIATIONS[:lc], np.float32)), [1, lc, 1, 1], F32)
    mean = model.Constant(HostTensor.FromFloats(np.asarray(WAN22_MEANS[:lc], np.float32)), [1, lc, 1, 1], F32)
    z = latent * Layers.Broadcast(dev, latent.Shape) + Layers.Broadcast(mean, latent.Shape)
    z = Layers.Cast(z, compute)
    v = lambda n: W(n, "norm")
    h = Layers.Conv2d(model, z, W("conv2.weight"), v("conv2.bias"), padding=0)
    h = Layers.Conv2d(model, h, W("decoder.conv1.weight"), v("decoder.conv1.bias"))
    h = wan_residual_block(model, W, h, "decoder.middle.0")
    h = wan_attention_block(model, W, h, "decoder.middle.1")
    h = wan_residual_block(model, W, h, "decoder.middle.2")
    levels = 0
    while W.has(f"decoder.upsamples.{levels}.upsamples.0.residual.0.gamma"):
        levels += 1
    for level in range(levels):
        p = f"decoder.upsamples.{level}.upsamples"
        level_in = h
        index = 0
        while W.has(f"{p}.{index}.residual.0.gamma"):
            h = wan_residual_block(model, W, h, f"{p}.{index}")
            index += 1
        if level != levels - 1:
            # The up-shortcut's sum rides the resample convolution's residual
            # epilogue (the product rounded first, as the separate add has it).
            wr = W(f"{p}.{index}.resample.1.weight")
            shortcut = up_shortcut(level_in, wr.Shape[0], WAN22_TEMPORAL[levels - 2 - level])
            h = Layers.Conv2d(model, Layers.UpsampleNearest(h), wr, v(f"{p}.{index}.resample.1.bias"),
                              residual=shortcut)
    _, c, hh, ww = h.Shape
    t = Layers.Silu(_channel_rms_tokens(model, W, h, "decoder.head.0.gamma"))
    image = Layers.Conv2d(model, Layers.ToImage(t, hh, ww), W("decoder.head.2.weight"), v("decoder.head.2.bias"))
    if image.Shape[1] != cfg.image_channels:
        raise ValueError(f"the decoder makes {image.Shape[1]} channels, not {cfg.image_channels}")
    rgb = Ops.Identity(Ops.Slice(image, [0, 0, 0, 0], [1, 3, height, width]))
    model.Compile([rgb])
    W.release()
    return model


class Wan22Decoder:
    """ILatentDecoder for Qwen-Image 2.1 (QwenImageLatentCodec over
    Wan22Vae.Decoder): Decode(latent in the model's scale) -> [1, 3, H, W]."""

    def __init__(self, device: Device, cfg: Wan22Config, weights: dict, height: int, width: int,
                 compute: HostDataType = HostDataType.BFloat16):
        self.cfg, self.height, self.width = cfg, height, width
        self.model = build_wan22_decoder(device, cfg, weights, height, width, compute)

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
