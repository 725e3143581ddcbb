"""Anima's diffusion transformer (Cosmos-Predict2 2B on one frame) on the
device: Models/Anima/AnimaDit.cs.

Twenty-eight single-stream blocks over the 2x2 patches of a 16-channel
latent, each self-attention with 3-D rotary positions (AnimaDit.RopeTables,
:149-188), cross-attention into the 512 x 1024 adapter context and an
exact-GELU MLP, all three modulated and gated from the time embedding
through a low-rank adaLN plus a shared term (Modulation, :270-291). No
linear has a bias. Built from the same per-layer primitives as the
reference (Layers.Linear, Transformer.Modulate, HeadNorm, Rotate,
Layers.Attend, the gated residual), with the MI355X path's fused kernels:
the three self-attention projections run as one GEMM over their stacked
weights, so do the cross-attention's key and value projections, and the
patch layouts at both ends run on the device.

Precision follows AnimaDit.cs:46-70: weights are stored narrow (fp16 at
fp32 compute, else at the compute type), the residual stream, the norms,
the rotary positions, the embeddings and the final layer stay fp32, and
at half/bf16 compute the products and the attention run narrow. The
context enters the blocks at the compute type (one cast at the start).
"""

from __future__ import annotations

import dataclasses
from typing import Dict

import numpy as np

from . import rng
from .chain import GraphChain
from .graph import PATCH_CHANNEL_FIRST, PATCH_CHANNEL_LAST, ModelBuilder, Ops
from .layers import Layers, Transformer
from .tensors import Device, DeviceTensor, HostDataType, HostTensor, bf16_to_f32, f32_to_bf16
from .weights import WeightSet

ROPE_THETA = 10000.0
NTK_EXTRAPOLATION = 4.0


@dataclasses.dataclass(frozen=True)
class AnimaConfig:
    width: int = 2048          # D
    heads: int = 16            # head size D / H = 128
    mlp: int = 8192
    blocks: int = 28
    latent_channels: int = 16
    patch: int = 2
    context_width: int = 1024  # LlmAdapter.Width
    adaln_rank: int = 256
    eps: float = 1e-6

    @property
    def head_dim(self) -> int:
        return self.width // self.heads


PARTS = ("self_attn", "cross_attn", "mlp")


def block_weight_shapes(cfg: AnimaConfig, i: int) -> Dict[str, tuple]:
    D, F, R, d, Cw = cfg.width, cfg.mlp, cfg.adaln_rank, cfg.head_dim, cfg.context_width
    p = f"blocks.{i}"
    out = {}
    for part in PARTS:
        out[f"{p}.adaln_modulation_{part}.1.weight"] = (R, D)
        out[f"{p}.adaln_modulation_{part}.2.weight"] = (3 * D, R)
    for a in ("self_attn", "cross_attn"):
        src = D if a == "self_attn" else Cw
        out[f"{p}.{a}.q_proj.weight"] = (D, D)
        out[f"{p}.{a}.k_proj.weight"] = (D, src)
        out[f"{p}.{a}.v_proj.weight"] = (D, src)
        out[f"{p}.{a}.output_proj.weight"] = (D, D)
        out[f"{p}.{a}.q_norm.weight"] = (d,)
        out[f"{p}.{a}.k_norm.weight"] = (d,)
    out[f"{p}.mlp.layer1.weight"] = (F, D)
    out[f"{p}.mlp.layer2.weight"] = (D, F)
    return out


def weight_shapes(cfg: AnimaConfig) -> Dict[str, tuple]:
    """The checkpoint's names and shapes (AnimaDit.cs:84-115, 360-404)."""
    D, R = cfg.width, cfg.adaln_rank
    pp = cfg.patch * cfg.patch
    out = {
        "x_embedder.proj.1.weight": (D, (cfg.latent_channels + 1) * pp),
        "t_embedding_norm.weight": (D,),
        "t_embedder.1.linear_1.weight": (D, D),
        "t_embedder.1.linear_2.weight": (3 * D, D),
        "final_layer.adaln_modulation.1.weight": (R, D),
        "final_layer.adaln_modulation.2.weight": (2 * D, R),
        "final_layer.linear.weight": (cfg.latent_channels * pp, D),
    }
    for i in range(cfg.blocks):
        out.update(block_weight_shapes(cfg, i))
    return out


def _is_norm(name: str) -> bool:
    return name.endswith("_norm.weight") or name == "t_embedding_norm.weight"


def synthetic_weights(cfg: AnimaConfig, seed: int, names=None, norm_spread: float = 0.0) -> Dict[str, np.ndarray]:
    """Host weights: N(0, 0.02) rounded to bf16 (fp32 values of those bf16
    numbers, which fp16 also holds); norm weights 1 (+ N(0, norm_spread))."""
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


def device_weights(device: Device, cfg: AnimaConfig, seed: int, dtype: HostDataType = HostDataType.BFloat16,
                   names=None, norm_spread: float = 0.0) -> Dict[str, DeviceTensor]:
    """The synthetic weights made on the GPU at `dtype` (norm weights 1, +
    N(0, norm_spread) made on the host as synthetic_weights makes them)."""
    shapes = weight_shapes(cfg)
    out = {}
    for name in (names or shapes):
        shape = shapes[name]
        if _is_norm(name):
            v = np.ones(shape, np.float32)
            if norm_spread:
                v = v + rng.normal(rng.tensor_seed(seed, name), shape, 0.0, norm_spread)
            out[name] = device.Upload(HostTensor.FromFloats(v).ConvertTo(dtype))
        else:
            out[name] = device.Normal(dtype, shape, rng.tensor_seed(seed, name), 0.0, 0.02)
    return out


def rope_tables(rows: int, cols: int, head_dim: int = 128):
    """AnimaDit.RopeTables (:149-188): [rows*cols, head_dim/2] fp32 tables,
    the temporal pairs still, then the row pairs, then the column pairs, at
    1 / theta^(2k / s) with theta = 10000 * 4^(s / (s - 2)), s = head_dim/6*2."""
    spatial = head_dim // 6 * 2
    temporal = head_dim - 2 * spatial
    pairs = head_dim // 2
    theta = np.float32(ROPE_THETA * NTK_EXTRAPOLATION ** (spatial / (spatial - 2)))
    k = np.arange(spatial // 2, dtype=np.float32)
    freq = (np.float32(1.0) / np.power(theta, np.float32(2.0) * k / np.float32(spatial))).astype(np.float32)
    ii, jj = np.meshgrid(np.arange(rows, dtype=np.float32), np.arange(cols, dtype=np.float32), indexing="ij")
    ra = (ii.reshape(-1, 1) * freq).astype(np.float32)
    ca = (jj.reshape(-1, 1) * freq).astype(np.float32)
    n = rows * cols
    cos = np.ones((n, pairs), np.float32)
    sin = np.zeros((n, pairs), np.float32)
    t0, t1 = temporal // 2, temporal // 2 + spatial // 2
    cos[:, t0:t1], sin[:, t0:t1] = np.cos(ra), np.sin(ra)
    cos[:, t1:], sin[:, t1:] = np.cos(ca), np.sin(ca)
    return cos, sin


def _chunk(mod, i: int, D: int):
    s = mod.Shape
    return Ops.Slice(mod, [0, 0, 0, i * D], [s[0], s[1], s[2], D])


def modulation(model: ModelBuilder, W: WeightSet, prefix: str, silu_temb, lora, chunks: int, D: int):
    """AnimaDit.Modulation (:270-291): Linear(Linear(SiLU(temb), W1), W2)
    plus the shared term's first chunks * D entries (fused as the second
    linear's residual), cut into `chunks` fp32 rows of the model width."""
    low = Layers.Linear(model, silu_temb, W(f"{prefix}.1.weight"))
    shared = lora if chunks == 3 else Ops.Slice(lora, [0, 0, 0, 0], [1, 1, 1, chunks * D])
    mod = Layers.Linear(model, low, W(f"{prefix}.2.weight"), residual=shared)
    return [_chunk(mod, i, D) for i in range(chunks)]


def build_block(model: ModelBuilder, W: WeightSet, i: int, cfg: AnimaConfig, x, silu_temb, lora, context, cos, sin,
                compute: HostDataType):
    """AnimaDit.Block (:325-358). x [1, 1, N, D] fp32 residual; context [1,
    1, Nc, Cw] at the compute type; cos/sin [1, N, 1, d/2]. Returns x."""
    D, H, eps = cfg.width, cfg.heads, cfg.eps
    n = x.Shape[2]
    p = f"blocks.{i}"
    mods = {part: modulation(model, W, f"{p}.adaln_modulation_{part}", silu_temb, lora, 3, D) for part in PARTS}

    # Self-attention: q, k, v from one GEMM over the stacked projections.
    sh, sc, g = mods["self_attn"]
    h = Transformer.Modulate(x, sh, sc, eps, compute)
    a = f"{p}.self_attn"
    qkv = Layers.Linear(model, h, W.stacked([f"{a}.q_proj.weight", f"{a}.k_proj.weight", f"{a}.v_proj.weight"]))
    q = Transformer.HeadNormRotate(model, Ops.Slice(qkv, [0, 0, 0, 0], [1, 1, n, D]), W(f"{a}.q_norm.weight", "norm"),
                                   H, eps, cos, sin, compute)
    k = Transformer.HeadNormRotate(model, Ops.Slice(qkv, [0, 0, 0, D], [1, 1, n, D]), W(f"{a}.k_norm.weight", "norm"),
                                   H, eps, cos, sin, compute)
    v = Ops.Slice(qkv, [0, 0, 0, 2 * D], [1, 1, n, D])
    att = Layers.Attend(q, k, v, H)
    x = Layers.Linear(model, att, W(f"{a}.output_proj.weight"), gate=g, residual=x)

    # Cross-attention into the context: k and v from one GEMM.
    sh, sc, g = mods["cross_attn"]
    h = Transformer.Modulate(x, sh, sc, eps, compute)
    a = f"{p}.cross_attn"
    nc = context.Shape[2]
    q = Transformer.HeadNormRotate(model, Layers.Linear(model, h, W(f"{a}.q_proj.weight")),
                                   W(f"{a}.q_norm.weight", "norm"), H, eps, None, None, compute)
    kv = Layers.Linear(model, context, W.stacked([f"{a}.k_proj.weight", f"{a}.v_proj.weight"]))
    k = Transformer.HeadNormRotate(model, Ops.Slice(kv, [0, 0, 0, 0], [1, 1, nc, D]), W(f"{a}.k_norm.weight", "norm"),
                                   H, eps, None, None, compute)
    v = Ops.Slice(kv, [0, 0, 0, D], [1, 1, nc, D])
    att = Layers.Attend(q, k, v, H)
    x = Layers.Linear(model, att, W(f"{a}.output_proj.weight"), gate=g, residual=x)

    # MLP, exact GELU.
    sh, sc, g = mods["mlp"]
    h = Transformer.Modulate(x, sh, sc, eps, compute)
    f = Layers.Linear(model, h, W(f"{p}.mlp.layer1.weight"), activation="gelu")
    return Layers.Linear(model, f, W(f"{p}.mlp.layer2.weight"), gate=g, residual=x)


# Names of the values the step's chain carries (AnimaDit.cs:37-45; the
# latent replaces the reference's host-made patches: it is patchified on the
# device).
LATENT, TIME, CONTEXT, COS, SIN = "latent", "time", "context", "cos", "sin"
X, TEMB, LORA, OUT = "x", "temb", "lora", "out"


def build_step_chain(device: Device, cfg: AnimaConfig, weights: dict, latent_h: int, latent_w: int, n_ctx: int,
                     compute: HostDataType, int8: bool = False, blocks: int = None) -> GraphChain:
    """The denoiser step as a GraphChain (AnimaDit.Build, :360-404): the
    embeddings, one link per block, the final layer. Inputs by name: latent
    [1, 16, H, W], time [1, 1, 1, D] (Sinusoid(sigma, D)), context [1, 1,
    Nc, Cw], cos, sin [1, N, 1, d/2], all fp32. Result: the flow [1, 16, H,
    W] fp32. The links compile into one model."""
    D, C, p = cfg.width, cfg.latent_channels, cfg.patch
    n = (latent_h // p) * (latent_w // p)
    blocks = cfg.blocks if blocks is None else blocks
    F32 = HostDataType.Float32
    store = compute if compute != F32 else HostDataType.Float16
    chain = GraphChain(device, store, None, int8)
    try:
        model = chain.Current
        W = WeightSet(model, weights, compute, device)
        chain.Input(LATENT, [1, C, latent_h, latent_w], F32)
        chain.Input(TIME, [1, 1, 1, D], F32)
        chain.Input(CONTEXT, [1, 1, n_ctx, cfg.context_width], F32)
        chain.Input(COS, [1, n, 1, cfg.head_dim // 2], F32)
        chain.Input(SIN, [1, n, 1, cfg.head_dim // 2], F32)

        # Embeddings, wide: the sixteen real channels' columns of the patch
        # embedding (RealChannelColumns, :251-262), the normed time and the
        # shared adaLN term through the time embedder. The blocks read
        # silu(temb); it is carried under the temb name.
        chain.Set(X, Layers.Linear(model, Ops.Patchify(chain.Get(LATENT), p, PATCH_CHANNEL_FIRST),
                                   W.columns("x_embedder.proj.1.weight", C * p * p)))
        chain.Drop(LATENT)
        time = chain.Get(TIME)
        chain.Set(TEMB, Layers.Silu(Layers.RmsNorm(model, time, W("t_embedding_norm.weight", "wide"), cfg.eps)))
        chain.Set(LORA, Layers.Linear(model, Layers.Silu(Layers.Linear(model, time,
                                                                        W("t_embedder.1.linear_1.weight"))),
                                      W("t_embedder.1.linear_2.weight")))
        chain.Drop(TIME)
        if compute != F32:
            chain.Set(CONTEXT, Layers.Cast(chain.Get(CONTEXT), compute))
        chain.Cut()

        for i in range(blocks):
            chain.Set(X, build_block(model, W, i, cfg, chain.Get(X), chain.Get(TEMB), chain.Get(LORA),
                                     chain.Get(CONTEXT), chain.Get(COS), chain.Get(SIN), compute))
            chain.Cut()

        sh, sc = modulation(model, W, "final_layer.adaln_modulation", chain.Get(TEMB), chain.Get(LORA), 2, D)
        y = Transformer.Modulate(chain.Get(X), sh, sc, cfg.eps, F32)
        out = Layers.Linear(model, y, W("final_layer.linear.weight"))
        chain.Set(OUT, Ops.Unpatchify(out, p, C, latent_h, latent_w, PATCH_CHANNEL_LAST))
        for name in (X, TEMB, LORA, CONTEXT, COS, SIN):
            chain.Drop(name)
        chain.Finish(OUT)
        W.release()
    except BaseException:
        chain.Dispose()
        raise
    return chain


def build_step_model(device: Device, cfg: AnimaConfig, weights: dict, latent_h: int, latent_w: int, n_ctx: int,
                     compute: HostDataType, int8: bool = False, blocks: int = None) -> ModelBuilder:
    """The step chain's compiled model, its inputs bound in the order
    latent, time, context, cos, sin."""
    return build_step_chain(device, cfg, weights, latent_h, latent_w, n_ctx, compute, int8, blocks).Current


def build_block_model(device: Device, cfg: AnimaConfig, weights: dict, n_tokens: int, n_ctx: int,
                      compute: HostDataType, int8: bool = False, block: int = 0):
    """One compiled block. Inputs: x [1, 1, N, D] fp32, temb [1, 1, 1, D]
    (the normed time embedding), lora [1, 1, 1, 3D], context [1, 1, Nc, Cw],
    cos, sin [1, N, 1, d/2], all fp32. Output: x fp32."""
    F32 = HostDataType.Float32
    D = cfg.width
    store = compute if compute != F32 else HostDataType.Float16
    model = ModelBuilder(device, store, int8)
    W = WeightSet(model, weights, compute, device)
    x = model.Placeholder([1, 1, n_tokens, D], F32)
    temb = model.Placeholder([1, 1, 1, D], F32)
    lora = model.Placeholder([1, 1, 1, 3 * D], F32)
    context = model.Placeholder([1, 1, n_ctx, cfg.context_width], F32)
    cos = model.Placeholder([1, n_tokens, 1, cfg.head_dim // 2], F32)
    sin = model.Placeholder([1, n_tokens, 1, cfg.head_dim // 2], F32)
    ctx = context if compute == F32 else Layers.Cast(context, compute)
    y = build_block(model, W, block, cfg, x, Layers.Silu(temb), lora, ctx, cos, sin, compute)
    model.Compile([y])
    W.release()
    return model


class AnimaDit:
    """IDenoiser over the compiled step (Pipeline/IDenoiser.cs:16-17;
    AnimaDit.Predict, :120-132): Predict(latent, timestep, sigma,
    conditioning) -> flow, host tensors in and out; conditioning holds
    'context' [Nc, 1024] rows. The level is embedded as it is."""

    def __init__(self, device: Device, cfg: AnimaConfig, weights: dict, height: int, width: int, context_rows: int,
                 compute: HostDataType = HostDataType.BFloat16, int8: bool = False):
        scale = 8  # the Wan VAE's spatial factor
        self.cfg = cfg
        self.latent_h, self.latent_w = height // scale, width // scale
        if self.latent_h % cfg.patch or self.latent_w % cfg.patch:
            from ._lib import ArgumentError
            raise ArgumentError(f"{width}x{height} does not divide into 16-pixel patches")
        self.context_rows = context_rows
        self.chain = build_step_chain(device, cfg, weights, self.latent_h, self.latent_w, context_rows, compute, int8)
        self.cos, self.sin = rope_tables(self.latent_h // cfg.patch, self.latent_w // cfg.patch, cfg.head_dim)

    @property
    def Tokens(self) -> int:
        return (self.latent_h // self.cfg.patch) * (self.latent_w // self.cfg.patch)

    def Predict(self, latent: HostTensor, timestep: float, sigma: float, conditioning: dict) -> HostTensor:
        cfg = self.cfg
        n, half = self.cos.shape
        ctx = np.asarray(conditioning["context"], np.float32).reshape(1, 1, self.context_rows, cfg.context_width)
        t = Transformer.Sinusoid(float(sigma), cfg.width).reshape(1, 1, 1, cfg.width)
        return self.chain.Run({
            LATENT: latent.Reshape(1, cfg.latent_channels, self.latent_h, self.latent_w),
            TIME: HostTensor.FromFloats(t), CONTEXT: HostTensor.FromFloats(ctx),
            COS: HostTensor.FromFloats(self.cos.reshape(1, n, 1, half)),
            SIN: HostTensor.FromFloats(self.sin.reshape(1, n, 1, half))})

    @property
    def PersistentBytes(self) -> int:
        return self.chain.PersistentBytes

    @property
    def TemporaryBytes(self) -> int:
        return self.chain.TemporaryBytes

    @property
    def GraphCount(self) -> int:
        return self.chain.LinkCount

    def Dispose(self):
        self.chain.Dispose()


# ---- LoRAs (Models/Anima/AnimaLoras.cs) ----------------------------------------------------

LORA_DIT, LORA_TEXT_ENCODER = "dit", "te"


def lora_layout():
    """AnimaLoras.Layout (AnimaLoras.cs:14-31): the transformer as
    lora_unet_... or diffusion_model..., the Qwen3 encoder as lora_te_... or
    text_encoders...; SDXL's two text towers refused on their names."""
    from .lora import LoraLayout, LoraTower
    sdxl = "was trained for SDXL, whose text encoders are two CLIP towers where Anima has Qwen3"
    return LoraLayout("Anima", [LoraTower(LORA_DIT, "transformer", "unet", "diffusion_model"),
                                LoraTower(LORA_TEXT_ENCODER, "Qwen3 text encoder", "te", "text_encoders")],
                      {"te1": sdxl, "te2": sdxl})
