"""Pins for the oracle's model compositions: Anima's whole step and SDXL's
resnet, transformer block, Transformer2d and UNet (oracle/__init__.py).

Each is checked against a float64 numpy restatement written from the
reference's graph builders (Models/Anima/AnimaDit.cs:120-132, 270-404;
Models/Sdxl/UNetModel.cs:230-426; Models/Sdxl/UNetLayers.cs:14-47), vectorised
where the oracle loops, with scipy's erf for the exact GELU; and against
structural invariants that a plausible composition mistake breaks:
- a resnet with zero conv2 is its shortcut: the input itself, or the 1x1
  shortcut's channel selection;
- a Transformer2d with a zero proj_out is the identity;
- the UNet joins [running value, skip] and pops the newest skip first: with
  identity units and up-path shortcuts that keep only the skip half, the
  whole UNet reduces to conv_out(SiLU(GroupNorm(conv_in(sample))));
- the final layer of Anima takes (shift, scale) in that order;
- GEGLU gates the first half by the exact GELU of the second.
"""

import math

import numpy as np
import pytest
from scipy.special import erf

import oracle
from naivediffusion_amd import sdxl

f64 = np.float64


def rnd(g, *shape, s=0.2):
    return (g.standard_normal(shape) * s).astype(np.float32)


# ---- float64 restatement ---------------------------------------------------------------

def lin(x, w, b=None):
    y = np.asarray(x, f64) @ np.asarray(w, f64).T
    return y if b is None else y + np.asarray(b, f64)


def silu(x):
    return x / (1 + np.exp(-x))


def gelu(x):
    return 0.5 * x * (1 + erf(x / math.sqrt(2)))


def layer_norm(x, w=None, b=None, eps=1e-5):
    x = np.asarray(x, f64)
    m = x.mean(-1, keepdims=True)
    y = (x - m) / np.sqrt(((x - m) ** 2).mean(-1, keepdims=True) + eps)
    if w is not None:
        y = y * np.asarray(w, f64)
    if b is not None:
        y = y + np.asarray(b, f64)
    return y


def rms(x, w, eps):
    x = np.asarray(x, f64)
    return x / np.sqrt((x ** 2).mean(-1, keepdims=True) + eps) * np.asarray(w, f64)


def group_norm(x, groups, w, b, eps, act=False):
    x = np.asarray(x, f64)
    B, C = x.shape[:2]
    g = x.reshape(B, groups, -1)
    y = ((g - g.mean(-1, keepdims=True)) / np.sqrt(g.var(-1, keepdims=True) + eps)).reshape(x.shape)
    y = y * np.asarray(w, f64)[None, :, None, None] + np.asarray(b, f64)[None, :, None, None]
    return silu(y) if act else y


def conv(x, w, b, stride=1, pad=1):
    x = np.asarray(x, f64)
    w = np.asarray(w, f64)
    xp = np.pad(x, ((0, 0), (0, 0), (pad, pad), (pad, pad)))
    kh, kw = w.shape[2:]
    win = np.lib.stride_tricks.sliding_window_view(xp, (kh, kw), axis=(2, 3))[:, :, ::stride, ::stride]
    return np.einsum("bchwij,ocij->bohw", win, w) + np.asarray(b, f64)[None, :, None, None]


def attention(q, k, v, heads):
    """softmax(q k^T / sqrt(d)) v per head over [B, T, H*d]."""
    B, T, D = q.shape
    d = D // heads
    q = q.reshape(B, T, heads, d).transpose(0, 2, 1, 3)
    k = k.reshape(B, -1, heads, d).transpose(0, 2, 1, 3)
    v = v.reshape(B, -1, heads, d).transpose(0, 2, 1, 3)
    s = q @ k.transpose(0, 1, 3, 2) / math.sqrt(d)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    return (p @ v).transpose(0, 2, 1, 3).reshape(B, T, D)


def rotate(t, heads, cos, sin):
    n, D = t.shape
    d = D // heads
    t = t.reshape(n, heads, d)
    lo, hi = t[..., :d // 2], t[..., d // 2:]
    c, s = np.asarray(cos, f64)[:, None, :], np.asarray(sin, f64)[:, None, :]
    return np.concatenate([lo * c - hi * s, hi * c + lo * s], -1).reshape(n, D)


# ---- Anima (AnimaDit.cs) -----------------------------------------------------------------

def anima_modulation64(silu_temb, lora, w1, w2, chunks, D):
    m = lin(lin(silu_temb, w1), w2)[0] + np.asarray(lora, f64)[: chunks * D]
    return [m[i * D:(i + 1) * D] for i in range(chunks)]


def anima_attention64(x, src, w, p, heads, cos, sin, eps):
    D = x.shape[-1]
    d = D // heads
    q = rms(lin(x, w[f"{p}.q_proj.weight"]).reshape(-1, heads, d), w[f"{p}.q_norm.weight"], eps).reshape(-1, D)
    k = rms(lin(src, w[f"{p}.k_proj.weight"]).reshape(-1, heads, d), w[f"{p}.k_norm.weight"], eps).reshape(-1, D)
    v = lin(src, w[f"{p}.v_proj.weight"])
    if cos is not None:
        q, k = rotate(q, heads, cos, sin), rotate(k, heads, cos, sin)
    return lin(attention(q[None], k[None], v[None], heads)[0], w[f"{p}.output_proj.weight"])


def anima_step64(latent, sigma, ctx, w, blocks, heads, eps=1e-6):
    C, H, W = latent.shape
    D = w["x_embedder.proj.1.weight"].shape[0]
    tokens = latent.reshape(C, H // 2, 2, W // 2, 2).transpose(1, 3, 0, 2, 4).reshape(-1, C * 4)
    x = lin(tokens, w["x_embedder.proj.1.weight"][:, :C * 4])
    half = D // 2
    ang = sigma * np.exp(-math.log(10000.0) * np.arange(half) / half)
    time = np.concatenate([np.cos(ang), np.sin(ang)])[None]
    st = silu(rms(time, w["t_embedding_norm.weight"], eps))
    lora = lin(silu(lin(time, w["t_embedder.1.linear_1.weight"])), w["t_embedder.1.linear_2.weight"])[0]
    cos, sin = oracle.anima_rope_tables(H // 2, W // 2, D // heads)
    for i in range(blocks):
        p = f"blocks.{i}"
        m = {part: anima_modulation64(st, lora, w[f"{p}.adaln_modulation_{part}.1.weight"],
                                      w[f"{p}.adaln_modulation_{part}.2.weight"], 3, D)
             for part in ("self_attn", "cross_attn", "mlp")}
        sh, sc, g = m["self_attn"]
        h = layer_norm(x, eps=eps) * (1 + sc) + sh
        x = x + g * anima_attention64(h, h, w, f"{p}.self_attn", heads, cos, sin, eps)
        sh, sc, g = m["cross_attn"]
        h = layer_norm(x, eps=eps) * (1 + sc) + sh
        x = x + g * anima_attention64(h, ctx, w, f"{p}.cross_attn", heads, None, None, eps)
        sh, sc, g = m["mlp"]
        h = layer_norm(x, eps=eps) * (1 + sc) + sh
        x = x + g * lin(gelu(lin(h, w[f"{p}.mlp.layer1.weight"])), w[f"{p}.mlp.layer2.weight"])
    sh, sc = anima_modulation64(st, lora, w["final_layer.adaln_modulation.1.weight"],
                                w["final_layer.adaln_modulation.2.weight"], 2, D)
    out = lin(layer_norm(x, eps=eps) * (1 + sc) + sh, w["final_layer.linear.weight"])
    return out.reshape(H // 2, W // 2, 2, 2, C).transpose(4, 0, 2, 1, 3).reshape(C, H, W)


def tiny_anima(seed, D=128, heads=2, F=192, R=24, Cw=48, blocks=2):
    from naivediffusion_amd import anima
    cfg = anima.AnimaConfig(width=D, heads=heads, mlp=F, blocks=blocks, context_width=Cw, adaln_rank=R)
    g = np.random.default_rng(seed)
    w = {}
    for name, shape in anima.weight_shapes(cfg).items():
        w[name] = (1 + rnd(g, *shape, s=0.1)) if name.endswith("norm.weight") else rnd(g, *shape, s=0.15)
    return cfg, w, g


def test_anima_step_against_float64():
    cfg, w, g = tiny_anima(1)
    latent = rnd(g, 16, 4, 6, s=1.0)
    ctx = rnd(g, 5, cfg.context_width, s=1.0)
    got = oracle.anima_step(latent, 0.6, ctx, w, cfg.blocks, cfg.heads)
    exp = anima_step64(latent, 0.6, ctx, w, cfg.blocks, cfg.heads)
    assert got.shape == exp.shape == latent.shape
    assert np.max(np.abs(got - exp)) <= 2e-5 * np.max(np.abs(exp))


def test_anima_final_layer_takes_shift_then_scale():
    """No blocks, no shared term, and a final modulation whose scale chunk
    is zero: the output is W_final (LN(x) + shift), not W_final (LN(x) (1 +
    shift))."""
    cfg, w, g = tiny_anima(2, blocks=0)
    D = cfg.width
    w["t_embedder.1.linear_2.weight"][:] = 0
    w["final_layer.adaln_modulation.2.weight"][D:] = 0
    latent = rnd(g, 16, 4, 4, s=1.0)
    got = oracle.anima_step(latent, 0.3, rnd(g, 3, cfg.context_width), w, 0, cfg.heads)
    tokens = latent.reshape(16, 2, 2, 2, 2).transpose(1, 3, 0, 2, 4).reshape(-1, 64)
    x = lin(tokens, w["x_embedder.proj.1.weight"][:, :64])
    half = D // 2
    ang = 0.3 * np.exp(-math.log(10000.0) * np.arange(half) / half)
    st = silu(rms(np.concatenate([np.cos(ang), np.sin(ang)])[None], w["t_embedding_norm.weight"], 1e-6))
    shift = lin(lin(st, w["final_layer.adaln_modulation.1.weight"]), w["final_layer.adaln_modulation.2.weight"])[0, :D]
    out = lin(layer_norm(x, eps=1e-6) + shift, w["final_layer.linear.weight"])
    exp = out.reshape(2, 2, 2, 2, 16).transpose(4, 0, 2, 1, 3).reshape(16, 4, 4)
    assert np.max(np.abs(got - exp)) <= 2e-5 * np.max(np.abs(exp))
    swapped = lin(layer_norm(x, eps=1e-6) * (1 + shift), w["final_layer.linear.weight"])
    assert np.max(np.abs(got.ravel() - swapped.reshape(2, 2, 2, 2, 16).transpose(4, 0, 2, 1, 3).ravel())) > 1e-2


# ---- SDXL (UNetModel.cs, UNetLayers.cs) ---------------------------------------------------

def resnet64(x, temb, w, p, groups, eps):
    h = conv(group_norm(x, groups, w[f"{p}.norm1.weight"], w[f"{p}.norm1.bias"], eps, True),
             w[f"{p}.conv1.weight"], w[f"{p}.conv1.bias"])
    h = h + lin(silu(np.asarray(temb, f64)), w[f"{p}.time_emb_proj.weight"], w[f"{p}.time_emb_proj.bias"])[:, :, None,
                                                                                                          None]
    h = conv(group_norm(h, groups, w[f"{p}.norm2.weight"], w[f"{p}.norm2.bias"], eps, True),
             w[f"{p}.conv2.weight"], w[f"{p}.conv2.bias"])
    if f"{p}.conv_shortcut.weight" in w:
        x = conv(x, w[f"{p}.conv_shortcut.weight"], w[f"{p}.conv_shortcut.bias"], 1, 0)
    return np.asarray(x, f64) + h


def diffusers_attention64(x, src, w, p, heads):
    a = attention(lin(x, w[f"{p}.to_q.weight"]), lin(src, w[f"{p}.to_k.weight"]), lin(src, w[f"{p}.to_v.weight"]),
                  heads)
    return lin(a, w[f"{p}.to_out.0.weight"], w[f"{p}.to_out.0.bias"])


def transformer_block64(x, ctx, w, p, heads, eps):
    x = np.asarray(x, f64)
    h = layer_norm(x, w[f"{p}.norm1.weight"], w[f"{p}.norm1.bias"], eps)
    x = x + diffusers_attention64(h, h, w, f"{p}.attn1", heads)
    h = layer_norm(x, w[f"{p}.norm2.weight"], w[f"{p}.norm2.bias"], eps)
    x = x + diffusers_attention64(h, ctx, w, f"{p}.attn2", heads)
    h = layer_norm(x, w[f"{p}.norm3.weight"], w[f"{p}.norm3.bias"], eps)
    proj = lin(h, w[f"{p}.ff.net.0.proj.weight"], w[f"{p}.ff.net.0.proj.bias"])
    inner = proj.shape[-1] // 2
    return x + lin(proj[..., :inner] * gelu(proj[..., inner:]), w[f"{p}.ff.net.2.weight"], w[f"{p}.ff.net.2.bias"])


def transformer2d64(x, ctx, w, p, heads, layers, groups, eps, ln_eps):
    B, C, H, W = x.shape
    t = group_norm(x, groups, w[f"{p}.norm.weight"], w[f"{p}.norm.bias"], eps).reshape(B, C, H * W).transpose(0, 2, 1)
    t = lin(t, w[f"{p}.proj_in.weight"], w[f"{p}.proj_in.bias"])
    for j in range(layers):
        t = transformer_block64(t, ctx, w, f"{p}.transformer_blocks.{j}", heads, ln_eps)
    t = lin(t, w[f"{p}.proj_out.weight"], w[f"{p}.proj_out.bias"])
    return t.transpose(0, 2, 1).reshape(B, C, H, W) + np.asarray(x, f64)


def unet64(sample, time, add, ctx, w, cfg):
    """UNetModel.Build (:333-426): a stack of named skips, newest consumed
    first on the way up, each joined after the running value."""
    def emb(v, p):
        return lin(silu(lin(v, w[f"{p}.linear_1.weight"], w[f"{p}.linear_1.bias"])), w[f"{p}.linear_2.weight"],
                   w[f"{p}.linear_2.bias"])

    temb = emb(time, "time_embedding") + emb(add, "add_embedding")

    def unit(x, prefix, idx, level):
        x = resnet64(x, temb, w, f"{prefix}.resnets.{idx}", cfg.groups, cfg.eps)
        if cfg.transformer_layers[level]:
            x = transformer2d64(x, ctx, w, f"{prefix}.attentions.{idx}", cfg.heads[level],
                                cfg.transformer_layers[level], cfg.groups, cfg.transformer_eps, cfg.layer_norm_eps)
        return x

    stack = [conv(sample, w["conv_in.weight"], w["conv_in.bias"])]
    n = len(cfg.block_out)
    for level in range(n):
        for i in range(cfg.layers_per_block):
            stack.append(unit(stack[-1], f"down_blocks.{level}", i, level))
        if level < n - 1:
            p = f"down_blocks.{level}.downsamplers.0.conv"
            stack.append(conv(stack[-1], w[f"{p}.weight"], w[f"{p}.bias"], 2, 1))
    x = resnet64(stack[-1], temb, w, "mid_block.resnets.0", cfg.groups, cfg.eps)
    x = transformer2d64(x, ctx, w, "mid_block.attentions.0", cfg.heads[-1], cfg.transformer_layers[-1], cfg.groups,
                        cfg.transformer_eps, cfg.layer_norm_eps)
    x = resnet64(x, temb, w, "mid_block.resnets.1", cfg.groups, cfg.eps)
    for i in range(n):
        level = n - 1 - i
        for j in range(cfg.layers_per_block + 1):
            x = unit(np.concatenate([x, stack.pop()], 1), f"up_blocks.{i}", j, level)
        if i < n - 1:
            th, tw = stack[-1].shape[2:]
            up = x.repeat(2, 2).repeat(2, 3)[:, :, :th, :tw]
            p = f"up_blocks.{i}.upsamplers.0.conv"
            x = conv(up, w[f"{p}.weight"], w[f"{p}.bias"])
    x = group_norm(x, cfg.groups, w["conv_norm_out.weight"], w["conv_norm_out.bias"], cfg.eps, True)
    return conv(x, w["conv_out.weight"], w["conv_out.bias"])


TINY = sdxl.SdxlConfig(block_out=(8, 16, 16), transformer_layers=(0, 1, 1), heads=(1, 2, 2), context_width=12,
                       time_embed=16, add_time_dim=4, pooled_width=8, groups=4)


def tiny_sdxl(seed, cfg=TINY):
    g = np.random.default_rng(seed)
    w = {}
    for name, shape in sdxl.weight_shapes(cfg).items():
        if ".norm" in name or name.startswith("conv_norm_out"):
            w[name] = (1.0 if name.endswith("weight") else 0.0) + rnd(g, *shape, s=0.1)
        elif len(shape) == 1:
            w[name] = rnd(g, *shape, s=0.1)
        else:
            w[name] = rnd(g, *shape, s=1.0 / math.sqrt(np.prod(shape[1:])))
    return w, g


def close(got, exp, tol=2e-5):
    return np.max(np.abs(np.asarray(got, f64) - exp)) <= tol * np.max(np.abs(exp))


@pytest.mark.parametrize("prefix", ["down_blocks.1.resnets.0", "down_blocks.1.resnets.1", "up_blocks.1.resnets.2"])
def test_sdxl_resnet_against_float64(prefix):
    w, g = tiny_sdxl(3)
    cin = w[f"{prefix}.norm1.weight"].shape[0]
    x, temb = rnd(g, 2, cin, 6, 5, s=1.0), rnd(g, 2, TINY.time_embed, s=1.0)
    got = oracle.sdxl_resnet(x, oracle.silu(temb), w, prefix, TINY.groups, TINY.eps)
    assert close(got, resnet64(x, temb, w, prefix, TINY.groups, TINY.eps))


def test_sdxl_resnet_with_zero_conv2_is_its_shortcut():
    w, g = tiny_sdxl(4)
    temb = rnd(g, 2, TINY.time_embed, s=1.0)
    p = "down_blocks.1.resnets.1"  # 16 -> 16: no shortcut
    w[f"{p}.conv2.weight"][:] = 0
    w[f"{p}.conv2.bias"][:] = 0
    x = rnd(g, 2, 16, 5, 4, s=1.0)
    assert np.array_equal(oracle.sdxl_resnet(x, oracle.silu(temb), w, p, TINY.groups, TINY.eps), x)
    p = "up_blocks.2.resnets.0"  # 16 + 8 -> 8: a 1x1 shortcut, here keeping channels 3..10
    cin = w[f"{p}.norm1.weight"].shape[0]
    w[f"{p}.conv2.weight"][:] = 0
    w[f"{p}.conv2.bias"][:] = 0
    w[f"{p}.conv_shortcut.weight"][:] = 0
    w[f"{p}.conv_shortcut.bias"][:] = 0
    for o in range(8):
        w[f"{p}.conv_shortcut.weight"][o, o + 3, 0, 0] = 1
    x = rnd(g, 2, cin, 5, 4, s=1.0)
    assert np.array_equal(oracle.sdxl_resnet(x, oracle.silu(temb), w, p, TINY.groups, TINY.eps), x[:, 3:11])


def test_sdxl_transformer_block_against_float64():
    w, g = tiny_sdxl(5)
    p = "down_blocks.1.attentions.0.transformer_blocks.0"
    x, ctx = rnd(g, 2, 7, 16, s=1.0), rnd(g, 2, 3, TINY.context_width, s=1.0)
    got = oracle.sdxl_transformer_block(x, ctx, w, p, 2, TINY.layer_norm_eps)
    assert close(got, transformer_block64(x, ctx, w, p, 2, TINY.layer_norm_eps))


def test_sdxl_geglu_gates_the_first_half_by_the_gelu_of_the_second():
    """Attention outputs closed (zero to_out), norm3 the plain LayerNorm: the
    block is x + W2 (a * GELU(b)) with [a, b] = W1 LN(x) + b1, the GELU the
    exact one (scipy's erf; the tanh form differs by up to ~1e-3)."""
    w, g = tiny_sdxl(6)
    p = "down_blocks.1.attentions.0.transformer_blocks.0"
    for a in ("attn1", "attn2"):
        w[f"{p}.{a}.to_out.0.weight"][:] = 0
        w[f"{p}.{a}.to_out.0.bias"][:] = 0
    w[f"{p}.norm3.weight"][:] = 1
    w[f"{p}.norm3.bias"][:] = 0
    x = rnd(g, 1, 9, 16, s=2.0)
    got = oracle.sdxl_transformer_block(x, rnd(g, 1, 3, TINY.context_width), w, p, 2, TINY.layer_norm_eps)
    proj = lin(layer_norm(x, eps=TINY.layer_norm_eps), w[f"{p}.ff.net.0.proj.weight"], w[f"{p}.ff.net.0.proj.bias"])
    a, b = proj[..., :64], proj[..., 64:]
    exp = x + lin(a * gelu(b), w[f"{p}.ff.net.2.weight"], w[f"{p}.ff.net.2.bias"])
    assert close(got, exp)
    wrong = x + lin(b * gelu(a), w[f"{p}.ff.net.2.weight"], w[f"{p}.ff.net.2.bias"])
    assert not close(got, wrong, 1e-2)


@pytest.mark.parametrize("amplitude", [1.0, 3e-3], ids=["unit", "small"])
def test_sdxl_transformer2d_against_float64_and_identity(amplitude):
    """At a small amplitude the GroupNorm's variance is comparable to its
    epsilon, so the Transformer2d's 1e-6 and the resnets' 1e-5 differ."""
    w, g = tiny_sdxl(7)
    p = "down_blocks.1.attentions.0"
    x, ctx = rnd(g, 2, 16, 4, 3, s=amplitude), rnd(g, 2, 5, TINY.context_width, s=1.0)
    got = oracle.sdxl_transformer2d(x, ctx, w, p, 2, 1, TINY.groups, TINY.transformer_eps, TINY.layer_norm_eps)
    exp = transformer2d64(x, ctx, w, p, 2, 1, TINY.groups, TINY.transformer_eps, TINY.layer_norm_eps)
    assert close(got - x, exp - x)
    w[f"{p}.proj_out.weight"][:] = 0
    w[f"{p}.proj_out.bias"][:] = 0
    same = oracle.sdxl_transformer2d(x, ctx, w, p, 2, 1, TINY.groups, TINY.transformer_eps, TINY.layer_norm_eps)
    assert np.array_equal(same, x)


@pytest.mark.parametrize("H,W", [(8, 8), (9, 7)])
def test_sdxl_unet_against_float64(H, W):
    w, g = tiny_sdxl(8)
    B = 2
    sample = rnd(g, B, 4, H, W, s=1.0)
    time = rnd(g, B, TINY.block_out[0], s=1.0)
    add = rnd(g, B, TINY.add_width, s=1.0)
    ctx = rnd(g, B, 3, TINY.context_width, s=1.0)
    got = oracle.sdxl_unet(sample, time, add, ctx, w, TINY)
    exp = unet64(sample, time, add, ctx, w, TINY)
    assert got.shape == exp.shape == sample.shape
    assert close(got, exp, 5e-5)


def test_sdxl_unet_joins_value_then_skip_newest_first():
    """Every unit an identity (zero conv2, zero proj_out) and every up-path
    shortcut keeping only the skip half of [value, skip]: each up unit then
    returns the skip it consumed, the last one consumed is conv_in's output,
    and the UNet is conv_out(SiLU(GroupNorm(conv_in(sample)))). A join in the
    other order, or skips taken oldest first, gives another function."""
    cfg = sdxl.SdxlConfig(block_out=(8, 8, 8), transformer_layers=(0, 1, 1), heads=(1, 2, 2), context_width=12,
                          time_embed=16, add_time_dim=4, pooled_width=8, groups=4)
    w, g = tiny_sdxl(9, cfg)
    for name in w:
        if name.endswith((".conv2.weight", ".conv2.bias", ".proj_out.weight", ".proj_out.bias",
                          ".conv_shortcut.weight", ".conv_shortcut.bias")):
            w[name][:] = 0
    for name in w:
        if name.endswith(".conv_shortcut.weight"):
            for o in range(8):
                w[name][o, 8 + o, 0, 0] = 1
    sample = rnd(g, 1, 4, 9, 7, s=1.0)
    got = oracle.sdxl_unet(sample, rnd(g, 1, 8), rnd(g, 1, cfg.add_width), rnd(g, 1, 3, 12), w, cfg)
    x = conv(sample, w["conv_in.weight"], w["conv_in.bias"])
    exp = conv(group_norm(x, 4, w["conv_norm_out.weight"], w["conv_norm_out.bias"], cfg.eps, True), w["conv_out.weight"],
               w["conv_out.bias"])
    assert close(got, exp)


# ---- Qwen-Image 2.1 (QwenImageDit.cs) ----------------------------------------------------

def attend_allowed(q, k, v, heads, allowed):
    """Softmax attention per head over [T, H*d] with a [T, S] table of the
    keys each query may read (a masked score gets no weight)."""
    T, D = q.shape
    d = D // heads
    q = q.reshape(T, heads, d).transpose(1, 0, 2)
    k = k.reshape(-1, heads, d).transpose(1, 0, 2)
    v = v.reshape(-1, heads, d).transpose(1, 0, 2)
    s = q @ k.transpose(0, 2, 1) / math.sqrt(d)
    s = np.where(allowed[None], s, -np.inf)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    return (p @ v).transpose(1, 0, 2).reshape(T, D)


def qwen_block64(x, mod, w, p, heads, n_img, cos, sin, key_len, text_mask, eps=1e-6):
    """The block with Qwen's own rotary form: adjacent feature pairs (2i,
    2i + 1) of the unpermuted projections turn by the table's angle i, the
    form PairsToHalves turns into halves."""
    x = np.asarray(x, f64)
    N, D = x.shape
    d = D // heads

    def rows(c):
        r = np.empty((N, D))
        r[:n_img], r[n_img:] = mod[0, c * D:(c + 1) * D], mod[1, c * D:(c + 1) * D]
        return r

    def rot_pairs(t):
        t = t.reshape(N, heads, d)
        ev, od = t[..., 0::2], t[..., 1::2]
        c, s = np.asarray(cos, f64)[:, None, :], np.asarray(sin, f64)[:, None, :]
        out = np.empty_like(t)
        out[..., 0::2], out[..., 1::2] = ev * c - od * s, od * c + ev * s
        return out.reshape(N, D)

    h = layer_norm(x, eps=eps) * (1 + rows(0))
    q = rot_pairs(rms(lin(h, w[f"{p}.attn.to_q.weight"]).reshape(N, heads, d), w[f"{p}.attn.norm_q.weight"], eps))
    k = rot_pairs(rms(lin(h, w[f"{p}.attn.to_k.weight"]).reshape(N, heads, d), w[f"{p}.attn.norm_k.weight"], eps))
    v = lin(h, w[f"{p}.attn.to_v.weight"])
    image = attend_allowed(q[:n_img], k, v, heads, np.broadcast_to(np.arange(N) < key_len, (n_img, N)))
    text = attend_allowed(q[n_img:], k[n_img:], v[n_img:], heads, np.asarray(text_mask, bool))
    x = x + rows(1) * lin(np.concatenate([image, text]), w[f"{p}.attn.to_out.0.weight"])
    gu = lin(layer_norm(x, eps=eps) * (1 + rows(2)), w[f"{p}.img_mlp.gate_up.weight"])
    F = gu.shape[1] // 2
    return x + rows(3) * lin(silu(gu[:, :F]) * gu[:, F:], w[f"{p}.img_mlp.out.weight"])


def tiny_qwen(seed, blocks=1):
    from naivediffusion_amd import qwen
    cfg = qwen.QwenImageConfig(width=256, heads=2, mlp=96, blocks=blocks, latent_channels=8, context_width=24,
                               time_dim=32)
    g = np.random.default_rng(seed)
    w = {}
    for name, shape in qwen.weight_shapes(cfg).items():
        if name.endswith(("norm_q.weight", "norm_k.weight")):
            w[name] = 1 + rnd(g, *shape, s=0.2)
        elif name == "txt_in.text_norm.weight":
            w[name] = rnd(g, *shape, s=0.2)
        else:
            w[name] = rnd(g, *shape, s=0.08)
    return cfg, w, g


def test_qwen_pairs_to_halves_in_the_product_follow_the_reference_rows():
    from naivediffusion_amd import qwen
    g = np.random.default_rng(0)
    m, v = rnd(g, 3 * 128, 5), rnd(g, 128)
    assert np.array_equal(qwen.pairs_to_halves(m, 128), oracle.qwen_pairs_to_halves(m, 128))
    assert np.array_equal(qwen.pairs_to_halves(v, 128), oracle.qwen_pairs_to_halves(v, 128))
    gu = rnd(g, 2 * 6, 4)
    il = qwen.interleave_gate_up(gu)
    assert np.array_equal(il[0::2], gu[:6]) and np.array_equal(il[1::2], gu[6:])


def test_qwen_block_against_float64_pair_rotation():
    """The oracle's block (PairsToHalves, then rotate-half) against a float64
    block that rotates the reference's adjacent pairs on the unpermuted
    weights: a wrong permutation, a rotation in the wrong form, a missing
    tanh gate or a swapped gate / up would all part them."""
    cfg, w, g = tiny_qwen(1)
    n_img, n_txt, real = 6, 5, 3
    N = n_img + n_txt
    x = rnd(g, N, cfg.width, s=1.0)
    mod = rnd(g, 2, 4 * cfg.width, s=0.3)
    mod[:, cfg.width:2 * cfg.width] = np.tanh(mod[:, cfg.width:2 * cfg.width])
    mod[:, 3 * cfg.width:] = np.tanh(mod[:, 3 * cfg.width:])
    cos, sin = oracle.qwen_rope_tables(2, 3, real, n_txt)
    mask = oracle.causal_table(real, n_txt).reshape(n_txt, n_txt)
    key_len = n_img + real
    got = oracle.qwen_block(x, mod, w, 0, cfg.heads, n_img, cos, sin, key_len, mask)
    exp = qwen_block64(x, mod, w, "transformer_blocks.0", cfg.heads, n_img, cos, sin, key_len, mask)
    assert close(got - x, exp - x)
    # The image rows are blind to the padding past the key length.
    x2 = x.copy()
    x2[n_img + real:] += rnd(g, n_txt - real, cfg.width, s=1.0)
    got2 = oracle.qwen_block(x2, mod, w, 0, cfg.heads, n_img, cos, sin, key_len, mask)
    assert np.max(np.abs(got2[:n_img + real] - got[:n_img + real])) < 1e-5


def test_qwen_step_against_float64():
    from naivediffusion_amd import qwen
    cfg, w, g = tiny_qwen(2, blocks=2)
    C, H, W, n_txt, real = cfg.latent_channels, 2, 3, 5, 4
    latent = rnd(g, C, H, W, s=1.0)
    ctx = np.zeros((n_txt, cfg.context_width), np.float32)
    ctx[:real] = rnd(g, real, cfg.context_width, s=1.0)
    cos, sin = oracle.qwen_rope_tables(H, W, real, n_txt)
    mask = oracle.causal_table(real, n_txt).reshape(n_txt, n_txt)
    key_len = H * W + real
    got = oracle.qwen_step(latent, 0.4, ctx, mask, key_len, w, cfg.blocks, cfg.heads, cos, sin, cfg.time_dim)
    # float64: the embeddings, the time path and the final layer by hand.
    D = cfg.width
    image = lin(latent.reshape(C, -1).T, w["img_in.weight"])
    t = rms(ctx, 1.0 + np.asarray(w["txt_in.text_norm.weight"], f64), 1e-6)
    u = lin(t, w["txt_in.in_layer.weight"])
    u = 0.5 * u * (1 + np.tanh(math.sqrt(2 / math.pi) * (u + 0.044715 * u ** 3)))
    x = np.concatenate([image, lin(u, w["txt_in.out_layer.weight"])])

    def sinus(tv, width):
        half = width // 2
        ang = tv * np.exp(-math.log(10000.0) * np.arange(half) / half)
        return np.concatenate([np.cos(ang), np.sin(ang)])

    time = np.stack([sinus(400.0, cfg.time_dim), sinus(0.0, cfg.time_dim)])
    temb = lin(silu(lin(time, w["time_text_embed.timestep_embedder.linear_1.weight"])),
               w["time_text_embed.timestep_embedder.linear_2.weight"])
    mod = lin(silu(temb), w["modulation.1.weight"])
    mod[:, D:2 * D], mod[:, 3 * D:] = np.tanh(mod[:, D:2 * D]), np.tanh(mod[:, 3 * D:])
    for i in range(cfg.blocks):
        x = qwen_block64(x, mod, w, f"transformer_blocks.{i}", cfg.heads, H * W, cos, sin, key_len, mask)
    scale = lin(silu(temb[:1]), w["norm_out.linear.weight"])[0]
    out = lin(layer_norm(x[:H * W], eps=1e-6) * (1 + scale), w["proj_out.weight"])
    exp = out.T.reshape(C, H, W)
    assert close(got, exp, 5e-5)
    # and the product's host inputs are the oracle's
    c2, s2 = qwen.rope_tables(H, W, real, n_txt)
    assert np.max(np.abs(c2 - cos)) < 2e-6 and np.max(np.abs(s2 - sin)) < 2e-6
    assert np.array_equal(qwen.causal_table(real, n_txt), mask)


# ---- AutoencoderKL's decoder (Vae/AutoencoderKl.cs) ------------------------------------------

def vae_resnet64(x, w, p, groups, eps):
    h = conv(group_norm(x, groups, w[f"{p}.norm1.weight"], w[f"{p}.norm1.bias"], eps, True),
             w[f"{p}.conv1.weight"], w[f"{p}.conv1.bias"])
    h = conv(group_norm(h, groups, w[f"{p}.norm2.weight"], w[f"{p}.norm2.bias"], eps, True),
             w[f"{p}.conv2.weight"], w[f"{p}.conv2.bias"])
    if f"{p}.conv_shortcut.weight" in w:
        x = conv(x, w[f"{p}.conv_shortcut.weight"], w[f"{p}.conv_shortcut.bias"], 1, 0)
    return np.asarray(x, f64) + h


def vae_attention64(x, w, p, groups, eps):
    x = np.asarray(x, f64)
    B, C, H, W = x.shape
    t = group_norm(x, groups, w[f"{p}.group_norm.weight"], w[f"{p}.group_norm.bias"], eps).reshape(B, C, -1)
    t = t.transpose(0, 2, 1)
    q, k, v = (lin(t, w[f"{p}.{n}.weight"], w[f"{p}.{n}.bias"]) for n in ("to_q", "to_k", "to_v"))
    s = q @ k.transpose(0, 2, 1) / math.sqrt(C)
    s = np.exp(s - s.max(-1, keepdims=True))
    o = lin((s / s.sum(-1, keepdims=True)) @ v, w[f"{p}.to_out.0.weight"], w[f"{p}.to_out.0.bias"])
    return o.transpose(0, 2, 1).reshape(B, C, H, W) + x


def vae_decoder64(z, w, block_out, layers, groups, eps):
    h = conv(conv(z, w["post_quant_conv.weight"], w["post_quant_conv.bias"], 1, 0),
             w["decoder.conv_in.weight"], w["decoder.conv_in.bias"])
    h = vae_resnet64(h, w, "decoder.mid_block.resnets.0", groups, eps)
    h = vae_attention64(h, w, "decoder.mid_block.attentions.0", groups, eps)
    h = vae_resnet64(h, w, "decoder.mid_block.resnets.1", groups, eps)
    for i in range(len(block_out)):
        for j in range(layers + 1):
            h = vae_resnet64(h, w, f"decoder.up_blocks.{i}.resnets.{j}", groups, eps)
        if f"decoder.up_blocks.{i}.upsamplers.0.conv.weight" in w:
            h = conv(h.repeat(2, 2).repeat(2, 3), w[f"decoder.up_blocks.{i}.upsamplers.0.conv.weight"],
                     w[f"decoder.up_blocks.{i}.upsamplers.0.conv.bias"])
    h = group_norm(h, groups, w["decoder.conv_norm_out.weight"], w["decoder.conv_norm_out.bias"], eps, True)
    return conv(h, w["decoder.conv_out.weight"], w["decoder.conv_out.bias"])


def tiny_vae(seed):
    from naivediffusion_amd import vae
    cfg = vae.VaeConfig(block_out=(8, 16, 16), groups=4)
    g = np.random.default_rng(seed)
    w = {}
    for name, shape in vae.decoder_weight_shapes(cfg).items():
        if ".norm" in name or "group_norm" in name or "conv_norm_out" in name:
            w[name] = (1.0 if name.endswith("weight") else 0.0) + rnd(g, *shape, s=0.1)
        elif len(shape) == 1:
            w[name] = rnd(g, *shape, s=0.1)
        else:
            w[name] = rnd(g, *shape, s=1.0 / math.sqrt(np.prod(shape[1:])))
    return cfg, w, g


def test_vae_decoder_shapes_follow_the_diffusers_layout():
    """SDXL's VAE (block_out 128/256/512/512, 2 resnets a level, 3 in the
    decoder): 14 resnets (2 mid + 4 x 3), one attention, three upsamplers,
    the up blocks widest first, upsamplers on all but the last."""
    from naivediffusion_amd import vae
    shapes = vae.decoder_weight_shapes(vae.SDXL)
    assert len([k for k in shapes if k.endswith(".conv1.weight")]) == 14
    assert len([k for k in shapes if k.endswith("upsamplers.0.conv.weight")]) == 3
    assert shapes["decoder.up_blocks.0.resnets.0.conv1.weight"] == (512, 512, 3, 3)
    assert shapes["decoder.up_blocks.2.resnets.0.conv_shortcut.weight"] == (256, 512, 1, 1)
    assert shapes["decoder.up_blocks.3.resnets.0.conv_shortcut.weight"] == (128, 256, 1, 1)
    assert "decoder.up_blocks.3.upsamplers.0.conv.weight" not in shapes
    assert shapes["decoder.conv_out.weight"] == (3, 128, 3, 3)


@pytest.mark.parametrize("H,W", [(4, 4), (5, 3)])
def test_vae_decoder_against_float64(H, W):
    cfg, w, g = tiny_vae(11)
    z = rnd(g, 1, 4, H, W, s=1.0)
    got = oracle.vae_decoder(z, w, cfg.block_out, cfg.layers_per_block, cfg.groups, cfg.eps)
    exp = vae_decoder64(z, w, cfg.block_out, cfg.layers_per_block, cfg.groups, cfg.eps)
    assert got.shape == exp.shape == (1, 3, H * 4, W * 4)
    assert close(got, exp, 5e-5)


def test_vae_attention_pins():
    """The attention block against float64; with a zero output projection
    it is the identity; its scale is 1/sqrt(C) (1/sqrt of anything else, or
    no softmax, gives another function)."""
    cfg, w, g = tiny_vae(12)
    p = "decoder.mid_block.attentions.0"
    x = rnd(g, 1, 16, 3, 5, s=2.0)
    got = oracle.vae_attention(x, w, p, cfg.groups, cfg.eps)
    exp = vae_attention64(x, w, p, cfg.groups, cfg.eps)
    assert close(got - x, exp - x)
    w2 = dict(w)
    w2[f"{p}.to_q.weight"] = w[f"{p}.to_q.weight"] * 4.0   # the same as a 4x larger scale
    assert not close(oracle.vae_attention(x, w2, p, cfg.groups, cfg.eps) - x, exp - x, 1e-2)
    w2 = dict(w, **{f"{p}.to_out.0.weight": np.zeros_like(w[f"{p}.to_out.0.weight"]),
                    f"{p}.to_out.0.bias": np.zeros_like(w[f"{p}.to_out.0.bias"])})
    assert np.array_equal(oracle.vae_attention(x, w2, p, cfg.groups, cfg.eps), x)


def test_vae_resnet_with_zero_conv2_is_its_shortcut():
    cfg, w, g = tiny_vae(13)
    p = "decoder.up_blocks.1.resnets.1"   # 16 -> 16
    w[f"{p}.conv2.weight"][:] = 0
    w[f"{p}.conv2.bias"][:] = 0
    x = rnd(g, 1, 16, 4, 6, s=1.0)
    assert np.array_equal(oracle.vae_resnet(x, w, p, cfg.groups, cfg.eps), x)
    p = "decoder.up_blocks.2.resnets.0"   # 16 -> 8 through a 1x1 shortcut keeping channels 5..12
    for n in ("conv2.weight", "conv2.bias", "conv_shortcut.weight", "conv_shortcut.bias"):
        w[f"{p}.{n}"][:] = 0
    for o in range(8):
        w[f"{p}.conv_shortcut.weight"][o, o + 5, 0, 0] = 1
    x = rnd(g, 1, 16, 4, 6, s=1.0)
    assert np.array_equal(oracle.vae_resnet(x, w, p, cfg.groups, cfg.eps), x[:, 5:13])


# ---- Wan 2.2's single-frame decoder (Vae/Wan22Vae.cs, Vae/WanVae.cs) ------------------------

def channel_rms64(x, g):
    x = np.asarray(x, f64)
    c = x.shape[1]
    return x / np.sqrt((x * x).mean(1, keepdims=True) + 1e-24 / c) * np.asarray(g, f64)[None, :, None, None]


def wan_residual64(x, w, p):
    h = conv(silu(channel_rms64(x, w[f"{p}.residual.0.gamma"])), w[f"{p}.residual.2.weight"], w[f"{p}.residual.2.bias"])
    h = conv(silu(channel_rms64(h, w[f"{p}.residual.3.gamma"])), w[f"{p}.residual.6.weight"], w[f"{p}.residual.6.bias"])
    if f"{p}.shortcut.weight" in w:
        x = conv(x, w[f"{p}.shortcut.weight"], w[f"{p}.shortcut.bias"], 1, 0)
    return np.asarray(x, f64) + h


def wan_attention64(x, w, p):
    x = np.asarray(x, f64)
    _, c, H, W = x.shape
    qkv = conv(channel_rms64(x, w[f"{p}.norm.gamma"]), w[f"{p}.to_qkv.weight"], w[f"{p}.to_qkv.bias"], 1, 0)
    q, k, v = (qkv[0, i * c:(i + 1) * c].reshape(c, -1).T for i in range(3))
    s = q @ k.T / math.sqrt(c)
    s = np.exp(s - s.max(-1, keepdims=True))
    a = (s / s.sum(-1, keepdims=True)) @ v
    o = conv(a.T.reshape(1, c, H, W), w[f"{p}.proj.weight"], w[f"{p}.proj.bias"], 1, 0)
    return o + x


def tiny_wan(seed, widths=(16, 16, 8, 4, 4)):
    from naivediffusion_amd import vae
    cfg = vae.Wan22Config(latent_channels=8, widths=widths, resnets=2)
    g = np.random.default_rng(seed)
    w = {}
    for name, shape in vae.wan22_decoder_shapes(cfg).items():
        if name.endswith(".gamma"):
            w[name] = 1.0 + rnd(g, *shape, s=0.1)
        elif len(shape) == 1:
            w[name] = rnd(g, *shape, s=0.1)
        else:
            w[name] = rnd(g, *shape, s=1.0 / math.sqrt(np.prod(shape[1:])))
    return cfg, w, g


def test_wan_up_shortcut_moves_each_value_where_dup_up_puts_it():
    """DupUp3D on one frame, checked element by element: the same width a
    nearest upsample; half the width either the odd channels upsampled or
    out[o, 2y + r, 2x + s] = x[2o + r, y, x]."""
    g = np.random.default_rng(1)
    x = rnd(g, 1, 8, 3, 5, s=1.0)
    same = oracle.wan_up_shortcut(x, 8, False)
    assert np.array_equal(same, x.repeat(2, 2).repeat(2, 3))
    odd = oracle.wan_up_shortcut(x, 4, True)
    assert np.array_equal(odd, x[:, [1, 3, 5, 7]].repeat(2, 2).repeat(2, 3))
    inter = oracle.wan_up_shortcut(x, 4, False)
    for o in range(4):
        for yy in range(6):
            for xx in range(10):
                assert inter[0, o, yy, xx] == x[0, 2 * o + yy % 2, yy // 2, xx // 2]


def test_wan_blocks_against_float64():
    cfg, w, g = tiny_wan(2)
    x = rnd(g, 1, 16, 4, 5, s=1.0)
    assert close(oracle.wan_residual(x, w, "decoder.middle.0"), wan_residual64(x, w, "decoder.middle.0"))
    p = "decoder.upsamples.2.upsamples.0"   # 16 -> 8 through the 1x1 shortcut
    assert close(oracle.wan_residual(x, w, p), wan_residual64(x, w, p))
    got = oracle.wan_attention(x, w, "decoder.middle.1")
    exp = wan_attention64(x, w, "decoder.middle.1")
    assert close(got - x, exp - x)
    # the norm is over channels, per pixel: scaling one pixel's channels leaves its normalised values
    y = x.copy()
    y[:, :, 1, 2] *= 7.0
    a = oracle.wan_channel_rms(x, w["decoder.middle.0.residual.0.gamma"])
    b = oracle.wan_channel_rms(y, w["decoder.middle.0.residual.0.gamma"])
    assert np.allclose(a, b, rtol=1e-5, atol=1e-6)
    # zero second convolution: the block is its shortcut
    w[f"{p}.residual.6.weight"][:] = 0
    w[f"{p}.residual.6.bias"][:] = 0
    sc = oracle.conv2d(x, w[f"{p}.shortcut.weight"], w[f"{p}.shortcut.bias"], 1, 0)
    assert np.array_equal(oracle.wan_residual(x, w, p), sc)


def test_wan22_decoder_against_float64():
    cfg, w, g = tiny_wan(3)
    z = rnd(g, 1, 8, 2, 3, s=1.0)
    got = oracle.wan22_decoder(z, w)
    h = conv(conv(z, w["conv2.weight"], w["conv2.bias"], 1, 0), w["decoder.conv1.weight"], w["decoder.conv1.bias"])
    h = wan_residual64(h, w, "decoder.middle.0")
    h = wan_attention64(h, w, "decoder.middle.1")
    h = wan_residual64(h, w, "decoder.middle.2")
    flags = (True, True, True, False)   # levels 0..3 from the latent: entries 3, 2, 1, 0 of (F, T, T, T)
    for level in range(5):
        p = f"decoder.upsamples.{level}.upsamples"
        inp = h
        for i in range(cfg.resnets):
            h = wan_residual64(h, w, f"{p}.{i}")
        if level < 4:
            h = conv(h.repeat(2, 2).repeat(2, 3), w[f"{p}.{cfg.resnets}.resample.1.weight"],
                     w[f"{p}.{cfg.resnets}.resample.1.bias"])
            c_in, c_out = inp.shape[1], h.shape[1]
            if c_in == c_out:
                sc = inp.repeat(2, 2).repeat(2, 3)
            elif flags[level]:
                sc = inp[:, 1::2].repeat(2, 2).repeat(2, 3)
            else:
                sc = np.empty_like(h)
                for r in range(2):
                    sc[:, :, r::2, :] = inp[:, r::2].repeat(2, 3)
            h = h + sc
    h = conv(silu(channel_rms64(h, w["decoder.head.0.gamma"])), w["decoder.head.2.weight"], w["decoder.head.2.bias"])
    exp = h[:, :3]
    assert got.shape == exp.shape == (1, 3, 32, 48)
    assert close(got, exp, 5e-5)
