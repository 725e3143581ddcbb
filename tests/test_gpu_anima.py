"""GPU parity of the Anima denoiser (Models/Anima/AnimaDit.cs) against the
oracle's composition of the same block from its pinned primitives: one
block (self-attention with the 3-D rotary tables, cross-attention into the
context, exact-GELU MLP, low-rank adaLN with the shared term) at fp32,
fp16 and bf16 compute, at the 2B's width and at a narrow width; the whole
step (device patchify, embedding, time path, blocks, final layer,
channel-last unpatchify); and the patch layouts bit-exact. Tolerances:
max|gpu - oracle| / max|oracle| <= 1e-3 at fp32, 2e-2 at bf16/fp16."""

import numpy as np
import pytest

import naivediffusion_amd as nd
import oracle
from naivediffusion_amd import anima, rng
from naivediffusion_amd.graph import PATCH_CHANNEL_FIRST, PATCH_CHANNEL_LAST, Ops
from naivediffusion_amd.layers import Transformer
from naivediffusion_amd.tensors import HostDataType as DT, HostTensor
from conftest import rel_err

pytestmark = pytest.mark.gpu

TOL = {DT.Float32: 1e-3, DT.Float16: 2e-2, DT.BFloat16: 2e-2}
NARROW = anima.AnimaConfig(width=512, heads=4, mlp=1024, blocks=2, context_width=256, adaln_rank=64)
FULL = anima.AnimaConfig(blocks=1)


def normal(name, shape, std=1.0):
    return rng.normal(rng.tensor_seed(23, name), shape, 0.0, std)


def block_case(cfg, n_rows, n_cols, n_ctx):
    n = n_rows * n_cols
    D = cfg.width
    w = anima.synthetic_weights(cfg, 5, list(anima.block_weight_shapes(cfg, 0)), norm_spread=0.1)
    x = normal("x", (n, D))
    time = Transformer.Sinusoid(0.7, D)
    temb = oracle.rms_norm(time.reshape(1, D), np.ones(D, np.float32) + normal("tn", (D,), 0.1))[0]
    lora = normal("lora", (3 * D,), 0.5)
    ctx = normal("ctx", (n_ctx, cfg.context_width))
    cos, sin = anima.rope_tables(n_rows, n_cols, cfg.head_dim)
    return w, x, temb, lora, ctx, cos, sin


@pytest.mark.parametrize("cfg,n_rows,n_cols,n_ctx", [(NARROW, 8, 10, 24), (FULL, 16, 16, 64)], ids=["narrow", "2B"])
@pytest.mark.parametrize("compute", [DT.Float32, DT.BFloat16, DT.Float16])
def test_anima_block(device, cfg, n_rows, n_cols, n_ctx, compute):
    print(f"[gpu] anima block D={cfg.width} tokens={n_rows * n_cols} ctx={n_ctx} {compute.name}", flush=True)
    n = n_rows * n_cols
    D = cfg.width
    w, x, temb, lora, ctx, cos, sin = block_case(cfg, n_rows, n_cols, n_ctx)
    model = anima.build_block_model(device, cfg, w, n, n_ctx, compute)
    half = cfg.head_dim // 2
    out = model.Run(HostTensor.FromFloats(x.reshape(1, 1, n, D)), HostTensor.FromFloats(temb.reshape(1, 1, 1, D)),
                    HostTensor.FromFloats(lora.reshape(1, 1, 1, 3 * D)),
                    HostTensor.FromFloats(ctx.reshape(1, 1, n_ctx, cfg.context_width)),
                    HostTensor.FromFloats(cos.reshape(1, n, 1, half)),
                    HostTensor.FromFloats(sin.reshape(1, n, 1, half)))[0].ToFloats().reshape(n, D)
    model.Dispose()
    # The GPU sees the context at the compute type.
    ctx_in = ctx if compute == DT.Float32 else HostTensor.FromFloats(ctx).ConvertTo(compute).ToFloats()
    ref = oracle.anima_block(x, temb, lora, ctx_in.reshape(n_ctx, -1), w, 0, cfg.heads, cos, sin)
    # The block's update, not the residual it is added to, is what the
    # tolerance measures.
    err = rel_err(out - x, ref - x)
    print(f"[gpu]   rel err of the update {err:.2e}", flush=True)
    assert err <= TOL[compute]


@pytest.mark.parametrize("compute", [DT.Float32, DT.BFloat16])
def test_anima_step(device, compute):
    cfg = NARROW
    lat_h, lat_w, n_ctx = 16, 20, 24
    print(f"[gpu] anima step {cfg.blocks} blocks latent {lat_h}x{lat_w} {compute.name}", flush=True)
    w = anima.synthetic_weights(cfg, 9, norm_spread=0.1)
    latent = normal("latent", (cfg.latent_channels, lat_h, lat_w))
    ctx = normal("context", (n_ctx, cfg.context_width))
    den = anima.AnimaDit(device, cfg, w, lat_h * 8, lat_w * 8, n_ctx, compute)
    flow = den.Predict(HostTensor.FromFloats(latent), 500.0, 0.6, {"context": ctx}).ToFloats()
    den.Dispose()
    ctx_in = ctx if compute == DT.Float32 else HostTensor.FromFloats(ctx).ConvertTo(compute).ToFloats()
    ref = oracle.anima_step(latent, 0.6, ctx_in.reshape(n_ctx, -1), w, cfg.blocks, cfg.heads)
    assert flow.reshape(ref.shape).shape == ref.shape
    err = rel_err(flow.reshape(ref.shape), ref)
    print(f"[gpu]   rel err {err:.2e}", flush=True)
    assert err <= TOL[compute]


def test_anima_patch_layouts_bit_exact(device):
    C, H, W = 16, 6, 10
    latent = normal("pl", (C, H, W))
    g = nd.Graph(device)
    x = g.Input(DT.Float32, [1, C, H, W])
    t = g.Input(DT.Float32, [1, 1, (H // 2) * (W // 2), C * 4])
    m = nd.CompiledModel(g, [Ops.Patchify(x, 2, PATCH_CHANNEL_FIRST),
                             Ops.Unpatchify(t, 2, C, H, W, PATCH_CHANNEL_LAST)], device)
    tok = normal("pt", ((H // 2) * (W // 2), C * 4))
    p, u = m.Dispatch([HostTensor.FromFloats(latent.reshape(1, C, H, W)),
                       HostTensor.FromFloats(tok.reshape(1, 1, -1, C * 4))])
    assert np.array_equal(p.ToFloats().reshape(tok.shape), oracle.anima_patchify(latent))
    assert np.array_equal(u.ToFloats().reshape(C, H, W), oracle.anima_unpatchify(tok, C, H, W))


def test_anima_device_weights_match_host_weights(device):
    """Weights made on the device (stacked and column-sliced there) give the
    same step, bit for bit, as the same values passed from the host."""
    cfg = NARROW
    lat, n_ctx = 8, 16
    dw = anima.device_weights(device, cfg, 13, DT.BFloat16)
    hw = {k: t.Download().ToFloats().reshape(t.Shape) for k, t in dw.items()}
    latent = normal("dl", (cfg.latent_channels, lat, lat))
    ctx = normal("dc", (n_ctx, cfg.context_width))
    outs = []
    for w in (dw, hw):
        den = anima.AnimaDit(device, cfg, w, lat * 8, lat * 8, n_ctx, DT.BFloat16)
        outs.append(den.Predict(HostTensor.FromFloats(latent), 500.0, 0.4, {"context": ctx}).ToFloats())
        den.Dispose()
    assert np.array_equal(outs[0], outs[1])
