"""GPU parity of SDXL's UNet units (Models/Sdxl/UNetModel.cs) against the
oracle's composition of the same units from its pinned primitives: the
resnet block with and without the 1x1 shortcut at SDXL's widths, the
Transformer2d with a 64-wide-head attention and the 2048-wide context,
and a whole UNet of SDXL's structure at narrow widths (every level, the
skip joins, the stride-2 downsamplers, the cropped upsample at an odd
extent). Tolerance: max|gpu - oracle| / max|oracle| <= 2e-2 at fp16/bf16,
1e-3 at fp32."""

import numpy as np
import pytest

import naivediffusion_amd as nd
import oracle
from naivediffusion_amd import rng, sdxl
from naivediffusion_amd.layers import Layers
from naivediffusion_amd.tensors import HostDataType as DT, HostTensor
from naivediffusion_amd.weights import WeightSet
from conftest import rel_err

pytestmark = pytest.mark.gpu

TOL = {DT.Float32: 1e-3, DT.Float16: 2e-2, DT.BFloat16: 2e-2}
SMALL = sdxl.SdxlConfig(block_out=(64, 128, 128), transformer_layers=(0, 1, 1), heads=(1, 2, 2), context_width=64,
                        time_embed=256, add_time_dim=32, pooled_width=128)


def normal(name, shape, std=1.0):
    return rng.normal(rng.tensor_seed(31, name), shape, 0.0, std)


def narrow(x, dtype):
    return HostTensor.FromFloats(np.asarray(x, np.float32)).ConvertTo(dtype).ToFloats().reshape(np.shape(x))


def unit_weights(cfg, prefix, dtype):
    full = sdxl.weight_shapes(cfg)
    return {k: narrow(np.asarray(sdxl._init(k, s, 3), np.float32), dtype)
            for k, s in full.items() if k.startswith(prefix + ".")}


@pytest.mark.parametrize("prefix,B,H,W", [("down_blocks.1.resnets.0", 2, 16, 12), ("up_blocks.0.resnets.2", 1, 8, 8),
                                          ("down_blocks.0.resnets.1", 2, 24, 20)])
@pytest.mark.parametrize("dtype", [DT.Float16, DT.BFloat16])
def test_resnet_block(device, prefix, B, H, W, dtype):
    cfg = sdxl.SdxlConfig()
    w = unit_weights(cfg, prefix, dtype)
    cin = w[f"{prefix}.norm1.weight"].shape[0]
    print(f"[gpu] resnet {prefix} cin={cin} {B}x{H}x{W} {dtype.name}", flush=True)
    x = narrow(normal("x", (B, cin, H, W)), dtype)
    temb = narrow(normal("t", (B, cfg.time_embed)), dtype)
    model = nd.ModelBuilder(device, dtype)
    W_ = WeightSet(model, w, dtype, device)
    xin = model.Placeholder([B, cin, H, W], dtype)
    tin = model.Placeholder([B, 1, 1, cfg.time_embed], dtype)
    y = sdxl.resnet_block(model, W_, cfg, xin, Layers.Silu(tin), prefix)
    model.Compile([y])
    model.Compiled.SetProfiling(True)
    out = model.Run(HostTensor.FromFloats(x).ConvertTo(dtype),
                    HostTensor.FromFloats(temb.reshape(B, 1, 1, -1)).ConvertTo(dtype))[0].ToFloats()
    fams = set(model.Compiled.Profile())
    model.Dispose()
    st = narrow(oracle.silu(temb), dtype)
    ref = oracle.sdxl_resnet(x, st, w, prefix, cfg.groups, cfg.eps)
    err = rel_err(out.reshape(ref.shape), ref)
    print(f"[gpu]   rel err {err:.2e} via {sorted(fams)}", flush=True)
    assert any(f.startswith("conv_mfma_") for f in fams), fams
    assert err <= TOL[dtype]


@pytest.mark.parametrize("dtype", [DT.Float16, DT.BFloat16])
def test_transformer2d(device, dtype):
    cfg = sdxl.SdxlConfig(transformer_layers=(0, 1, 1))
    prefix = "down_blocks.1.attentions.0"
    w = unit_weights(cfg, prefix, dtype)
    B, C, H, W, tokens = 2, 640, 12, 10, 77
    print(f"[gpu] transformer2d {C}ch {H}x{W} ctx {tokens} {dtype.name}", flush=True)
    x = narrow(normal("tx", (B, C, H, W)), dtype)
    ctx = narrow(normal("ctx", (B, tokens, cfg.context_width)), dtype)
    model = nd.ModelBuilder(device, dtype)
    W_ = WeightSet(model, w, dtype, device)
    xin = model.Placeholder([B, C, H, W], dtype)
    cin = model.Placeholder([B, 1, tokens, cfg.context_width], dtype)
    model.Compile([sdxl.transformer2d(model, W_, cfg, xin, cin, prefix, 10, 1)])
    out = model.Run(HostTensor.FromFloats(x).ConvertTo(dtype),
                    HostTensor.FromFloats(ctx.reshape(B, 1, tokens, -1)).ConvertTo(dtype))[0].ToFloats()
    model.Dispose()
    ref = oracle.sdxl_transformer2d(x, ctx, w, prefix, 10, 1, cfg.groups, cfg.transformer_eps, cfg.layer_norm_eps)
    err = rel_err(out.reshape(ref.shape) - x, ref - x)
    print(f"[gpu]   rel err of the update {err:.2e}", flush=True)
    assert err <= TOL[dtype]


@pytest.mark.parametrize("H,W", [(16, 16), (18, 14)])
@pytest.mark.parametrize("dtype", [DT.Float16, DT.Float32])
def test_unet_small(device, H, W, dtype):
    cfg = SMALL
    B, tokens = 2, 8
    print(f"[gpu] unet (narrow) latent {H}x{W} B={B} {dtype.name}", flush=True)
    store = DT.Float16 if dtype == DT.Float32 else dtype
    w = sdxl.synthetic_weights(cfg, 4, store)
    sample = narrow(normal("s", (B, cfg.in_channels, H, W)), dtype)
    time = narrow(np.tile(sdxl.timestep_embedding([500.0], cfg.block_out[0]), (B, 1)), dtype)
    add = narrow(np.stack([sdxl.add_conditioning(normal(f"pool{b}", (cfg.pooled_width,)),
                                                 add_time_dim=cfg.add_time_dim) for b in range(B)]), dtype)
    ctx = narrow(normal("c", (B, tokens, cfg.context_width)), dtype)
    model = sdxl.build_unet(device, cfg, w, B, H, W, tokens, dtype)
    out = model.Run(HostTensor.FromFloats(sample).ConvertTo(dtype),
                    HostTensor.FromFloats(time.reshape(B, 1, 1, -1)).ConvertTo(dtype),
                    HostTensor.FromFloats(add.reshape(B, 1, 1, -1)).ConvertTo(dtype),
                    HostTensor.FromFloats(ctx.reshape(B, 1, tokens, -1)).ConvertTo(dtype))[0].ToFloats()
    model.Dispose()
    ref = oracle.sdxl_unet(sample, time, add, ctx, w, cfg)
    err = rel_err(out.reshape(ref.shape), ref)
    print(f"[gpu]   rel err {err:.2e}", flush=True)
    assert err <= TOL[dtype]
