"""GPU parity at the real sizes of the five benchmark configurations.

Each configuration's unit (one block, or one resnet / Transformer2d per UNet
level) runs at its full token count against the oracle on the same seeded
inputs: max|gpu - oracle| / max|oracle| <= 2e-2 at bf16/fp16 compute and
1e-3 at fp32, with int8 weights compared against the oracle on the
dequantised weights. The full multi-block steps are too large for the oracle
(about 100 TFLOP for the 60-block MMDiT), so they are checked through
properties that hold at any size: every output finite; the two-stream
schedule equal to the one-stream schedule bit for bit, and a rerun equal to
the first run; each element of a CFG batch equal, within the bf16 bound, to
a batch-1 run on it alone; and the bf16 (fp16) step within 5e-2 of the same
step computed in fp32 on the GPU (the per-block bound, 2e-2, with headroom
for a chain of 28 to 60 blocks).

Weights are made on the GPU by the library's counter-based generator (the
host generator's values; about 100x faster than making 340 M host normals)
and one copy is downloaded for the oracle.
"""

import math

import numpy as np
import pytest

import naivediffusion_amd as nd
import oracle
from naivediffusion_amd import anima, mmdit, rng, sdxl
from naivediffusion_amd.layers import Layers, Transformer
from naivediffusion_amd.tensors import HostDataType as DT, HostTensor
from naivediffusion_amd.weights import WeightSet
from conftest import rel_err

pytestmark = pytest.mark.gpu

STEP_TOL = 5e-2
MM = mmdit.MmditConfig(blocks=1)


def say(msg):
    print(f"[gpu] {msg}", flush=True)


def download(ws):
    return {k: t.Download().ToFloats().reshape(t.Shape) for k, t in ws.items()}


def stream_weights(w, s):
    p = f"blocks.0.{s}"
    return dict(w_mod=w[f"{p}_mod.weight"], b_mod=w[f"{p}_mod.bias"], w_qkv=w[f"{p}_qkv.weight"],
                b_qkv=w[f"{p}_qkv.bias"], norm_q=w[f"{p}_norm_q.weight"], norm_k=w[f"{p}_norm_k.weight"],
                w_o=w[f"{p}_out.weight"], b_o=w[f"{p}_out.bias"], w_fc1=w[f"{p}_fc1.weight"],
                b_fc1=w[f"{p}_fc1.bias"], w_fc2=w[f"{p}_fc2.weight"], b_fc2=w[f"{p}_fc2.bias"])


def mmdit_block_names():
    return list(mmdit.block_weight_shapes(MM, 0))


def normal(device, seed, name, shape, std=1.0):
    """N(0, std) values from the library's device generator (the host
    generator's rule), downloaded."""
    t = device.Normal(DT.Float32, shape, rng.tensor_seed(seed, name), 0.0, std)
    a = t.Download().ToFloats().reshape(shape)
    t.Dispose()
    return a


def mmdit_inputs(device, seed, batch, ni, nt, grid):
    D = MM.width
    xi = normal(device, seed, "x_img", (batch, 1, ni, D))
    xt = normal(device, seed, "x_txt", (batch, 1, nt, D))
    temb = normal(device, seed, "temb", (batch, 1, 1, D))
    cos, sin = mmdit.rope_tables(grid[0], grid[1], nt)
    return xi, xt, temb, cos, sin


def run_mmdit_block(device, weights, xi, xt, temb, cos, sin, compute, int8=False):
    B, _, ni, D = xi.shape
    nt = xt.shape[2]
    n = ni + nt
    model = mmdit.build_block_model(device, MM, weights, B, ni, nt, compute, int8)
    yi, yt = model.Run(HostTensor.FromFloats(xi), HostTensor.FromFloats(xt), HostTensor.FromFloats(temb),
                       HostTensor.FromFloats(cos.reshape(1, n, 1, 64)), HostTensor.FromFloats(sin.reshape(1, n, 1, 64)))
    model.Dispose()
    return yi.ToFloats().reshape(B, ni, D), yt.ToFloats().reshape(B, nt, D)


# ---- configuration 3: 60-block MMDiT at 1024x1344 (5376 + 256 tokens) -------------

@pytest.fixture(scope="module")
def config3_block(device):
    say("config 3: one MMDiT block's weights (made on the GPU)")
    dw = mmdit.device_weights(device, MM, 31, mmdit_block_names(), norm_spread=0.1)
    w = download(dw)
    for t in dw.values():
        t.Dispose()
    xi, xt, temb, cos, sin = mmdit_inputs(device, 31, 1, 5376, 256, (64, 84))
    say("config 3: oracle block at 5376 + 256 tokens")
    ri, rt = oracle.mmdit_block(xi.reshape(-1, MM.width), xt.reshape(-1, MM.width), temb.ravel(),
                                stream_weights(w, "img"), stream_weights(w, "txt"), MM.heads, cos, sin, -1, MM.eps)
    return w, (xi, xt, temb, cos, sin), (ri, rt)


@pytest.mark.parametrize("compute,tol", [(DT.BFloat16, 2e-2), (DT.Float32, 1e-3)])
def test_config3_block_at_full_size(device, config3_block, compute, tol):
    w, (xi, xt, temb, cos, sin), (ri, rt) = config3_block
    say(f"config 3: block 5376 + 256 tokens, {compute.name}")
    yi, yt = run_mmdit_block(device, w, xi, xt, temb, cos, sin, compute)
    ei, et = rel_err(yi[0], ri), rel_err(yt[0], rt)
    say(f"  image {ei:.2e} text {et:.2e} (bound {tol})")
    assert ei <= tol and et <= tol
    assert rel_err(xi.reshape(ri.shape), ri) > 10 * tol


def _mmdit_step_inputs(device, B, lat_h, lat_w, nt, seed):
    cfg = mmdit.MmditConfig()
    gh, gw = lat_h // cfg.patch, lat_w // cfg.patch
    n = gh * gw + nt
    cos, sin = mmdit.rope_tables(gh, gw, nt)
    latent = normal(device, seed, "latent", (B, cfg.latent_channels, lat_h, lat_w))
    text = normal(device, seed, "text", (B, 1, nt, cfg.text_dim))
    temb = np.tile(mmdit.time_embedding(0.5, cfg.time_dim), (B, 1)).reshape(B, 1, 1, cfg.time_dim)
    return [latent, text, np.ascontiguousarray(temb, np.float32), cos.reshape(1, n, 1, 64), sin.reshape(1, n, 1, 64)]


def _mmdit_step(device, ins, B, lat_h, lat_w, nt, compute, seed, two_streams=True, int8=False, runs=1):
    cfg = mmdit.MmditConfig()
    model = mmdit.build_step_model(device, cfg, mmdit.device_weights(device, cfg, seed), B, nt, lat_h, lat_w,
                                   compute, int8, two_streams)
    host = [HostTensor.FromFloats(a) for a in ins]
    outs = [model.Run(*host)[0].ToFloats().reshape(B, cfg.latent_channels, lat_h, lat_w) for _ in range(runs)]
    model.Dispose()
    device.ReleasePooledBuffers()
    return outs


def test_config3_step_properties(device):
    """The 60-block step at 1024x1344: finite; the two-stream schedule and a
    rerun equal to the one-stream run bit for bit; bf16 within 5e-2 of the
    fp32 step on the GPU."""
    B, lat_h, lat_w, nt, seed = 1, 128, 168, 256, 3
    ins = _mmdit_step_inputs(device, B, lat_h, lat_w, nt, seed)
    say("config 3: 60-block step, bf16, two streams, two runs")
    two = _mmdit_step(device, ins, B, lat_h, lat_w, nt, DT.BFloat16, seed, runs=2)
    assert np.all(np.isfinite(two[0]))
    assert np.array_equal(two[0], two[1])
    say("config 3: 60-block step, bf16, one stream")
    one = _mmdit_step(device, ins, B, lat_h, lat_w, nt, DT.BFloat16, seed, two_streams=False)[0]
    assert np.array_equal(one, two[0])
    say("config 3: 60-block step, fp32")
    f32 = _mmdit_step(device, ins, B, lat_h, lat_w, nt, DT.Float32, seed)[0]
    assert np.all(np.isfinite(f32))
    err = rel_err(two[0], f32)
    say(f"  bf16 step vs fp32 step {err:.2e} (bound {STEP_TOL}); output std {np.std(f32):.3f}")
    assert err <= STEP_TOL


# ---- configuration 4: 60-block MMDiT at 1328x1328, CFG batch 2, int8 per channel ----

def test_config4_block_int8_per_channel_at_full_size(device):
    """One block at 6889 + 256 tokens, batch 2 (cond + uncond), every linear
    int8 with one fp32 scale per output channel, bf16 compute: each batch
    element against a batch-1 oracle run on the dequantised weights."""
    say("config 4: one block's weights, quantised per channel on the GPU")
    names = mmdit_block_names()
    dw = mmdit.device_weights(device, MM, 41, names, norm_spread=0.1)
    w = download(dw)
    deq = {}
    for k, v in w.items():
        if v.ndim == 2 and v.size >= (1 << 16):
            q, s = oracle.quantize(v, v.shape[0], block=v.shape[1], fp16_scales=False)
            deq[k] = q.astype(np.float32) * s
        else:
            deq[k] = v
    xi, xt, temb, cos, sin = mmdit_inputs(device, 41, 2, 6889, 256, (83, 83))
    say("config 4: block 6889 + 256 tokens, B=2, int8 per channel")
    yi, yt = run_mmdit_block(device, dw, xi, xt, temb, cos, sin, DT.BFloat16, int8="channel")
    for t in dw.values():
        t.Dispose()
    for b in range(2):
        say(f"config 4: oracle, batch element {b}")
        ri, rt = oracle.mmdit_block(xi[b].reshape(-1, MM.width), xt[b].reshape(-1, MM.width), temb[b].ravel(),
                                    stream_weights(deq, "img"), stream_weights(deq, "txt"), MM.heads, cos, sin, -1,
                                    MM.eps)
        ei, et = rel_err(yi[b], ri), rel_err(yt[b], rt)
        say(f"  element {b}: image {ei:.2e} text {et:.2e}")
        assert ei <= 2e-2 and et <= 2e-2


def test_config4_step_properties(device):
    """The 60-block int8 step at 1328x1328, batch 2: finite, and each batch
    element within the bf16 bound of a batch-1 step on it alone."""
    B, lat, nt, seed = 2, 166, 256, 4
    ins = _mmdit_step_inputs(device, B, lat, lat, nt, seed)
    say("config 4: 60-block step, int8 per channel, batch 2")
    both = _mmdit_step(device, ins, B, lat, lat, nt, DT.BFloat16, seed, int8="channel")[0]
    assert np.all(np.isfinite(both))
    one_ins = [ins[0][:1], ins[1][:1], ins[2][:1], ins[3], ins[4]]
    say("config 4: 60-block step, int8 per channel, batch 1")
    single = _mmdit_step(device, one_ins, 1, lat, lat, nt, DT.BFloat16, seed, int8="channel")[0]
    err = rel_err(both[:1], single)
    say(f"  batch element 0 vs the batch-1 step {err:.2e}")
    assert err <= 2e-2


# ---- configuration 1: Anima 2B, 28 blocks, 4096 tokens, context 512 ----------------------

AN = anima.AnimaConfig(blocks=1)


@pytest.fixture(scope="module")
def config1_block(device):
    say("config 1: one Anima block's weights (made on the GPU)")
    dw = anima.device_weights(device, AN, 51, DT.BFloat16, list(anima.block_weight_shapes(AN, 0)), norm_spread=0.1)
    w = download(dw)
    for t in dw.values():
        t.Dispose()
    D, n, n_ctx = AN.width, 4096, 512
    x = normal(device, 51, "x", (n, D))
    time = Transformer.Sinusoid(0.5, D)
    temb = oracle.rms_norm(time.reshape(1, D), np.ones(D, np.float32))[0]
    lora = rng.normal(rng.tensor_seed(51, "lora"), (3 * D,), 0.0, 0.5)
    ctx = normal(device, 51, "ctx", (n_ctx, AN.context_width))
    cos, sin = anima.rope_tables(64, 64, AN.head_dim)
    return w, (x, temb, lora, ctx, cos, sin)


@pytest.mark.parametrize("compute,tol", [(DT.Float32, 1e-3), (DT.BFloat16, 2e-2)])
def test_config1_block_at_full_size(device, config1_block, compute, tol):
    w, (x, temb, lora, ctx, cos, sin) = config1_block
    D, n, n_ctx, half = AN.width, x.shape[0], ctx.shape[0], AN.head_dim // 2
    say(f"config 1: Anima block, 4096 tokens, context 512x1024, {compute.name}")
    model = anima.build_block_model(device, AN, w, n, n_ctx, compute)
    out = model.Run(HostTensor.FromFloats(x.reshape(1, 1, n, D)), HostTensor.FromFloats(temb.reshape(1, 1, 1, D)),
                    HostTensor.FromFloats(lora.reshape(1, 1, 1, 3 * D)),
                    HostTensor.FromFloats(ctx.reshape(1, 1, n_ctx, -1)),
                    HostTensor.FromFloats(cos.reshape(1, n, 1, half)),
                    HostTensor.FromFloats(sin.reshape(1, n, 1, half)))[0].ToFloats().reshape(n, D)
    model.Dispose()
    ctx_in = ctx if compute == DT.Float32 else HostTensor.FromFloats(ctx).ConvertTo(compute).ToFloats()
    say("config 1: oracle block")
    ref = oracle.anima_block(x, temb, lora, ctx_in.reshape(n_ctx, -1), w, 0, AN.heads, cos, sin)
    err = rel_err(out - x, ref - x)
    say(f"  update rel err {err:.2e} (bound {tol})")
    assert err <= tol


def test_config1_step_properties(device):
    """The 28-block Anima step at 1024x1024: finite, a rerun equal bit for
    bit, bf16 within 5e-2 of the fp32 step on the GPU."""
    cfg = anima.AnimaConfig()
    lat, n_ctx, seed = 128, 512, 6
    latent = normal(device, seed, "latent", (cfg.latent_channels, lat, lat))
    ctx = normal(device, seed, "context", (n_ctx, cfg.context_width))
    outs = {}
    for compute in (DT.BFloat16, DT.Float32):
        say(f"config 1: 28-block Anima step, {compute.name}")
        den = anima.AnimaDit(device, cfg, anima.device_weights(device, cfg, seed, DT.BFloat16), lat * 8, lat * 8,
                             n_ctx, compute)
        runs = [den.Predict(HostTensor.FromFloats(latent), 500.0, 0.5, {"context": ctx}).ToFloats().ravel()
                for _ in range(2)]
        den.Dispose()
        device.ReleasePooledBuffers()
        assert np.all(np.isfinite(runs[0])) and np.array_equal(runs[0], runs[1])
        outs[compute] = runs[0]
    err = rel_err(outs[DT.BFloat16], outs[DT.Float32])
    say(f"  bf16 step vs fp32 step {err:.2e} (bound {STEP_TOL})")
    assert err <= STEP_TOL


# ---- configuration 2: SDXL UNet at 1024x1024, CFG batch 2, fp16 ----------------------

SD = sdxl.SdxlConfig()


def sdxl_unit_weights(device, prefix, dtype, seed=61):
    """The unit's weights as sdxl._init makes them (norm weights 1 and biases
    0 plus N(0, 0.05); matrices and filters N(0, 1/fan_in); biases N(0,
    0.02)), made on the GPU at dtype and downloaded."""
    out = {}
    for name, shape in sdxl.weight_shapes(SD).items():
        if not name.startswith(prefix + "."):
            continue
        if ".norm" in name:
            mean, std = (1.0 if name.endswith("weight") else 0.0), 0.05
        elif len(shape) == 1:
            mean, std = 0.0, 0.02
        else:
            mean, std = 0.0, 1.0 / math.sqrt(int(np.prod(shape[1:])))
        t = device.Normal(dtype, shape, rng.tensor_seed(seed, name), mean, std)
        out[name] = t.Download().ToFloats().reshape(shape)
        t.Dispose()
    return out


def narrow(x, dtype):
    return HostTensor.FromFloats(np.asarray(x, np.float32)).ConvertTo(dtype).ToFloats().reshape(np.shape(x))


@pytest.mark.parametrize("prefix,size", [("down_blocks.0.resnets.0", 128), ("down_blocks.1.resnets.0", 64),
                                         ("down_blocks.2.resnets.0", 32)], ids=["320ch-128", "640ch-64", "1280ch-32"])
def test_config2_resnet_at_full_size(device, prefix, size):
    """One resnet per UNet level at its 1024x1024 extent, batch 2, fp16 (the
    640 and 1280 levels' first resnets carry the 1x1 shortcut)."""
    dtype, B = DT.Float16, 2
    w = sdxl_unit_weights(device, prefix, dtype)
    cin = w[f"{prefix}.norm1.weight"].shape[0]
    x = narrow(normal(device, 62, prefix, (B, cin, size, size)), dtype)
    temb = narrow(rng.normal(rng.tensor_seed(63, prefix), (B, SD.time_embed)), dtype)
    say(f"config 2: resnet {prefix}, {cin} channels at {size}x{size}, B=2, fp16")
    model = nd.ModelBuilder(device, dtype)
    W = WeightSet(model, w, dtype, device)
    xin = model.Placeholder([B, cin, size, size], dtype)
    tin = model.Placeholder([B, 1, 1, SD.time_embed], dtype)
    model.Compile([sdxl.resnet_block(model, W, SD, xin, Layers.Silu(tin), prefix)])
    out = model.Run(HostTensor.FromFloats(x).ConvertTo(dtype),
                    HostTensor.FromFloats(temb.reshape(B, 1, 1, -1)).ConvertTo(dtype))[0].ToFloats()
    model.Dispose()
    say("config 2: oracle resnet")
    ref = oracle.sdxl_resnet(x, narrow(oracle.silu(temb), dtype), w, prefix, SD.groups, SD.eps)
    err = rel_err(out.reshape(ref.shape), ref)
    say(f"  rel err {err:.2e}")
    assert err <= 2e-2


@pytest.mark.parametrize("prefix,C,size,heads,layers", [("down_blocks.1.attentions.0", 640, 64, 10, 2),
                                                        ("mid_block.attentions.0", 1280, 32, 20, 10)],
                         ids=["640ch-64-depth2", "1280ch-32-depth10"])
def test_config2_transformer2d_at_full_size(device, prefix, C, size, heads, layers):
    """The Transformer2d of the 64x64 level (depth 2, 10 heads of 64) and of
    the 32x32 level (depth 10, 20 heads), batch 2, 77x2048 context, fp16."""
    dtype, B, tokens = DT.Float16, 2, 77
    w = sdxl_unit_weights(device, prefix, dtype)
    x = narrow(normal(device, 64, prefix, (B, C, size, size)), dtype)
    ctx = narrow(normal(device, 65, prefix, (B, tokens, SD.context_width)), dtype)
    say(f"config 2: Transformer2d {prefix}, {C} channels at {size}x{size}, depth {layers}, B=2, fp16")
    model = nd.ModelBuilder(device, dtype)
    W = WeightSet(model, w, dtype, device)
    xin = model.Placeholder([B, C, size, size], dtype)
    cin = model.Placeholder([B, 1, tokens, SD.context_width], dtype)
    model.Compile([sdxl.transformer2d(model, W, SD, xin, cin, prefix, heads, layers)])
    out = model.Run(HostTensor.FromFloats(x).ConvertTo(dtype),
                    HostTensor.FromFloats(ctx.reshape(B, 1, tokens, -1)).ConvertTo(dtype))[0].ToFloats()
    model.Dispose()
    say("config 2: oracle Transformer2d")
    ref = oracle.sdxl_transformer2d(x, ctx, w, prefix, heads, layers, SD.groups, SD.transformer_eps,
                                    SD.layer_norm_eps)
    err = rel_err(out.reshape(ref.shape) - x, ref - x)
    say(f"  update rel err {err:.2e}")
    assert err <= 2e-2


def test_config2_unet_step_properties(device):
    """The whole UNet at 1024x1024: batch 2 finite and a rerun equal bit for
    bit; batch element 0 within the fp16 bound of a batch-1 run on it; fp16
    within 5e-2 of the fp32 UNet on the GPU."""
    lat, tokens, seed = 128, 77, 7
    t = sdxl.timestep_embedding([500.0], SD.block_out[0])
    add = np.stack([sdxl.add_conditioning(rng.normal(rng.tensor_seed(seed, f"pool{b}"), (SD.pooled_width,)),
                                          add_time_dim=SD.add_time_dim) for b in range(2)])
    sample = normal(device, seed, "latent", (2, SD.in_channels, lat, lat))
    ctx = normal(device, seed, "context", (2, 1, tokens, SD.context_width))

    def run(B, compute, runs=1):
        model = sdxl.build_unet(device, SD, sdxl.device_weights(device, SD, seed, DT.Float16), B, lat, lat, tokens,
                                compute)
        ins = [HostTensor.FromFloats(sample[:B]).ConvertTo(compute),
               HostTensor.FromFloats(np.tile(t, (B, 1)).reshape(B, 1, 1, -1)).ConvertTo(compute),
               HostTensor.FromFloats(add[:B].reshape(B, 1, 1, -1)).ConvertTo(compute),
               HostTensor.FromFloats(ctx[:B]).ConvertTo(compute)]
        outs = [model.Run(*ins)[0].ToFloats().reshape(B, SD.in_channels, lat, lat) for _ in range(runs)]
        model.Dispose()
        device.ReleasePooledBuffers()
        return outs

    say("config 2: UNet step, B=2, fp16, two runs")
    both = run(2, DT.Float16, runs=2)
    assert np.all(np.isfinite(both[0])) and np.array_equal(both[0], both[1])
    say("config 2: UNet step, B=1, fp16")
    single = run(1, DT.Float16)[0]
    e1 = rel_err(both[0][:1], single)
    say(f"  batch element 0 vs the batch-1 run {e1:.2e}")
    assert e1 <= 2e-2
    say("config 2: UNet step, B=2, fp32")
    f32 = run(2, DT.Float32)[0]
    e2 = rel_err(both[0], f32)
    say(f"  fp16 UNet vs fp32 UNet {e2:.2e} (bound {STEP_TOL})")
    assert e2 <= STEP_TOL
