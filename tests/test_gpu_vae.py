"""GPU parity of the VAE decoders (AutoencoderKl.Decoder, Vae/AutoencoderKl.cs;
Wan22Vae.Decoder, Vae/Wan22Vae.cs)
against the oracle's composition, which a float64 restatement pins: a small
decoder of the same layout at fp32 (1e-3) and bf16 (2e-2), SDXL's own widths
on a 16x16 latent (a 128x128 image), and the full 1024x1024 decode checked
through what holds at any size (every pixel finite, the bf16 decode within
5e-2 of the fp32 one). The row softmax the attention uses is checked on its
own against float64. Tolerance: max|gpu - oracle| / max|oracle|. The latent
goes in in the sampler's scale; the decoder divides by SDXL's scaling factor
(LatentSpace.FromModelScale) and the oracle is handed the divided latent."""

import numpy as np
import pytest

import oracle
from naivediffusion_amd import rng, vae
from naivediffusion_amd.graph import CompiledModel, Graph, Ops
from naivediffusion_amd.tensors import HostDataType as DT, HostTensor
from conftest import rel_err

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu] {msg}", flush=True)


@pytest.mark.parametrize("dtype,tol", [(DT.Float32, 4e-6), (DT.BFloat16, 8e-3), (DT.Float16, 1e-3)])
@pytest.mark.parametrize("cols", [1, 7, 8, 300, 2048, 16384])
def test_row_softmax_against_float64(device, dtype, tol, cols):
    """Every probability within the output type's rounding of float64's, on
    rows not a multiple of the 8-wide loads and longer than
    one pass of the workgroup."""
    say(f"softmax {dtype.name} x {cols}")
    r = np.random.default_rng(cols)
    rows = 37
    x = HostTensor.FromFloats((r.standard_normal((rows, cols)) * 4).astype(np.float32)).ConvertTo(dtype)
    scale = 0.3
    g = Graph(device)
    xi = g.Input(dtype, [1, 1, rows, cols])
    m = CompiledModel(g, [Ops.ActivationSoftmax(xi, scale)], device)
    g.Dispose()
    (y,) = m.Dispatch([x.Reshape(1, 1, rows, cols)])
    m.Dispose()
    s = x.ToFloats().astype(np.float64) * np.float64(np.float32(scale))
    e = np.exp(s - s.max(-1, keepdims=True))
    want = e / e.sum(-1, keepdims=True)
    got = y.ToFloats().reshape(rows, cols)
    assert y.DataType == dtype
    # relative to each probability, plus float16's subnormal spacing (2^-24)
    # below its smallest normal
    floor = 2.0 ** -24 if dtype == DT.Float16 else 0.0
    assert np.all(np.abs(got - want) <= tol * want + floor)


def decode_case(cfg, seed, h, w, weight_dtype=DT.Float32):
    weights = vae.synthetic_weights(cfg, seed, weight_dtype)
    latent = rng.normal(rng.tensor_seed(seed, "latent"), (1, cfg.latent_channels, h, w)) * np.float32(
        cfg.scaling_factor)
    return weights, latent.astype(np.float32)


def oracle_decode(cfg, weights, latent):
    z = (latent / np.float32(cfg.scaling_factor)).astype(np.float32)
    return oracle.vae_decoder(z, weights, cfg.block_out, cfg.layers_per_block, cfg.groups, cfg.eps)


# Three levels (two upsamplers: 4 pixels a cell) at 64/128/128 wide.
SMALL = vae.VaeConfig(block_out=(64, 128, 128), groups=32, scale_factor=4)


@pytest.mark.parametrize("compute,tol", [(DT.Float32, 1e-3), (DT.BFloat16, 2e-2)])
def test_small_decoder_against_oracle(device, compute, tol):
    cfg = SMALL
    weights, latent = decode_case(cfg, 21, 6, 10, DT.BFloat16)
    say(f"vae decoder (64/128/128) 6x10 latent {compute.name}")
    dec = vae.AutoencoderKlDecoder(device, cfg, weights, 24, 40, compute)
    got = dec.Decode(latent)
    dec.Dispose()
    want = oracle_decode(cfg, weights, latent)
    err = rel_err(got.reshape(want.shape), want)
    say(f"  rel err {err:.2e}")
    assert got.shape == (1, 3, 24, 40) and err <= tol


@pytest.mark.parametrize("compute,tol", [(DT.BFloat16, 2e-2), (DT.Float32, 1e-3)])
def test_sdxl_widths_on_a_small_latent(device, compute, tol):
    cfg = vae.SDXL
    weights, latent = decode_case(cfg, 22, 16, 16, DT.BFloat16)
    say(f"vae decoder at SDXL's widths, 16x16 latent, {compute.name}")
    dec = vae.AutoencoderKlDecoder(device, cfg, weights, 128, 128, compute)
    got = dec.Decode(latent)
    dec.Dispose()
    say("  oracle")
    want = oracle_decode(cfg, weights, latent)
    err = rel_err(got.reshape(want.shape), want)
    say(f"  rel err {err:.2e}")
    assert got.shape == (1, 3, 128, 128) and err <= tol


def test_full_size_decode_properties(device):
    """1024x1024 (a 128x128 latent, 16384-token attention): every pixel
    finite, and the bf16 decode within 5e-2 of the fp32 one."""
    cfg = vae.SDXL
    weights, latent = decode_case(cfg, 23, 128, 128, DT.BFloat16)
    out = {}
    for compute in (DT.BFloat16, DT.Float32):
        say(f"vae decoder 1024x1024 {compute.name}")
        dec = vae.AutoencoderKlDecoder(device, cfg, weights, 1024, 1024, compute)
        out[compute] = dec.Decode(latent)
        dec.Dispose()
        assert out[compute].shape == (1, 3, 1024, 1024)
        assert np.isfinite(out[compute]).all()
    err = rel_err(out[DT.BFloat16], out[DT.Float32])
    say(f"  bf16 vs fp32 {err:.2e}")
    assert err <= 5e-2


# ---- Wan 2.2's single-frame decoder (Qwen-Image 2.1's VAE) ---------------------------------

def wan_case(cfg, seed, h, w, weight_dtype=DT.BFloat16):
    weights = vae.wan22_synthetic_weights(cfg, seed, weight_dtype)
    latent = rng.normal(rng.tensor_seed(seed, "latent"), (1, cfg.latent_channels, h, w))
    return weights, latent.astype(np.float32)


def wan_oracle(cfg, weights, latent):
    """FromModelScale in float32 (latent * deviation + mean, each rounded),
    then the oracle's decoder."""
    lc = cfg.latent_channels
    dev = np.asarray(vae.WAN22_DEVIATIONS[:lc], np.float32)[None, :, None, None]
    mean = np.asarray(vae.WAN22_MEANS[:lc], np.float32)[None, :, None, None]
    z = (latent * dev).astype(np.float32) + mean
    return oracle.wan22_decoder(z.astype(np.float32), weights, vae.WAN22_TEMPORAL)


WAN_SMALL = vae.Wan22Config(latent_channels=16, widths=(128, 128, 64, 32, 32), resnets=3)


@pytest.mark.parametrize("compute,tol", [(DT.Float32, 1e-3), (DT.BFloat16, 2e-2)])
def test_wan22_small_decoder_against_oracle(device, compute, tol):
    """Every level kind: same-width shortcuts, the odd channels of a level
    that doubled time, the row interleave of one that did not."""
    cfg = WAN_SMALL
    weights, latent = wan_case(cfg, 31, 3, 5)
    say(f"wan 2.2 decoder (128..32) 3x5 latent {compute.name}")
    dec = vae.Wan22Decoder(device, cfg, weights, 48, 80, compute)
    got = dec.Decode(latent)
    dec.Dispose()
    want = wan_oracle(cfg, weights, latent)
    err = rel_err(got.reshape(want.shape), want)
    say(f"  rel err {err:.2e}")
    assert got.shape == (1, 3, 48, 80) and err <= tol


@pytest.mark.parametrize("compute,tol", [(DT.BFloat16, 2e-2), (DT.Float32, 1e-3)])
def test_wan22_real_widths_on_a_small_latent(device, compute, tol):
    cfg = vae.WAN22
    weights, latent = wan_case(cfg, 32, 2, 3)
    say(f"wan 2.2 decoder at 1152..144 wide, 2x3 latent, {compute.name}")
    dec = vae.Wan22Decoder(device, cfg, weights, 32, 48, compute)
    got = dec.Decode(latent)
    dec.Dispose()
    say("  oracle")
    want = wan_oracle(cfg, weights, latent)
    err = rel_err(got.reshape(want.shape), want)
    say(f"  rel err {err:.2e}")
    assert got.shape == (1, 3, 32, 48) and err <= tol


def test_wan22_full_size_decode_properties(device):
    """1024x1024 from a 64x64 latent: finite, bf16 within 5e-2 of fp32."""
    cfg = vae.WAN22
    weights, latent = wan_case(cfg, 33, 64, 64)
    out = {}
    for compute in (DT.BFloat16, DT.Float32):
        say(f"wan 2.2 decoder 1024x1024 {compute.name}")
        dec = vae.Wan22Decoder(device, cfg, weights, 1024, 1024, compute)
        out[compute] = dec.Decode(latent)
        dec.Dispose()
        assert out[compute].shape == (1, 3, 1024, 1024)
        assert np.isfinite(out[compute]).all()
    err = rel_err(out[DT.BFloat16], out[DT.Float32])
    say(f"  bf16 vs fp32 {err:.2e}")
    assert err <= 5e-2
