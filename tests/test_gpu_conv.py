"""GPU parity of the convolution (Layers.Conv2d, Graph/Layers.cs:115-127 ->
DmlOps.Convolution, Dml/DmlOps.cs:265-299) against the oracle's direct
cross-correlation: the implicit-GEMM kernel at SDXL's shapes (3x3 pad 1,
the stride-2 downsampler, the 1x1 shortcut with the resnet's residual add)
scaled down in extent, ragged extents that leave partial pixel tiles, every
tile variant pinned, and the direct kernel for what the implicit GEMM does
not take (4 input channels, int8 filters). Input channels that are a
multiple of 8 but not of 64 run with K contiguous over the taps. Tolerance: max|gpu - oracle| /
max|oracle| <= 1e-2 at fp16, 2e-2 at bf16."""

import numpy as np
import pytest

import naivediffusion_amd as nd
import oracle
from naivediffusion_amd import rng
from naivediffusion_amd.layers import Layers
from naivediffusion_amd.tensors import HostDataType as DT, HostTensor
from conftest import rel_err

pytestmark = pytest.mark.gpu

TOL = {DT.Float16: 1e-2, DT.BFloat16: 2e-2}


def normal(name, shape, std=1.0):
    return rng.normal(rng.tensor_seed(11, name), shape, 0.0, std)


def narrow(x, dtype):
    """x rounded to dtype, as fp32 values (what the device holds)."""
    return HostTensor.FromFloats(np.asarray(x, np.float32)).ConvertTo(dtype).ToFloats().reshape(np.shape(x))


def run_conv(device, dtype, x, w, b, stride, pad, residual=None, int8=False):
    model = nd.ModelBuilder(device, dtype, int8Weights=int8)
    xin = model.Placeholder(list(x.shape), dtype)
    rin = model.Placeholder(list(residual.shape), dtype) if residual is not None else None
    y = Layers.Conv2d(model, xin, HostTensor.FromFloats(w), HostTensor.FromFloats(b), stride, pad, residual=rin)
    model.Compile([y])
    model.Compiled.SetProfiling(True)
    inputs = [HostTensor.FromFloats(x).ConvertTo(dtype)]
    if residual is not None:
        inputs.append(HostTensor.FromFloats(residual).ConvertTo(dtype))
    out = model.Run(*inputs)[0].ToFloats()
    families = set(model.Compiled.Profile())
    model.Dispose()
    return out, families


CASES = [
    # (batch, Cin, H, W, Cout, k, stride, pad): SDXL's resnet conv at 320 and
    # 640 channels, the downsampler, the 1x1 shortcut, a 1280-channel
    # output that takes the 256-row tile, and extents that are not multiples
    # of the pixel tile.
    (1, 320, 24, 20, 320, 3, 1, 1),
    (2, 64, 17, 15, 128, 3, 2, 1),
    (1, 128, 16, 16, 64, 1, 1, 0),
    (2, 640, 8, 8, 1280, 3, 1, 1),
    (1, 192, 9, 31, 96, 3, 1, 1),
    # Channel counts that are multiples of 8 but not of 64 (the Wan VAE's
    # 144 and 288, and narrower ones whose taps share a K tile): K runs over
    # the taps with no padding between them.
    (1, 144, 13, 11, 144, 3, 1, 1),
    (2, 288, 7, 9, 144, 1, 1, 0),
    (1, 288, 10, 6, 576, 3, 2, 1),
    (1, 16, 9, 11, 64, 3, 1, 1),
    (2, 40, 8, 6, 96, 3, 2, 1),
    (1, 8, 12, 12, 32, 3, 1, 1),
]


@pytest.mark.parametrize("B,Cin,H,W,Cout,k,stride,pad", CASES)
@pytest.mark.parametrize("dtype", [DT.Float16, DT.BFloat16])
def test_conv_implicit_gemm(device, B, Cin, H, W, Cout, k, stride, pad, dtype):
    print(f"[gpu] conv {B}x{Cin}x{H}x{W} -> {Cout} k{k} s{stride} p{pad} {dtype.name}", flush=True)
    x = narrow(normal("x", (B, Cin, H, W)), dtype)
    w = narrow(normal("w", (Cout, Cin, k, k), 1.0 / np.sqrt(Cin * k * k)), dtype)
    b = narrow(normal("b", (Cout,), 0.1), dtype)
    out, families = run_conv(device, dtype, x, w, b, stride, pad)
    ref = oracle.conv2d(x, w, b, stride, pad)
    assert out.shape == ref.shape
    assert any(f.startswith("conv_mfma_") for f in families), families
    assert "nchw_to_nhwc" in families, families
    err = rel_err(out, ref)
    print(f"[gpu]   rel err {err:.2e} via {sorted(families)}", flush=True)
    assert err <= TOL[dtype]


def test_conv_residual_is_fused(device):
    """The resnet's x + h rides the convolution's epilogue: conv(x) + r
    rounded once at fp16, as Cast(h) + r."""
    dtype = DT.Float16
    x = narrow(normal("rx", (2, 128, 12, 10)), dtype)
    w = narrow(normal("rw", (64, 128, 3, 3), 1.0 / np.sqrt(128 * 9)), dtype)
    b = narrow(normal("rb", (64,), 0.1), dtype)
    r = narrow(normal("rr", (2, 64, 12, 10)), dtype)
    out, families = run_conv(device, dtype, x, w, b, 1, 1, residual=r)
    assert rel_err(out, oracle.conv2d(x, w, b, 1, 1) + r) <= TOL[dtype]
    assert any(f.startswith("conv_mfma_") for f in families), families


def run_graph(device, dtype, build, *arrays):
    model = nd.ModelBuilder(device, dtype)
    ins = [model.Placeholder(list(a.shape), dtype) for a in arrays]
    model.Compile([build(model, *ins)])
    model.Compiled.SetProfiling(True)
    out = model.Run(*[HostTensor.FromFloats(a).ConvertTo(dtype) for a in arrays])[0].ToFloats()
    families = set(model.Compiled.Profile())
    model.Dispose()
    return out, families


@pytest.mark.parametrize("B,C,H,W,Cout", [(1, 128, 12, 10, 64), (2, 144, 9, 7, 96), (1, 288, 6, 11, 288)])
def test_conv_reads_token_rows_in_place(device, B, C, H, W, Cout):
    """A convolution of ToImage(tokens) (an NHWC image: what a norm over
    channels leaves) reads the token rows as they lie, with no transposed
    copy; 144 and 288 channels have their last K slab part zeros."""
    dtype = DT.BFloat16
    print(f"[gpu] conv of token rows {B}x{H * W}x{C} -> {Cout}", flush=True)
    t = narrow(normal("tr_t", (B, 1, H * W, C)), dtype)
    w = narrow(normal("tr_w", (Cout, C, 3, 3), 1.0 / np.sqrt(C * 9)), dtype)
    b = narrow(normal("tr_b", (Cout,), 0.1), dtype)
    out, families = run_graph(device, dtype, lambda m, ti: Layers.Conv2d(
        m, Layers.ToImage(ti, H, W), HostTensor.FromFloats(w), HostTensor.FromFloats(b), 1, 1), t)
    x = np.ascontiguousarray(t.reshape(B, H, W, C).transpose(0, 3, 1, 2))
    err = rel_err(out, oracle.conv2d(x, w, b, 1, 1))
    print(f"[gpu]   rel err {err:.2e} via {sorted(families)}", flush=True)
    assert err <= TOL[dtype]
    assert any(f.startswith("conv_mfma_") for f in families), families
    assert "nchw_to_nhwc" not in families and "elementwise" not in families, families


@pytest.mark.parametrize("B,C,H,W,Cout,k,stride,pad", [
    (1, 128, 7, 5, 64, 3, 1, 1), (2, 144, 6, 9, 144, 3, 1, 1), (1, 64, 8, 8, 128, 1, 1, 0),
    (1, 64, 5, 6, 64, 3, 2, 1)])
def test_conv_reads_through_a_fused_upsample(device, B, C, H, W, Cout, k, stride, pad):
    """Conv2d(UpsampleNearest(x)) (the decoders' upsamplers) never writes
    the upsampled image: the convolution reads pixel (y, x) of it from
    (y / 2, x / 2) of its source."""
    dtype = DT.BFloat16
    print(f"[gpu] conv through upsample {B}x{C}x{H}x{W} -> {Cout} k{k} s{stride}", flush=True)
    x = narrow(normal("up_x", (B, C, H, W)), dtype)
    w = narrow(normal("up_w", (Cout, C, k, k), 1.0 / np.sqrt(C * k * k)), dtype)
    b = narrow(normal("up_b", (Cout,), 0.1), dtype)
    out, families = run_graph(device, dtype, lambda m, xi: Layers.Conv2d(
        m, Layers.UpsampleNearest(xi), HostTensor.FromFloats(w), HostTensor.FromFloats(b), stride, pad), x)
    up = np.repeat(np.repeat(x, 2, 2), 2, 3)
    err = rel_err(out, oracle.conv2d(up, w, b, stride, pad))
    print(f"[gpu]   rel err {err:.2e} via {sorted(families)}", flush=True)
    assert err <= TOL[dtype]
    assert "upsample" not in families and any(f.startswith("conv_mfma_") for f in families), families


@pytest.mark.parametrize("tile", ["256", "128", "64x128", "64x64"])
def test_conv_every_tile(device, monkeypatch, tile):
    print(f"[gpu] pinned conv tile {tile}", flush=True)
    monkeypatch.setenv("NDX_CONV_TILE", tile)
    dtype = DT.Float16
    x = narrow(normal("tx", (2, 128, 13, 11)), dtype)
    w = narrow(normal("tw", (300, 128, 3, 3), 1.0 / np.sqrt(128 * 9)), dtype)
    b = narrow(normal("tb", (300,), 0.1), dtype)
    out, families = run_conv(device, dtype, x, w, b, 1, 1)
    want = {"256": "conv_mfma_256x256w8", "128": "conv_mfma_128x128", "64x128": "conv_mfma_64x128",
            "64x64": "conv_mfma_64x64"}[tile]
    assert want in families, families
    assert rel_err(out, oracle.conv2d(x, w, b, 1, 1)) <= TOL[dtype]


@pytest.mark.parametrize("case", ["conv_in", "int8"])
def test_conv_direct_path(device, case):
    """SDXL's conv_in (4 latent channels) and int8 filters stay on the direct kernel."""
    dtype = DT.Float16
    cin = 4 if case == "conv_in" else 64
    x = narrow(normal("dx", (2, cin, 16, 12)), dtype)
    w = narrow(normal("dw", (320 if case == "conv_in" else 128, cin, 3, 3), 1.0 / np.sqrt(cin * 9)), dtype)
    b = narrow(normal("db", (w.shape[0],), 0.1), dtype)
    out, families = run_conv(device, dtype, x, w, b, 1, 1, int8=case == "int8")
    wq = w
    if case == "int8":
        rows = w.shape[0]
        q, sc = oracle.quantize(w.reshape(rows, -1), rows)
        wq = (q.astype(np.float32).reshape(rows, -1, 32) * oracle.f16_bits_to_f32(sc)[:, :, None]).reshape(w.shape)
    assert not any(f.startswith("conv_mfma_") for f in families), families
    assert rel_err(out, oracle.conv2d(x, wq, b, 1, 1)) <= TOL[dtype]


@pytest.mark.parametrize("dtype,B,C,H,W,Cout", [(DT.BFloat16, 1, 128, 16, 16, 128), (DT.Float16, 2, 320, 8, 16, 64),
                                                (DT.Float16, 2, 640, 8, 12, 96)])
def test_group_norm_writes_the_convolutions_nhwc_input(device, monkeypatch, dtype, B, C, H, W, Cout):
    """GroupNorm(32) + SiLU read by a convolution alone writes the NHWC image
    the implicit GEMM reads (no transposed copy; 64-pixel tiles up to 512
    channels, 32-pixel ones above, taken with NDX_GN_NHWC_WIDE=1): bit for
    bit what the NCHW norm and the
    copy give (NDX_FUSE_GN_NHWC=0), and within the tolerance of the oracle's
    group norm and convolution (UNetLayers.cs:14-47, Graph/Layers.cs:166-185)."""
    print(f"[gpu] group norm into conv {dtype.name} {B}x{C}x{H}x{W} -> {Cout}", flush=True)
    if C > 512:
        monkeypatch.setenv("NDX_GN_NHWC_WIDE", "1")
    x = narrow(normal("gnc_x", (B, C, H, W)), dtype)
    gw = narrow(normal("gnc_gw", (C,), 0.2) + 1.0, dtype)
    gb = narrow(normal("gnc_gb", (C,), 0.2), dtype)
    w = narrow(normal("gnc_w", (Cout, C, 3, 3), 1.0 / np.sqrt(C * 9)), dtype)
    b = narrow(normal("gnc_b", (Cout,), 0.1), dtype)

    def build(m, xi):
        h = Layers.GroupNorm(m, xi, HostTensor.FromFloats(gw), HostTensor.FromFloats(gb), 32, 1e-5, silu=True)
        return Layers.Conv2d(m, h, HostTensor.FromFloats(w), HostTensor.FromFloats(b), 1, 1)

    fused, families = run_graph(device, dtype, build, x)
    assert "nchw_to_nhwc" not in families, families
    monkeypatch.setenv("NDX_FUSE_GN_NHWC", "0")
    plain, plain_families = run_graph(device, dtype, build, x)
    assert "nchw_to_nhwc" in plain_families, plain_families
    assert np.array_equal(fused, plain)
    h = narrow(oracle.group_norm(x, 32, gw, gb, 1e-5, silu=True), dtype)
    err = rel_err(fused, oracle.conv2d(h, w, b, 1, 1))
    print(f"[gpu]   rel err {err:.2e}", flush=True)
    assert err <= TOL[dtype]
