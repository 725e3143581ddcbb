"""GPU parity of each kernel family against the oracle, through the C ABI
(ModelBuilder -> ndx_graph_* -> libndx.so): the linear layer's GEMMs at the
MMDiT block's shapes and at ragged ones, int8 weights, attention with its
masks and segmented (joined) operands, the norm kernels, and the smoke
cases of the reference (Cli/SmokeTest.cs). Tolerances: max|gpu - oracle| /
max|oracle| <= 2e-2 at bf16/f16 compute and 1e-3 at fp32 (the measure of
QuantProbe.cs:50-57); integer work bit-exact."""

import math

import numpy as np
import pytest

import naivediffusion_amd as nd
import oracle
from naivediffusion_amd import rng
from naivediffusion_amd.graph import Ops
from naivediffusion_amd.layers import Layers, Transformer
from naivediffusion_amd.tensors import HostDataType as DT, HostTensor, bf16_to_f32, f32_to_bf16
from conftest import rel_err

pytestmark = pytest.mark.gpu

BF16_TOL, F32_TOL = 2e-2, 1e-3


def bf(x):
    """x rounded to bf16, as fp32 values."""
    return bf16_to_f32(f32_to_bf16(np.asarray(x, np.float32)))


def normal(name, shape, std=1.0):
    return rng.normal(rng.tensor_seed(7, name), shape, 0.0, std)


def run(model, *inputs):
    return [t.ToFloats() for t in model.Run(*inputs)]


# ---- linear ------------------------------------------------------------------------

LINEAR_CASES = [
    # (M, K, N, batch): the MMDiT block at 1024 + 128 tokens, the text stream,
    # the adaLN GEMV, and ragged shapes that leave partial tiles everywhere.
    (1024, 3072, 3072, 1),
    (1024, 3072, 12288, 1),
    (1024, 12288, 3072, 1),
    (128, 3072, 9216, 1),
    (1, 3072, 18432, 1),
    (2, 256, 3072, 1),
    (1000, 320, 257, 1),
    (77, 64, 96, 2),
    (5376 // 8, 64, 3072, 1),
]


@pytest.mark.parametrize("M,K,N,B", LINEAR_CASES)
@pytest.mark.parametrize("compute", [DT.BFloat16, DT.Float32])
def test_linear_against_oracle(device, M, K, N, B, compute):
    print(f"[gpu] linear M={M} K={K} N={N} B={B} {compute.name}", flush=True)
    x = bf(normal("x", (B, 1, M, K)))
    w = bf(normal("w", (N, K), 0.02))
    b = bf(normal("b", (N,), 0.02))
    model = nd.ModelBuilder(device, compute)
    xin = model.Placeholder([B, 1, M, K], compute)
    y = Layers.Linear(model, xin, HostTensor.FromFloats(w), HostTensor.FromFloats(b))
    model.Compile([y])
    out = run(model, HostTensor.FromFloats(x).ConvertTo(compute))[0]
    ref = oracle.linear(x, w, b)
    assert out.shape == ref.shape
    err = rel_err(out, ref)
    print(f"[gpu]   rel err {err:.2e}", flush=True)
    assert err <= (BF16_TOL if compute == DT.BFloat16 else F32_TOL)


# Shapes that reach every tile configuration of the GEMM dispatch; the
# family each one runs is checked to be an MFMA tile (or the GEMV) and the
# set of families over the cases to cover all of them.
TILE_CASES = [
    (64, 3072, 3072, 1), (40, 1024, 650, 1), (64, 512, 384, 3), (256, 3072, 9216, 1), (128, 3072, 9216, 1),
    (1536, 12288, 3072, 1), (1543, 1024, 8200, 1), (1024, 3072, 12288, 1), (1543, 1024, 10000, 1),
    (2048, 1024, 4096, 1), (3, 3072, 1000, 2),
]
SEEN_FAMILIES = set()


@pytest.mark.parametrize("M,K,N,B", TILE_CASES)
@pytest.mark.parametrize("int8", [False, True])
def test_linear_tile_configurations(device, M, K, N, B, int8):
    print(f"[gpu] tile case M={M} K={K} N={N} B={B} int8={int8}", flush=True)
    x = bf(normal("tx", (B, 1, M, K)))
    w = bf(normal("tw", (N, K), 0.02))
    b = bf(normal("tb", (N,), 0.02))
    model = nd.ModelBuilder(device, DT.BFloat16, int8Weights=int8)
    xin = model.Placeholder([B, 1, M, K])
    model.Compile([Layers.Linear(model, xin, HostTensor.FromFloats(w), HostTensor.FromFloats(b))])
    model.Compiled.SetProfiling(True)
    out = run(model, HostTensor.FromFloats(x).ConvertTo(DT.BFloat16))[0]
    (family,) = set(model.Compiled.Profile())
    SEEN_FAMILIES.add(family.replace("_w8_", "_").replace("_lds", "").removesuffix("w8"))
    wq = w
    if int8 and w.size >= (1 << 16):
        q, sc = oracle.quantize(w, N)
        wq = (q.astype(np.float32).reshape(N, -1, 32) * oracle.f16_bits_to_f32(sc)[:, :, None]).reshape(N, K)
        assert family == "gemv" or "_w8_" in family, family
    assert family == "gemv" or family.startswith("gemm_"), family
    assert rel_err(out, oracle.linear(x, wq, b)) <= BF16_TOL


def test_tile_cases_reached_every_configuration():
    assert SEEN_FAMILIES >= {"gemm_mfma_256x256", "gemm_mfma_128x128", "gemm_mfma_64x128", "gemm_mfma_64x64",
                             "gemv"}, SEEN_FAMILIES


@pytest.mark.parametrize("tile", ["256", "128", "64x128", "64x64", "256lds", "128lds", "64x128lds", "64x64lds",
                                  "256w8lds", "128w8lds"])
@pytest.mark.parametrize("M,K,N", [(600, 1024, 1000), (1024, 3072, 3072), (77, 320, 2056)])
def test_linear_every_kernel_variant(device, monkeypatch, tile, M, K, N):
    """Each GEMM kernel, pinned through NDX_GEMM_TILE, against the oracle on
    ragged shapes (partial tiles in M, N and K)."""
    print(f"[gpu] pinned tile {tile} M={M} K={K} N={N}", flush=True)
    monkeypatch.setenv("NDX_GEMM_TILE", tile)
    x = bf(normal("vx", (1, 1, M, K)))
    w = bf(normal("vw", (N, K), 0.02))
    b = bf(normal("vb", (N,), 0.02))
    model = nd.ModelBuilder(device, DT.BFloat16)
    xin = model.Placeholder([1, 1, M, K])
    model.Compile([Layers.Linear(model, xin, HostTensor.FromFloats(w), HostTensor.FromFloats(b), activation="gelu_tanh")])
    model.Compiled.SetProfiling(True)
    out = run(model, HostTensor.FromFloats(x).ConvertTo(DT.BFloat16))[0]
    (family,) = set(model.Compiled.Profile())
    assert family.endswith({"256": "mfma_256x256", "128": "mfma_128x128", "64x128": "mfma_64x128",
                            "64x64": "mfma_64x64", "256lds": "lds_256x256", "128lds": "lds_128x128",
                            "64x128lds": "lds_64x128", "64x64lds": "lds_64x64", "256w8lds": "lds_256x256w8",
                            "128w8lds": "lds_128x128w8"}[tile]), family
    assert rel_err(out, oracle.gelu_tanh(oracle.linear(x, w, b))) <= BF16_TOL


@pytest.mark.parametrize("epi", ["gelu_tanh", "gated", "none"])
@pytest.mark.parametrize("M,K,N", [(600, 1024, 1024), (1024, 3072, 3072), (77, 320, 2048)])
def test_linear_register_capped_tile(device, monkeypatch, epi, M, K, N):
    """The 64 x 64 tile capped at 64 registers (the second stream's, so it
    fits beside a 256 x 256 workgroup), pinned through NDX_GEMM_TILE=slim,
    against the oracle: ragged M, whole K tiles, the fast epilogue's
    activation, gated fp32 residual and plain forms."""
    print(f"[gpu] register-capped tile {epi} M={M} K={K} N={N}", flush=True)
    monkeypatch.setenv("NDX_GEMM_TILE", "slim")
    x = bf(normal("sx", (1, 1, M, K)))
    w = bf(normal("sw", (N, K), 0.02))
    b = bf(normal("sb", (N,), 0.02))
    res = normal("sr", (1, 1, M, N))
    gate = normal("sg", (1, 1, 1, N))
    model = nd.ModelBuilder(device, DT.BFloat16)
    xin = model.Placeholder([1, 1, M, K])
    rin = model.Placeholder([1, 1, M, N], DT.Float32)
    gin = model.Placeholder([1, 1, 1, N], DT.Float32)
    kw = {"gelu_tanh": {"activation": "gelu_tanh"}, "gated": {"gate": gin, "residual": rin}, "none": {}}[epi]
    model.Compile([Layers.Linear(model, xin, HostTensor.FromFloats(w), HostTensor.FromFloats(b), **kw)])
    model.Compiled.SetProfiling(True)
    out = run(model, HostTensor.FromFloats(x).ConvertTo(DT.BFloat16), HostTensor.FromFloats(res),
              HostTensor.FromFloats(gate))[0]
    (family,) = set(model.Compiled.Profile())
    model.Dispose()
    assert family == "gemm_mfma_lds_64x64_slim", family
    p = oracle.linear(x, w, b)
    ref = {"gelu_tanh": lambda: oracle.gelu_tanh(p), "gated": lambda: res + gate * p, "none": lambda: p}[epi]()
    assert rel_err(out, ref) <= BF16_TOL


@pytest.mark.parametrize("epi", ["gelu_tanh", "gelu", "silu", "gated", "residual"])
def test_linear_epilogues(device, epi):
    M, K, N = 300, 512, 384
    x = bf(normal("ex", (1, 1, M, K)))
    w = bf(normal("ew", (N, K), 0.05))
    b = bf(normal("eb", (N,), 0.05))
    res = normal("er", (1, 1, M, N))
    gate = normal("eg", (1, 1, 1, N))
    model = nd.ModelBuilder(device, DT.BFloat16)
    xin = model.Placeholder([1, 1, M, K])
    rin = model.Placeholder([1, 1, M, N], DT.Float32)
    gin = model.Placeholder([1, 1, 1, N], DT.Float32)
    kw = {}
    if epi in ("gelu_tanh", "gelu", "silu"):
        kw["activation"] = epi
    elif epi == "gated":
        kw.update(gate=gin, residual=rin)
    else:
        kw.update(residual=rin)
    y = Layers.Linear(model, xin, HostTensor.FromFloats(w), HostTensor.FromFloats(b), **kw)
    model.Compile([y])
    out = run(model, HostTensor.FromFloats(x).ConvertTo(DT.BFloat16), HostTensor.FromFloats(res),
              HostTensor.FromFloats(gate))[0]
    p = oracle.linear(x, w, b)
    ref = {"gelu_tanh": lambda: oracle.gelu_tanh(p), "gelu": lambda: oracle.gelu(p), "silu": lambda: oracle.silu(p),
           "gated": lambda: res + gate * p, "residual": lambda: res + p}[epi]()
    assert rel_err(out, ref) <= BF16_TOL


@pytest.mark.parametrize("compute", [DT.BFloat16, DT.Float32])
@pytest.mark.parametrize("M", [1, 256, 1024])
def test_int8_linear_against_oracle(device, compute, M):
    """ModelBuilder.Weight under int8 (Graph/ModelBuilder.cs:65-88): the GEMM
    matches the oracle's product with the dequantised weights, and stays
    within the bf16 bound of the unquantised product."""
    print(f"[gpu] int8 linear M={M} {compute.name}", flush=True)
    K, N = 3072, 3072
    x = bf(normal("qx", (1, 1, M, K)))
    w = bf(normal("qw", (N, K), 0.02))
    model = nd.ModelBuilder(device, compute, int8Weights=True)
    xin = model.Placeholder([1, 1, M, K], compute)
    model.Compile([Layers.Linear(model, xin, HostTensor.FromFloats(w))])
    out = run(model, HostTensor.FromFloats(x).ConvertTo(compute))[0]
    q, s = oracle.quantize(w, N)
    deq = (q.astype(np.float32).reshape(N, K // 32, 32) *
           oracle.f16_bits_to_f32(s)[:, :, None]).reshape(N, K)
    assert rel_err(out, oracle.linear(x, deq)) <= (BF16_TOL if compute == DT.BFloat16 else F32_TOL)
    assert rel_err(out, oracle.linear(x, w)) <= BF16_TOL


@pytest.mark.parametrize("tile", ["auto", "256w8lds", "128lds", "64x128lds", "64x64lds", "256"])
@pytest.mark.parametrize("fmt", ["block32", "channel"])
@pytest.mark.parametrize("K", [1024, 1056])
def test_int8_kernels_every_tile(device, monkeypatch, tile, fmt, K):
    """The int8 GEMMs (direct-to-LDS with the pipelined dequant, and the
    register-staged one pinned as "256") on ragged shapes, K a whole number
    of 64-wide tiles or ending in half of one, with the reference's block-32
    fp16 scales and with per-output-channel fp32 scales (Device.QuantizeInt8
    + ModelBuilder.WeightInt8)."""
    print(f"[gpu] int8 {fmt} tile {tile} K={K}", flush=True)
    if tile != "auto":
        monkeypatch.setenv("NDX_GEMM_TILE", tile)
    M, N = 700, 1000
    x = bf(normal("ix", (1, 1, M, K)))
    w = bf(normal("iw", (N, K), 0.02))
    b = bf(normal("ib", (N,), 0.02))
    if fmt == "block32":
        model = nd.ModelBuilder(device, DT.BFloat16, int8Weights=True)
        wv = HostTensor.FromFloats(w)
        q, sc = oracle.quantize(w, N)
        deq = (q.astype(np.float32).reshape(N, K // 32, 32) * oracle.f16_bits_to_f32(sc)[:, :, None]).reshape(N, K)
    else:
        model = nd.ModelBuilder(device, DT.BFloat16)
        wt = device.Upload(HostTensor.FromFloats(w).ConvertTo(DT.BFloat16))
        qd, sd = device.QuantizeInt8(wt, K, DT.Float32)
        q, sc = oracle.quantize(w, N, K, fp16_scales=False)
        # The device quantiser is bit-exact with the oracle in this format too.
        assert np.array_equal(qd.Download().Data, q) and np.array_equal(sd.Download().Data.ravel(), sc.ravel())
        wv = model.WeightInt8(qd, sd, K)
        deq = q.astype(np.float32) * np.asarray(sc, np.float32).reshape(N, 1)
    xin = model.Placeholder([1, 1, M, K])
    model.Compile([Layers.Linear(model, xin, wv, HostTensor.FromFloats(b), activation="gelu_tanh")])
    model.Compiled.SetProfiling(True)
    out = run(model, HostTensor.FromFloats(x).ConvertTo(DT.BFloat16))[0]
    (family,) = set(model.Compiled.Profile())
    assert "_w8_" in family, family
    if tile not in ("auto", "256"):
        assert "w8_lds" in family, family
    assert rel_err(out, oracle.gelu_tanh(oracle.linear(x, deq, b))) <= BF16_TOL


def test_device_quantizer_is_bit_exact_with_the_oracle(device):
    w = bf(normal("dq", (640, 3072), 0.02))
    wt = device.Upload(HostTensor.FromFloats(w).ConvertTo(DT.BFloat16))
    q = device.Empty(DT.Int8, [640, 3072])
    s = device.Empty(DT.Float16, [640, 96])
    nd._lib.call("ndx_quantize_block_int8_device", wt.handle, 32, int(DT.Float16), q.handle, s.handle)
    oq, os_ = oracle.quantize(w, 640)
    assert np.array_equal(q.Download().Data, oq)
    assert np.array_equal(s.Download().Data.view(np.uint16), os_)


# ---- attention -----------------------------------------------------------------------

@pytest.mark.parametrize("T,S,H,d,dtype", [
    (1152, 1152, 24, 128, DT.BFloat16),
    (300, 77, 10, 64, DT.Float16),
    (130, 517, 4, 128, DT.BFloat16),
    (257, 257, 2, 128, DT.Float32),
    (64, 100, 3, 64, DT.Float32),
    (1500, 1433, 3, 128, DT.Float32),
    (129, 4096, 2, 64, DT.Float32),
])
def test_attention_against_oracle(device, T, S, H, d, dtype):
    print(f"[gpu] attention T={T} S={S} H={H} d={d} {dtype.name}", flush=True)
    q = bf(normal("aq", (1, T, H * d)))
    k = bf(normal("ak", (1, S, H * d)))
    v = bf(normal("av", (1, S, H * d)))
    model = nd.ModelBuilder(device, dtype)
    ins = [model.Placeholder([1, 1, n, H * d]) for n in (T, S, S)]
    model.Compile([Layers.Attend(*ins, H)])
    out = run(model, *[HostTensor.FromFloats(a.reshape(1, 1, -1, H * d)).ConvertTo(dtype) for a in (q, k, v)])[0]
    ref = oracle.mha(q, k, v, H)
    err = rel_err(out.reshape(ref.shape), ref)
    print(f"[gpu]   rel err {err:.2e}", flush=True)
    assert err <= (F32_TOL if dtype == DT.Float32 else BF16_TOL)


@pytest.mark.parametrize("dtype", [DT.BFloat16, DT.Float32])
def test_attention_masks(device, dtype):
    """Key-length and boolean masks with DirectML's -10000 (DmlOps.cs:483);
    the causal table of QwenImageConditioner.cs:69-80 broadcast over heads."""
    T, H, d = 200, 2, 128
    q, k, v = (bf(normal(n, (1, T, H * d))) for n in ("mq", "mk", "mv"))
    table = oracle.causal_table(150, T).reshape(1, 1, T, T)
    model = nd.ModelBuilder(device, dtype)
    ins = [model.Placeholder([1, 1, T, H * d]) for _ in range(3)]
    kl = model.Placeholder([1, 1, 1, 1], DT.Int32)
    tb = model.Placeholder([1, 1, T, T], DT.Int32)
    a1 = Layers.Attend(*ins, H, kl, nd.MaskType.KeySequenceLength)
    a2 = Layers.Attend(*ins, H, Layers.Broadcast(tb, [1, H, T, T]), nd.MaskType.Boolean)
    model.Compile([a1, a2])
    host = [HostTensor.FromFloats(a.reshape(1, 1, T, H * d)).ConvertTo(dtype) for a in (q, k, v)]
    o1, o2 = run(model, *host, HostTensor.FromInt32(np.array([137]), 1, 1, 1, 1), HostTensor.FromInt32(table))
    tol = F32_TOL if dtype == DT.Float32 else BF16_TOL
    assert rel_err(o1.reshape(1, T, -1), oracle.mha(q, k, v, H, mask_kind=1, key_len=137)) <= tol
    assert rel_err(o2.reshape(1, T, -1), oracle.mha(q, k, v, H, mask_kind=2, mask=table)) <= tol


@pytest.mark.parametrize("dtype", [DT.BFloat16, DT.Float32])
def test_attention_reads_joined_streams_in_place(device, dtype):
    """A join of the image and text rows feeding the attention is read as
    two row segments; the result equals attention over the packed join.
    Scores spread wide (x3) so the running max moves across key tiles."""
    ni, nt, H, d = 300, 45, 4, 128
    parts = {n: bf(normal(n, (1, 1, r, H * d), 3.0 if n[0] == "q" else 1.0)) for n, r in
             (("qi", ni), ("qt", nt), ("ki", ni), ("kt", nt), ("vi", ni), ("vt", nt))}
    model = nd.ModelBuilder(device, dtype)
    ph = {n: model.Placeholder(list(a.shape)) for n, a in parts.items()}
    j = [Ops.Join([ph[a], ph[b]], 2) for a, b in (("qi", "qt"), ("ki", "kt"), ("vi", "vt"))]
    model.Compile([Layers.Attend(*j, H)])
    out = run(model, *[HostTensor.FromFloats(a).ConvertTo(dtype) for a in parts.values()])[0]
    cat = [np.concatenate([parts[a], parts[b]], 2).reshape(1, ni + nt, H * d)
           for a, b in (("qi", "qt"), ("ki", "kt"), ("vi", "vt"))]
    err = rel_err(out.reshape(1, ni + nt, -1), oracle.mha(*cat, H))
    print(f"[gpu]   joined attention {dtype.name} rel err {err:.2e}", flush=True)
    assert err <= (F32_TOL if dtype == DT.Float32 else BF16_TOL)


# ---- norms ------------------------------------------------------------------------------

@pytest.mark.parametrize("out_dtype", [DT.BFloat16, DT.Float32])
def test_modulate_against_oracle(device, out_dtype):
    rows, D = 1000, 3072
    x = normal("mx", (1, 1, rows, D)) * 3 + 1
    shift, scale = normal("ms", (1, 1, 1, D), 0.5), normal("mc", (1, 1, 1, D), 0.5)
    model = nd.ModelBuilder(device, DT.BFloat16)
    xi = model.Placeholder([1, 1, rows, D], DT.Float32)
    si = model.Placeholder([1, 1, 1, D], DT.Float32)
    ci = model.Placeholder([1, 1, 1, D], DT.Float32)
    model.Compile([Transformer.Modulate(xi, si, ci, 1e-6, out_dtype)])
    out = run(model, *map(HostTensor.FromFloats, (x, shift, scale)))[0]
    ref = oracle.modulate(x.reshape(rows, D), shift.ravel(), scale.ravel(), 1e-6)
    assert rel_err(out.reshape(rows, D), ref) <= (BF16_TOL / 4 if out_dtype == DT.BFloat16 else 1e-5)


@pytest.mark.parametrize("D", [64, 640, 3072, 4096, 10240])
def test_layer_and_rms_norm(device, D):
    rows = 37
    x = normal("nx", (1, 1, rows, D)) * 2 + 0.5
    w, b = normal("nw", (D,), 0.3) + 1, normal("nb", (D,), 0.3)
    model = nd.ModelBuilder(device, DT.Float32)
    xi = model.Placeholder([1, 1, rows, D])
    ln = Layers.LayerNorm(model, xi, HostTensor.FromFloats(w), HostTensor.FromFloats(b), 1e-5)
    rms = Layers.RmsNorm(model, xi, HostTensor.FromFloats(w), 1e-6)
    model.Compile([ln, rms])
    o1, o2 = run(model, HostTensor.FromFloats(x))
    assert rel_err(o1.reshape(rows, D), oracle.layer_norm(x.reshape(rows, D), w, b, 1e-5)) <= 1e-5
    assert rel_err(o2.reshape(rows, D), oracle.rms_norm(x.reshape(rows, D), w, 1e-6)) <= 1e-5


@pytest.mark.parametrize("dtype", [DT.BFloat16, DT.Float32])
def test_head_norm_rotate_against_oracle(device, dtype):
    T, H, d = 333, 24, 128
    x = bf(normal("hx", (1, 1, T, H * d)) * 2)
    w = bf(normal("hw", (d,), 0.2) + 1)
    cos, sin = oracle.mmdit_rope_tables(9, 37, 0)
    model = nd.ModelBuilder(device, dtype)
    xi = model.Placeholder([1, 1, T, H * d])
    ci = model.Placeholder([1, T, 1, 64], DT.Float32)
    si = model.Placeholder([1, T, 1, 64], DT.Float32)
    y = Transformer.HeadNormRotate(model, xi, HostTensor.FromFloats(w), H, 1e-6, ci, si, dtype)
    # the reference's unfused composition of the same two steps
    z = Transformer.Flat(Transformer.Rotate(Transformer.HeadNorm(model, xi, HostTensor.FromFloats(w), H, d, 1e-6),
                                            ci, si, H, d, dtype), H * d)
    model.Compile([y, z])
    o1, o2 = run(model, HostTensor.FromFloats(x).ConvertTo(dtype), HostTensor.FromFloats(cos.reshape(1, T, 1, 64)),
                 HostTensor.FromFloats(sin.reshape(1, T, 1, 64)))
    ref = oracle.rope(oracle.rms_norm(x.reshape(T * H, d), w, 1e-6).reshape(T, H * d), H, cos, sin)
    tol = BF16_TOL if dtype == DT.BFloat16 else F32_TOL
    assert rel_err(o1.reshape(T, -1), ref) <= tol
    assert rel_err(o2.reshape(T, -1), ref) <= tol


@pytest.mark.parametrize("tile,fused", [("256w8lds", True), ("128lds", True), ("64x128lds", True), ("64x64lds", False)])
def test_qkv_projection_with_fused_head_norm(device, monkeypatch, tile, fused):
    """With NDX_FUSE_QK_NORM=1, Rotate(HeadNorm(...)) of a QKV projection's
    q and k thirds (QwenImageDit.cs:342-347) runs in the projection's
    epilogue on the tiles whose waves hold half a head (no head-norm kernel
    runs), and stays a pass of its own on a tile whose waves do not; 300
    rows leave a partial tile.
    Both against the oracle: the product rounded to bf16, the RMS norm over
    each head of 128 with the weight, the rotation; v is the rounded
    product's last third."""
    print(f"[gpu] fused qkv head norm, tile {tile}", flush=True)
    monkeypatch.setenv("NDX_GEMM_TILE", tile)
    monkeypatch.setenv("NDX_FUSE_QK_NORM", "1")
    T, Dm, H, d = 300, 256, 4, 128
    D = H * d
    x = bf(normal("fq_x", (1, 1, T, Dm)))
    w = bf(normal("fq_w", (3 * D, Dm), 1.0 / math.sqrt(Dm)))
    b = bf(normal("fq_b", (3 * D,), 0.1))
    wq, wk = bf(normal("fq_q", (d,), 0.2) + 1), bf(normal("fq_k", (d,), 0.2) + 1)
    cos, sin = oracle.mmdit_rope_tables(10, 30, 0)
    dt = DT.BFloat16
    model = nd.ModelBuilder(device, dt)
    xi = model.Placeholder([1, 1, T, Dm], dt)
    ci = model.Placeholder([1, T, 1, 64], DT.Float32)
    si = model.Placeholder([1, T, 1, 64], DT.Float32)
    qkv = Layers.Linear(model, xi, HostTensor.FromFloats(w), HostTensor.FromFloats(b))
    q = Transformer.HeadNormRotate(model, Ops.Slice(qkv, [0, 0, 0, 0], [1, 1, T, D]), HostTensor.FromFloats(wq), H,
                                   1e-6, ci, si, dt)
    k = Transformer.HeadNormRotate(model, Ops.Slice(qkv, [0, 0, 0, D], [1, 1, T, D]), HostTensor.FromFloats(wk), H,
                                   1e-6, ci, si, dt)
    v = Ops.ActivationIdentity(Ops.Slice(qkv, [0, 0, 0, 2 * D], [1, 1, T, D]))
    model.Compile([q, k, v])
    model.Compiled.SetProfiling(True)
    oq, ok_, ov = run(model, HostTensor.FromFloats(x).ConvertTo(dt), HostTensor.FromFloats(cos.reshape(1, T, 1, 64)),
                      HostTensor.FromFloats(sin.reshape(1, T, 1, 64)))
    families = set(model.Compiled.Profile())
    model.Dispose()
    p = bf(oracle.linear(x.reshape(T, Dm), w, b))
    want = [oracle.rope(oracle.rms_norm(p[:, i * D:(i + 1) * D].reshape(T * H, d), wn, 1e-6).reshape(T, D), H, cos,
                        sin) for i, wn in ((0, wq), (1, wk))]
    for got, ref in zip((oq, ok_), want):
        err = rel_err(got.reshape(T, D), ref)
        print(f"[gpu]   rel err {err:.2e} via {sorted(families)}", flush=True)
        assert err <= BF16_TOL
    assert rel_err(ov.reshape(T, D), p[:, 2 * D:]) <= BF16_TOL
    assert ("head_norm_rotate" not in families) == fused, families


@pytest.mark.parametrize("dtype", [DT.BFloat16, DT.Float16, DT.Float32])
@pytest.mark.parametrize("shape,odd", [((2, 6, 5, 8), False), ((1, 12, 4, 12), True), ((1, 3, 3, 7), False)])
def test_nearest_upsample_exact(device, dtype, shape, odd):
    """UpsampleNearest of an image, or of its odd channels (a strided view,
    as Wan's DupUp3D shortcut takes them), equals numpy's repeat bit for bit:
    16-bit rows a multiple of 4 wide take the 16-byte kernel, the rest the
    per-element one."""
    B, C, H, W = shape
    print(f"[gpu] upsample {dtype.name} {shape} odd={odd}", flush=True)
    x = _round(normal("up_x", shape), dtype)
    g = nd.Graph(device)
    xi = g.Input(dtype, list(shape))
    src = Ops.Slice(xi, [0, 1, 0, 0], [B, C - 1, H, W], [1, 2, 1, 1]) if odd else xi
    m = nd.CompiledModel(g, [Layers.UpsampleNearest(src)], device)
    host = HostTensor.FromFloats(x)
    (y,) = m.Dispatch([host if dtype == DT.Float32 else host.ConvertTo(dtype)])
    m.Dispose()
    want = x[:, 1::2] if odd else x
    want = np.repeat(np.repeat(want, 2, 2), 2, 3)
    np.testing.assert_array_equal(y.ToFloats().reshape(want.shape), want)


# ---- the reference's smoke cases (Cli/SmokeTest.cs) ---------------------------------------

def test_smoke_gemm_and_broadcast_weight(device):
    # SmokeTest.Gemm (:66-91) and GemmBroadcastWeight (:93-119)
    g = nd.Graph(device)
    a = g.Input(DT.Float32, [1, 1, 2, 3])
    b = g.Input(DT.Float32, [1, 1, 3, 4])
    m = nd.CompiledModel(g, [Ops.Gemm(a, b)], device)
    ad = np.arange(1, 7, dtype=np.float32).reshape(2, 3)
    bd = np.arange(12, dtype=np.float32).reshape(3, 4)
    out = m.Dispatch([HostTensor.FromFloats(ad, 1, 1, 2, 3), HostTensor.FromFloats(bd, 1, 1, 3, 4)])[0]
    assert np.max(np.abs(out.ToFloats().reshape(2, 4) - ad @ bd)) <= 1e-4

    g = nd.Graph(device)
    x = g.Input(DT.Float32, [2, 1, 2, 3])
    w = g.Input(DT.Float32, [1, 1, 4, 3])
    bw = Ops.Reinterpret(w, [2, 1, 4, 3], [0, 12, 3, 1])
    m = nd.CompiledModel(g, [Ops.Gemm(x, bw, transB=True)], device)
    xd = np.arange(12, dtype=np.float32).reshape(2, 2, 3)
    wd = (np.arange(12) % 5 - 2).astype(np.float32).reshape(4, 3)
    out = m.Dispatch([HostTensor.FromFloats(xd, 2, 1, 2, 3), HostTensor.FromFloats(wd, 1, 1, 4, 3)])[0]
    assert np.max(np.abs(out.ToFloats().reshape(2, 2, 4) - xd @ wd.T)) <= 1e-4


def test_smoke_arithmetic_broadcast_transpose(device):
    # SmokeTest.ScaleBiasAndArithmetic / BroadcastAdd / TransposeView (:121-190)
    g = nd.Graph(device)
    x = g.Input(DT.Float32, [1, 1, 1, 4])
    y = 2.0 * x + 1.0
    z = (x * y - x) / y
    m = nd.CompiledModel(g, [z], device)
    d = np.array([1, 2, 3, 4], np.float32)
    out = m.Dispatch([HostTensor.FromFloats(d, 1, 1, 1, 4)])[0].ToFloats().ravel()
    yy = 2 * d + 1
    assert np.max(np.abs(out - (d * yy - d) / yy)) <= 1e-4

    g = nd.Graph(device)
    a = g.Input(DT.Float32, [1, 1, 3, 4])
    row = g.Input(DT.Float32, [1, 1, 1, 4])
    img = g.Input(DT.Float32, [1, 4, 2, 3])
    m = nd.CompiledModel(g, [a + Layers.Broadcast(row, [1, 1, 3, 4]), Layers.ToTokens(img) * 1.0], device)
    ad, rd = np.arange(12, dtype=np.float32), np.array([10, 20, 30, 40], np.float32)
    imd = np.arange(24, dtype=np.float32)
    o1, o2 = m.Dispatch([HostTensor.FromFloats(ad, 1, 1, 3, 4), HostTensor.FromFloats(rd, 1, 1, 1, 4),
                         HostTensor.FromFloats(imd, 1, 4, 2, 3)])
    assert np.array_equal(o1.ToFloats().reshape(3, 4), ad.reshape(3, 4) + rd)
    assert np.array_equal(o2.ToFloats().reshape(6, 4), imd.reshape(4, 6).T)


def test_smoke_group_norm_conv_join_upsample(device):
    # SmokeTest.GroupNormalization (:208-239), Convolution (:241-281),
    # JoinSliceUpsample (:308-335)
    g = nd.Graph(device)
    x = g.Input(DT.Float32, [1, 4, 1, 3])
    grouped = Ops.Reinterpret(x, [1, 2, 2, 3])
    gn = Ops.Reinterpret(Ops.MeanVarianceNormalization(grouped, [2, 3], 1e-5), [1, 4, 1, 3])
    m = nd.CompiledModel(g, [gn], device)
    data = np.array([1, 2, 3, 4, 5, 6, 0, 0, 0, 1, 1, 4], np.float32)
    out = m.Dispatch([HostTensor.FromFloats(data, 1, 4, 1, 3)])[0].ToFloats().ravel()
    assert np.max(np.abs(out - oracle.group_norm(data.reshape(1, 4, 1, 3), 2, eps=1e-5).ravel())) <= 1e-4

    g = nd.Graph(device)
    xi = g.Input(DT.Float32, [1, 1, 3, 3])
    fi = g.Input(DT.Float32, [2, 1, 3, 3])
    bi = g.Input(DT.Float32, [1, 2, 1, 1])
    m = nd.CompiledModel(g, [Ops.Convolution(xi, fi, bi, [1, 1], [1, 1], [1, 1])], device)
    f = np.zeros((2, 1, 3, 3), np.float32)
    f[0, 0, 1, 1] = 1
    f[1] = 1
    xd = np.arange(9, dtype=np.float32).reshape(1, 1, 3, 3)
    bias = np.array([0.5, -1], np.float32)
    out = m.Dispatch([HostTensor.FromFloats(xd), HostTensor.FromFloats(f), HostTensor.FromFloats(bias, 1, 2, 1, 1)])
    assert np.max(np.abs(out[0].ToFloats() - oracle.conv2d(xd, f, bias))) <= 1e-4

    g = nd.Graph(device)
    a = g.Input(DT.Float32, [1, 1, 2, 2])
    b = g.Input(DT.Float32, [1, 1, 2, 2])
    up = Ops.Upsample2D(Ops.Join([a, b], 1), 2, 2)
    cropped = Ops.Slice(up, [0, 0, 0, 0], [1, 2, 3, 3], [1, 1, 1, 1])
    m = nd.CompiledModel(g, [cropped], device)
    ad, bd = np.array([1, 2, 3, 4], np.float32), np.array([5, 6, 7, 8], np.float32)
    out = m.Dispatch([HostTensor.FromFloats(ad, 1, 1, 2, 2), HostTensor.FromFloats(bd, 1, 1, 2, 2)])[0]
    exp = oracle.upsample_nearest(np.concatenate([ad, bd]).reshape(1, 2, 2, 2))[:, :, :3, :3]
    assert np.array_equal(out.ToFloats(), exp)


def test_smoke_owned_weights_cast_tanh(device):
    # SmokeTest.OwnedWeights (:487-512), CastBothWays (:574-595), tanh (:498)
    model = nd.ModelBuilder(device)
    x = model.Placeholder([1, 1, 2, 2])
    w = model.Constant(HostTensor.FromFloats(np.array([1, 0, 0, 2], np.float32), 1, 1, 2, 2))
    model.Compile([Ops.Gemm(x, w)])
    for rnd in range(2):
        xd = np.array([1 + rnd, 2, 3, 4], np.float32)
        out = model.Run(HostTensor.FromFloats(xd, 1, 1, 2, 2))[0].ToFloats().ravel()
        assert np.array_equal(out, [xd[0], 2 * xd[1], xd[2], 2 * xd[3]])
    g = nd.Graph(device)
    x = g.Input(DT.Float32, [1, 1, 2, 4])
    half = Ops.Cast(x, DT.Float16)
    m = nd.CompiledModel(g, [half, Ops.Cast(half * 2.0, DT.Float32), Ops.ActivationTanh(x)], device)
    data = ((np.random.default_rng(4).random(8) - 0.5) * 4).astype(np.float32)
    o1, o2, o3 = m.Dispatch([HostTensor.FromFloats(data, 1, 1, 2, 4)])
    rounded = data.astype(np.float16).astype(np.float32)
    assert np.array_equal(o1.ToFloats().ravel(), rounded)
    assert np.array_equal(o2.ToFloats().ravel(), (rounded * 2).astype(np.float16).astype(np.float32))
    assert np.max(np.abs(o3.ToFloats().ravel() - np.tanh(data))) <= 1e-4


def test_smoke_mixed_precision_block(device):
    # SmokeTest.MixedPrecisionBlock (:778-813), at bf16 with tolerance 2e-2
    model = nd.ModelBuilder(device, DT.BFloat16)
    x = model.Placeholder([1, 1, 3, 4], DT.Float32)
    shift = model.Placeholder([1, 1, 1, 4], DT.Float32)
    weight = ((np.random.default_rng(8).random(16) - 0.5)).astype(np.float32)
    normed = Layers.Cast(Layers.LayerNorm(x, 1e-6) * 1.5 + Layers.Broadcast(shift, x.Shape), DT.BFloat16)
    projected = Layers.Linear(model, normed, HostTensor.FromFloats(weight, 4, 4))
    model.Compile([x + Layers.Cast(projected, DT.Float32) * 0.5])
    data = ((np.random.default_rng(9).random(12) - 0.5) * 4).astype(np.float32)
    sd = ((np.random.default_rng(10).random(4) - 0.5)).astype(np.float32)
    out = model.Run(HostTensor.FromFloats(data, 1, 1, 3, 4), HostTensor.FromFloats(sd, 1, 1, 1, 4))[0].ToFloats()
    n = oracle.modulate(data.reshape(3, 4), sd, np.full(4, 0.5, np.float32), 1e-6)
    exp = data.reshape(3, 4) + oracle.linear(n, weight.reshape(4, 4)) * 0.5
    assert np.max(np.abs(out.reshape(3, 4) - exp)) <= 2e-2


def test_repeat_dispatch_is_bitwise_identical(device):
    # SmokeTest.RmsNormHalfRepeats (:625-645): the first dispatch of a
    # process must equal the second to the bit.
    model = nd.ModelBuilder(device, DT.BFloat16)
    x = model.Placeholder([1, 256, 16, 128])
    w = HostTensor.FromFloats(normal("rw", (128,), 0.4))
    model.Compile([Layers.Cast(Layers.RmsNorm(model, x, w, 1e-6), DT.Float32),
                   Layers.Attend(*[Ops.Reinterpret(x, [1, 1, 256, 2048])] * 3, 16)])
    inp = HostTensor.FromFloats(normal("rx", (1, 256, 16, 128), 3)).ConvertTo(DT.BFloat16)
    first = [t.Data.copy() for t in model.Run(inp)]
    second = [t.Data.copy() for t in model.Run(inp)]
    for a, b in zip(first, second):
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8))


def test_errors_leave_the_device_usable(device):
    """OutOfVideoMemoryException leaves the device usable
    (Dml/DmlDevice.cs:918-937): forced from the host, no GPU fault."""
    device.SetFaultInjection(1)
    with pytest.raises(nd.OutOfVideoMemoryError):
        device.Empty(DT.Float32, [1024])
    t = device.Upload(HostTensor.FromFloats(np.arange(4, dtype=np.float32)))
    assert np.array_equal(t.Download().ToFloats(), np.arange(4, dtype=np.float32))
    model = nd.ModelBuilder(device)
    x = model.Placeholder([1, 1, 2, 2])
    with pytest.raises(nd.InvalidOperationError, match="Compile"):
        model.Run(HostTensor.FromFloats(np.zeros(4, np.float32), 1, 1, 2, 2))
    model.Compile([x * 2.0])
    with pytest.raises(nd.ArgumentError, match="expected 1 inputs"):
        model.Run()
    with pytest.raises(nd.ArgumentError):
        model.Compiled.DispatchOnDevice([device.Upload(HostTensor.FromFloats(np.zeros(3, np.float32)))])


def test_device_lost_is_fatal_to_that_device_only(device):
    """DeviceRemovedException (Dml/DmlDevice.cs:948-953): once a device
    reports itself lost, every call on it fails with DeviceRemovedError
    (uploads, runs of a model compiled before, new graphs), while another
    device on the same GPU keeps working. Forced from the host on a second
    device: no GPU fault."""
    other = nd.Device()
    model = nd.ModelBuilder(other)
    x = model.Placeholder([1, 1, 2, 2])
    model.Compile([x * 2.0])
    inp = HostTensor.FromFloats(np.ones(4, np.float32), 1, 1, 2, 2)
    assert np.array_equal(model.Run(inp)[0].ToFloats().ravel(), np.full(4, 2, np.float32))
    other.SetFaultInjection(2)
    with pytest.raises(nd.DeviceRemovedError):
        other.Upload(HostTensor.FromFloats(np.zeros(4, np.float32)))
    with pytest.raises(nd.DeviceRemovedError):
        model.Run(inp)
    with pytest.raises(nd.DeviceRemovedError):
        other.Empty(DT.Float32, [16])
    model.Dispose()
    other.Dispose()
    t = device.Upload(HostTensor.FromFloats(np.arange(4, dtype=np.float32)))
    assert np.array_equal(t.Download().ToFloats(), np.arange(4, dtype=np.float32))


@pytest.mark.parametrize("shape,groups", [((2, 320, 64, 64), 32), ((2, 1920, 32, 32), 32), ((1, 64, 7, 9), 32),
                                          ((2, 640, 33, 31), 32), ((1, 32, 256, 256), 4)])
@pytest.mark.parametrize("dtype,silu", [(DT.Float16, True), (DT.BFloat16, False), (DT.Float32, True)])
def test_group_norm_split_statistics(device, shape, groups, dtype, silu):
    """Layers.GroupNorm (+ SiLU) at SDXL's shapes: the statistics split over
    many workgroups per group, ragged extents that take the scalar paths, and
    groups large enough to need every split."""
    print(f"[gpu] group norm {shape} g={groups} {dtype.name} silu={silu}", flush=True)
    x = normal("gx", shape) * 2.0 + 0.5
    c = shape[1]
    w = 1.0 + normal("gw", (c,), 0.2)
    b = normal("gb", (c,), 0.2)
    xin = HostTensor.FromFloats(x).ConvertTo(dtype)
    xr = xin.ToFloats().reshape(shape)
    model = nd.ModelBuilder(device, dtype)
    p = model.Placeholder(list(shape), dtype)
    model.Compile([Layers.GroupNorm(model, p, HostTensor.FromFloats(w), HostTensor.FromFloats(b), groups, 1e-5,
                                    silu=silu)])
    out = run(model, xin)[0]
    wd = HostTensor.FromFloats(w).ConvertTo(dtype).ToFloats()
    bd = HostTensor.FromFloats(b).ConvertTo(dtype).ToFloats()
    ref = oracle.group_norm(xr, groups, wd, bd, 1e-5, silu)
    assert rel_err(out.reshape(shape), ref) <= (F32_TOL if dtype == DT.Float32 else BF16_TOL)


@pytest.mark.parametrize("B,T,S,H,d,mask", [
    (4, 1100, 300, 16, 128, None),     # 576 tiles on 512 slots: one round whole, 64 tiles split by keys
    (4, 1100, 300, 16, 128, "length"),
    (2, 2100, 260, 16, 64, None),      # 544 tiles, d 64
    (2, 2100, 517, 16, 64, "table"),
    (3, 1500, 1111, 15, 128, None),    # 540 tiles, 18 key blocks
])
def test_attention_split_schedule(device, B, T, S, H, d, mask):
    """More query tiles than the 512 resident workgroups: whole tiles first,
    the leftover tiles' key blocks spread over every workgroup and merged by
    the combine kernel (the running max, the rescaled sums)."""
    print(f"[gpu] split attention B={B} T={T} S={S} H={H} d={d} mask={mask}", flush=True)
    q = bf(normal("sq", (B, T, H * d), 2.0))
    k = bf(normal("sk", (B, S, H * d)))
    v = bf(normal("sv", (B, S, H * d)))
    model = nd.ModelBuilder(device, DT.BFloat16)
    ins = [model.Placeholder([B, 1, n, H * d]) for n in (T, S, S)]
    extra = []
    if mask == "length":
        kl = model.Placeholder([1, 1, 1, 1], DT.Int32)
        out = Layers.Attend(*ins, H, kl, nd.MaskType.KeySequenceLength)
        extra = [HostTensor.FromInt32(np.array([S - 37]), 1, 1, 1, 1)]
        ref = oracle.mha(q, k, v, H, mask_kind=1, key_len=S - 37)
    elif mask == "table":
        table = (normal("tbl", (B, 1, T, S)) > -0.5).astype(np.int32)
        tb = model.Placeholder([B, 1, T, S], DT.Int32)
        out = Layers.Attend(*ins, H, Layers.Broadcast(tb, [B, H, T, S]), nd.MaskType.Boolean)
        extra = [HostTensor.FromInt32(table)]
        ref = oracle.mha(q, k, v, H, mask_kind=2, mask=table)
    else:
        out = Layers.Attend(*ins, H)
        ref = oracle.mha(q, k, v, H)
    model.Compile([out])
    got = run(model, *[HostTensor.FromFloats(a.reshape(B, 1, -1, H * d)).ConvertTo(DT.BFloat16) for a in (q, k, v)],
              *extra)[0]
    err = rel_err(got.reshape(ref.shape), ref)
    print(f"[gpu]   rel err {err:.2e}", flush=True)
    assert err <= BF16_TOL


@pytest.mark.parametrize("M1,M2,K,N", [(1000, 77, 512, 384), (5376 // 4, 256, 1024, 1536), (300, 300, 256, 2056)])
def test_paired_linears_run_as_one_launch(device, M1, M2, K, N):
    """Two independent linears of equal N and K emitted back to back (the
    image and text streams' projections) run as one launch, each with its
    own epilogue; a third that reads the first's output is not paired."""
    print(f"[gpu] paired linears M1={M1} M2={M2} K={K} N={N}", flush=True)
    x1, x2 = bf(normal("px1", (1, 1, M1, K))), bf(normal("px2", (1, 1, M2, K)))
    w1, w2 = bf(normal("pw1", (N, K), 0.05)), bf(normal("pw2", (N, K), 0.05))
    b1, b2 = bf(normal("pb1", (N,), 0.05)), bf(normal("pb2", (N,), 0.05))
    r2 = normal("pr2", (1, 1, M2, N))
    g2 = normal("pg2", (1, 1, 1, N))
    w3 = bf(normal("pw3", (N, N), 0.05))
    model = nd.ModelBuilder(device, DT.BFloat16)
    p1 = model.Placeholder([1, 1, M1, K])
    p2 = model.Placeholder([1, 1, M2, K])
    pr = model.Placeholder([1, 1, M2, N], DT.Float32)
    pg = model.Placeholder([1, 1, 1, N], DT.Float32)
    y1 = Layers.Linear(model, p1, HostTensor.FromFloats(w1), HostTensor.FromFloats(b1), activation="gelu_tanh")
    y2 = Layers.Linear(model, p2, HostTensor.FromFloats(w2), HostTensor.FromFloats(b2), gate=pg, residual=pr)
    y3 = Layers.Linear(model, y1, HostTensor.FromFloats(w3))
    model.Compile([y1, y2, y3])
    model.Compiled.SetProfiling(True)
    o1, o2, o3 = run(model, HostTensor.FromFloats(x1).ConvertTo(DT.BFloat16),
                     HostTensor.FromFloats(x2).ConvertTo(DT.BFloat16), HostTensor.FromFloats(r2), HostTensor.FromFloats(g2))
    launches = sum(e["launches"] for k, e in model.Compiled.Profile().items() if k.startswith("gemm"))
    assert launches == 2, model.Compiled.Profile()
    e1 = oracle.gelu_tanh(oracle.linear(x1, w1, b1))
    e2 = r2 + g2 * bf(oracle.linear(x2, w2, b2))
    e3 = oracle.linear(bf(e1), w3)
    assert rel_err(o1, e1) <= BF16_TOL
    assert rel_err(o2 - r2, e2 - r2) <= BF16_TOL
    assert rel_err(o3, e3) <= BF16_TOL


def _round(x, dtype):
    x = np.asarray(x, np.float32)
    if dtype == DT.BFloat16:
        return bf(x)
    if dtype == DT.Float16:
        return x.astype(np.float16).astype(np.float32)
    return x


@pytest.mark.parametrize("dtype", [DT.Float16, DT.BFloat16, DT.Float32])
def test_elementwise_vector_and_generic_paths(device, dtype):
    """Elementwise ops over rows whose length is a multiple of 8 (the
    vectorised kernel: a row slice times GELU of the other half, as SDXL's
    GEGLU; a per-channel broadcast add, as its time embedding; unary and
    binary ops on packed rows) and over ragged rows (the generic kernel),
    against numpy on the same rounded inputs."""
    print(f"[gpu] elementwise paths {dtype.name}", flush=True)
    B, C, H, W, n, inner = 2, 6, 5, 40, 7, 48
    p_h = _round(normal("ep", (B, 1, n, 2 * inner)), dtype)
    x_h = _round(normal("ex", (B, C, H, W)), dtype)
    t_h = _round(normal("et", (B, C, 1, 1)), dtype)
    r_h = _round(normal("er", (B, 1, 3, 21)), dtype)
    g = nd.Graph(device)
    proj = g.Input(dtype, [B, 1, n, 2 * inner])
    x = g.Input(dtype, [B, C, H, W])
    t = g.Input(dtype, [B, C, 1, 1])
    r = g.Input(dtype, [B, 1, 3, 21])
    a = Ops.Slice(proj, [0, 0, 0, 0], [B, 1, n, inner])
    b = Ops.Slice(proj, [0, 0, 0, inner], [B, 1, n, inner])
    outs = [a * Ops.ActivationGelu(b), x + Layers.Broadcast(t, [B, C, H, W]), Ops.ActivationSwish(x),
            Ops.Divide(x, Ops.ActivationSigmoid(x)), Ops.Subtract(x, x * 0.5), r * r + r]
    m = nd.CompiledModel(g, outs, device)

    def host(v):
        ht = HostTensor.FromFloats(v)
        return ht if dtype == DT.Float32 else ht.ConvertTo(dtype)

    got = [o.ToFloats().reshape(e.shape) for o, e in zip(
        m.Dispatch([host(p_h), host(x_h), host(t_h), host(r_h)]),
        [p_h[..., :inner], x_h, x_h, x_h, x_h, r_h])]
    a_n, b_n = p_h[..., :inner], p_h[..., inner:]
    gelu = lambda v: 0.5 * v * (1.0 + np.vectorize(math.erf)(v / math.sqrt(2.0)))
    sig = lambda v: 1.0 / (1.0 + np.exp(-v))
    ref = [a_n * _round(gelu(b_n), dtype), x_h + t_h, x_h * sig(x_h), x_h / _round(sig(x_h), dtype),
           x_h - _round(x_h * 0.5, dtype), _round(r_h * r_h, dtype) + r_h]
    tol = 1e-5 if dtype == DT.Float32 else 1.5e-2
    for k, (o, e) in enumerate(zip(got, ref)):
        err = rel_err(o, e)
        print(f"[gpu]   output {k}: rel err {err:.2e}", flush=True)
        assert err <= tol, (k, err)


@pytest.mark.parametrize("dtype", [DT.Float16, DT.BFloat16, DT.Float32])
@pytest.mark.parametrize("width", [48, 21])
def test_geglu_fused_equals_unfused(device, dtype, width):
    """a * Gelu(b) over two halves of one projection (SDXL's GEGLU) runs as
    one elementwise pass when nothing else reads the GELU; the GELU is still
    rounded to the compute type before the product, so the fused result
    equals the two-pass one (the GELU kept as an output) bit for bit, and
    numpy's within the type's rounding."""
    B, n = 2, 7
    print(f"[gpu] GEGLU fused {dtype.name} width {width}", flush=True)
    p_h = _round(normal("gg", (B, 1, n, 2 * width)), dtype)

    def build(keep_gelu):
        g = nd.Graph(device)
        proj = g.Input(dtype, [B, 1, n, 2 * width])
        gl = Ops.ActivationGelu(Ops.Slice(proj, [0, 0, 0, width], [B, 1, n, width]))
        y = Ops.Slice(proj, [0, 0, 0, 0], [B, 1, n, width]) * gl
        m = nd.CompiledModel(g, [y, gl] if keep_gelu else [y], device)
        m.SetProfiling(True)
        ht = HostTensor.FromFloats(p_h)
        out = m.Dispatch([ht if dtype == DT.Float32 else ht.ConvertTo(dtype)])[0].ToFloats()
        return out, m.Profile()["elementwise"]["launches"]

    fused, n_fused = build(False)
    split, n_split = build(True)
    assert (n_fused, n_split) == (1, 2)
    np.testing.assert_array_equal(fused, split)
    gelu = lambda v: 0.5 * v * (1.0 + np.vectorize(math.erf)(v / math.sqrt(2.0)))
    ref = p_h[..., :width] * _round(gelu(p_h[..., width:]), dtype)
    assert rel_err(fused.reshape(ref.shape), ref) <= (1e-5 if dtype == DT.Float32 else 1.5e-2)


@pytest.mark.parametrize("dtype", [DT.Float16, DT.BFloat16, DT.Float32])
@pytest.mark.parametrize("shape", [(2, 128, 8, 24), (1, 96, 5, 7)])
def test_to_image_residual(device, dtype, shape):
    """SDXL's ToImage(tokens) + x (sdxl.py's transformer residual): 16-bit
    tensors whose channels and pixels are multiples of 64 take the tiled
    transpose kernel, the rest the generic one; both round the fp32 sum once,
    so the result equals numpy's bit for bit. ToImage alone (a copy) is checked
    too."""
    B, C, H, W = shape
    print(f"[gpu] ToImage residual {dtype.name} {shape}", flush=True)
    t_h = _round(normal("ti_t", (B, 1, H * W, C)), dtype)
    x_h = _round(normal("ti_x", (B, C, H, W)), dtype)
    g = nd.Graph(device)
    t = g.Input(dtype, [B, 1, H * W, C])
    x = g.Input(dtype, [B, C, H, W])
    img = Layers.ToImage(t, H, W)
    m = nd.CompiledModel(g, [img + x, Ops.ActivationIdentity(img)], device)

    def host(v):
        ht = HostTensor.FromFloats(v)
        return ht if dtype == DT.Float32 else ht.ConvertTo(dtype)

    got = [o.ToFloats().reshape(B, C, H, W) for o in m.Dispatch([host(t_h), host(x_h)])]
    t_img = t_h.reshape(B, H, W, C).transpose(0, 3, 1, 2)
    np.testing.assert_array_equal(got[0], _round(t_img + x_h, dtype))
    np.testing.assert_array_equal(got[1], t_img)


@pytest.mark.parametrize("dtype", [DT.Float16, DT.BFloat16, DT.Float32])
@pytest.mark.parametrize("shape", [(2, 128, 8, 24), (1, 96, 5, 7), (2, 64, 4, 16)])
def test_to_tokens_and_channel_join(device, dtype, shape):
    """SDXL's proj_in input, ToTokens of a computed NCHW image made packed
    (16-bit channels and pixels multiples of 64: the vectorised NCHW -> NHWC
    tile; other 16-bit shapes: the scalar tile; fp32: the generic copy), and
    its up path's channel concatenation (each input written into a channel
    slice: the vectorised kernel when rows are multiples of 8), both exact."""
    B, C, H, W = shape
    print(f"[gpu] ToTokens / channel join {dtype.name} {shape}", flush=True)
    x_h = _round(normal("tt_x", (B, C, H, W)), dtype)
    s_h = _round(normal("tt_s", (B, C // 2, H, W)), dtype)
    g = nd.Graph(device)
    x = g.Input(dtype, [B, C, H, W])
    s = g.Input(dtype, [B, C // 2, H, W])
    img = Ops.ActivationIdentity(x)
    m = nd.CompiledModel(g, [Layers.ToTokens(img), Ops.Join([img, s], 1)], device)

    def host(v):
        ht = HostTensor.FromFloats(v)
        return ht if dtype == DT.Float32 else ht.ConvertTo(dtype)

    tok, cat = (o.ToFloats() for o in m.Dispatch([host(x_h), host(s_h)]))
    np.testing.assert_array_equal(tok.reshape(B, H * W, C), x_h.reshape(B, C, H * W).transpose(0, 2, 1))
    np.testing.assert_array_equal(cat.reshape(B, C + C // 2, H, W), np.concatenate([x_h, s_h], 1))


@pytest.mark.parametrize("dtype", [DT.BFloat16, DT.Float16])
@pytest.mark.parametrize("weight", ["none", "same", "f32"])
@pytest.mark.parametrize("rotate", [True, False])
def test_head_norm_rotate_typed_forms(device, dtype, weight, rotate):
    """The compile-time-typed d = 128 kernel in each of its forms: no
    weight, a weight of the input's type or fp32, with and without the
    rotation, against the oracle."""
    print(f"[gpu] head norm rotate {dtype.name} weight={weight} rotate={rotate}", flush=True)
    T, H, d = 77, 4, 128
    x = _round(normal("tx", (1, 1, T, H * d)) * 2, dtype)
    w = _round(normal("tw", (d,), 0.2) + 1, dtype if weight == "same" else DT.Float32)
    cos, sin = oracle.mmdit_rope_tables(7, 11, 0)
    model = nd.ModelBuilder(device, dtype)
    xi = model.Placeholder([1, 1, T, H * d], dtype)
    ci = model.Placeholder([1, T, 1, 64], DT.Float32)
    si = model.Placeholder([1, T, 1, 64], DT.Float32)
    wi = None
    if weight == "same":
        wi = model.Constant(HostTensor.FromFloats(w), [d], dtype)
    elif weight == "f32":
        wi = model.Constant(HostTensor.FromFloats(w), [d], DT.Float32)
    y = Ops.HeadNormRotate(xi, wi, 1e-6, ci if rotate else None, si if rotate else None, H, dtype)
    model.Compile([y])
    host_x = HostTensor.FromFloats(x).ConvertTo(dtype)
    (o,) = run(model, host_x, HostTensor.FromFloats(cos.reshape(1, T, 1, 64)),
               HostTensor.FromFloats(sin.reshape(1, T, 1, 64)))
    normed = oracle.rms_norm(x.reshape(T * H, d), w if weight != "none" else np.ones(d, np.float32), 1e-6)
    ref = normed.reshape(T, H * d)
    if rotate:
        ref = oracle.rope(ref, H, cos, sin)
    assert rel_err(o.reshape(T, -1), ref) <= BF16_TOL


@pytest.mark.parametrize("d,dtype", [(128, DT.BFloat16), (64, DT.Float16), (128, DT.Float32)])
@pytest.mark.parametrize("rising", [True, False])
def test_attention_score_drift(device, d, dtype, rising):
    """Scores whose scale drifts along the keys (each key row scaled by a ramp
    from 1 to 12): rising, the running max grows by more than 2^8 many times
    after the first block and the output is rescaled each time; falling, the
    max is set early and later probabilities are tiny. Both against the
    oracle."""
    print(f"[gpu] attention drift d={d} {dtype.name} rising={rising}", flush=True)
    T, S, H = 130, 700, 2
    q = bf(normal("dq", (1, T, H * d)))
    ramp = np.linspace(1.0, 12.0, S, dtype=np.float32)
    if not rising:
        ramp = ramp[::-1].copy()
    k = bf(normal("dk", (1, S, H * d)) * ramp[None, :, None])
    v = bf(normal("dv", (1, S, H * d)))
    model = nd.ModelBuilder(device, dtype)
    ins = [model.Placeholder([1, 1, n, H * d]) for n in (T, S, S)]
    model.Compile([Layers.Attend(*ins, H)])
    host = lambda a: HostTensor.FromFloats(a.reshape(1, 1, -1, H * d))
    out = run(model, *[host(a) if dtype == DT.Float32 else host(a).ConvertTo(dtype) for a in (q, k, v)])[0]
    ref = oracle.mha(q, k, v, H)
    err = rel_err(out.reshape(ref.shape), ref)
    print(f"[gpu]   rel err {err:.2e}", flush=True)
    assert err <= (F32_TOL if dtype == DT.Float32 else BF16_TOL)


@pytest.mark.parametrize("dtype", [DT.Float16, DT.BFloat16])
@pytest.mark.parametrize("D", [512, 640, 1280, 200, 202])
def test_layer_and_rms_norm_16bit(device, dtype, D):
    """LayerNorm and RMSNorm on 16-bit rows with 16-bit affine terms (SDXL's
    640 / 1280 channels; 512 and 1280 take the vectorised kernel, 640 and 200
    its form for widths that are a multiple of 4 but not of 256, 202 the
    per-element one), against the oracle on the same rounded inputs."""
    print(f"[gpu] 16-bit norms {dtype.name} D={D}", flush=True)
    rows = 37
    x = _round(normal("n16x", (1, 1, rows, D)) * 2 + 0.5, dtype)
    w = _round(normal("n16w", (D,), 0.3) + 1, dtype)
    b = _round(normal("n16b", (D,), 0.3), dtype)
    model = nd.ModelBuilder(device, dtype)
    xi = model.Placeholder([1, 1, rows, D], dtype)
    ln = Layers.LayerNorm(model, xi, HostTensor.FromFloats(w), HostTensor.FromFloats(b), 1e-5)
    rms = Layers.RmsNorm(model, xi, HostTensor.FromFloats(w), 1e-6)
    model.Compile([ln, rms])
    o1, o2 = run(model, HostTensor.FromFloats(x).ConvertTo(dtype))
    assert rel_err(o1.reshape(rows, D), oracle.layer_norm(x.reshape(rows, D), w, b, 1e-5)) <= BF16_TOL
    assert rel_err(o2.reshape(rows, D), oracle.rms_norm(x.reshape(rows, D), w, 1e-6)) <= BF16_TOL


@pytest.mark.parametrize("dtype", [DT.BFloat16, DT.Float16, DT.Float32])
@pytest.mark.parametrize("shape", [(1, 144, 9, 13), (1, 1152, 5, 7), (2, 64, 8, 8), (1, 96, 8, 12),
                                   (1, 144, 8, 12), (1, 288, 4, 10), (1, 576, 4, 6), (2, 1152, 4, 18)])
@pytest.mark.parametrize("silu", [False, True])
def test_channel_norm_of_an_image(device, dtype, shape, silu):
    """RMSNorm and LayerNorm of an NCHW image's token view (the Wan VAE's
    channel norms) run on the image as it lies and write tokens, a SiLU
    after them joined in: no transposed copy, no separate SiLU pass. Against
    the oracle's row norms of the transposed image, the SiLU taken of the
    norm rounded to the compute type (what the unfused graph computes).
    Channel counts above and below one 64-channel slab, pixels not a
    multiple of 64, two images. 16-bit images whose pixels are a multiple
    of 8 take the 16-byte kernel (each register-held width of the RMSNorm,
    256 and 512 threads, and the re-reading form at 256 and 1024 threads),
    the rest the per-element one."""
    B, C, H, W = shape
    print(f"[gpu] channel norm {dtype.name} {shape} silu={silu}", flush=True)
    x = _round(normal("cn_x", shape) * 2 + 0.5, dtype)
    w = _round(normal("cn_w", (C,), 0.3) + 1, dtype)
    b = _round(normal("cn_b", (C,), 0.3), dtype)
    model = nd.ModelBuilder(device, dtype)
    xi = model.Placeholder(list(shape), dtype)
    t = Layers.ToTokens(xi)
    rms = Layers.RmsNorm(model, t, HostTensor.FromFloats(w), 1e-6)
    ln = Layers.LayerNorm(model, t, HostTensor.FromFloats(w), HostTensor.FromFloats(b), 1e-5)
    if silu:
        rms, ln = Layers.Silu(rms), Layers.Silu(ln)
    model.Compile([rms, ln])
    model.Compiled.SetProfiling(True)
    host = HostTensor.FromFloats(x)
    o1, o2 = run(model, host if dtype == DT.Float32 else host.ConvertTo(dtype))
    families = set(model.Compiled.Profile())
    model.Dispose()
    rows = x.transpose(0, 2, 3, 1).reshape(B * H * W, C)
    want = [oracle.rms_norm(rows, w, 1e-6), oracle.layer_norm(rows, w, b, 1e-5)]
    if silu:
        want = [(lambda v: v / (1.0 + np.exp(-v)))(_round(r, dtype)) for r in want]
    tol = 1e-5 if dtype == DT.Float32 else 1e-2
    for got, ref in zip((o1, o2), want):
        err = rel_err(got.reshape(ref.shape), ref)
        print(f"[gpu]   rel err {err:.2e}", flush=True)
        assert err <= tol
    assert {"channel_rms_norm", "channel_layer_norm"} <= families, families
    assert "nchw_to_nhwc" not in families and "elementwise" not in families, families
