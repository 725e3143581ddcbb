"""The C ABI on the CPU: libndx.so loads, exports exactly what include/ndx.h
declares, and its device-free paths behave — the host quantiser (bit-exact
against the golden vectors and the oracle), shape inference with the
reference's argument errors on a graph without a device, and the call-order
errors. No GPU calls are made here."""

import ctypes
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

import naivediffusion_amd as nd
import oracle
from naivediffusion_amd import _lib
from naivediffusion_amd.graph import Graph, Ops
from naivediffusion_amd.layers import Layers, Transformer
from naivediffusion_amd.tensors import HostDataType as DT

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "ndx.h"
GOLDEN = ROOT / "tests" / "golden" / "quantizer_golden.npz"


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"NDX_API\s+[\w\s\*]+?\b(ndx_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    names = declared_symbols()
    assert len(names) > 40
    L = _lib.lib()
    for n in names:
        assert hasattr(L, n), n
    # and nothing undeclared is exported under the ndx_ prefix
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True).stdout
    exported = sorted(set(re.findall(r"\bT (ndx_\w+)", out)))
    assert exported == names
    # the ctypes signature table covers the header
    assert sorted(n for n, _, _ in _lib.SIGNATURES) == names


def test_version_and_device_count_without_a_gpu():
    assert b"gfx950" in _lib.lib().ndx_version()
    assert nd.Device.Count() >= 0


def test_the_library_was_built_from_these_sources():
    """ndx_version() ends with the hash of the sources the library was built
    from; the loader refuses a library whose hash is not the sources' now."""
    from naivediffusion_amd import build
    built = _lib.lib().ndx_version().decode().rsplit(" ", 1)[-1]
    assert built == build.source_hash()
    fake = type("L", (), {"ndx_version": staticmethod(lambda: b"ndx 0.2 (gfx950) src 0123456789abcdef")})
    with pytest.raises(ImportError, match="stale"):
        _lib._check_fresh(fake)


def test_host_quantizer_is_bit_exact_with_golden_and_oracle():
    g = np.load(GOLDEN)
    for name in ("mixed", "zero", "ties", "big", "small"):
        w = np.ascontiguousarray(g[f"{name}_w"], np.float32)
        rows, cols = w.shape
        q = np.empty((rows, cols), np.int8)
        s = np.empty((rows, cols // 32), np.uint16)
        _lib.call("ndx_quantize_block_int8", w.ctypes.data_as(ctypes.c_void_p), int(DT.Float32), rows, cols, 32,
                  int(DT.Float16), q.ctypes.data_as(ctypes.c_void_p), s.ctypes.data_as(ctypes.c_void_p))
        assert np.array_equal(q, g[f"{name}_q"]), name
        assert np.array_equal(s, g[f"{name}_s"]), name


def test_host_quantizer_reads_bf16_and_f16_like_their_widened_values():
    rng = np.random.default_rng(4)
    w32 = (rng.standard_normal((64, 256)) * 0.02).astype(np.float32)
    bits = nd.tensors.f32_to_bf16(w32)
    wide = nd.tensors.bf16_to_f32(bits)
    for data, dt in ((bits, DT.BFloat16), (wide.astype(np.float16), DT.Float16)):
        q = np.empty((64, 256), np.int8)
        s = np.empty((64, 8), np.uint16)
        _lib.call("ndx_quantize_block_int8", data.ctypes.data_as(ctypes.c_void_p), int(dt), 64, 256, 32,
                  int(DT.Float16), q.ctypes.data_as(ctypes.c_void_p), s.ctypes.data_as(ctypes.c_void_p))
        ref = wide if dt == DT.BFloat16 else wide.astype(np.float16).astype(np.float32)
        oq, os_ = oracle.quantize(ref, 64)
        assert np.array_equal(q, oq) and np.array_equal(s, os_)
    # per-output-channel fp32 scales
    q = np.empty((64, 256), np.int8)
    s = np.empty((64, 1), np.float32)
    _lib.call("ndx_quantize_block_int8", wide.ctypes.data_as(ctypes.c_void_p), int(DT.Float32), 64, 256, 256,
              int(DT.Float32), q.ctypes.data_as(ctypes.c_void_p), s.ctypes.data_as(ctypes.c_void_p))
    oq, os_ = oracle.quantize(wide, 64, block=256, fp16_scales=False)
    assert np.array_equal(q, oq) and np.array_equal(s, os_)


def test_quantizer_fits_rule():
    # BlockQuantizerTests.FitsNeedsWholeBlocksPerRow (:9-16)
    fits = _lib.lib().ndx_quantize_fits
    assert fits(4 * 64, 4, 32) == 1
    assert fits(4 * 48, 4, 32) == 0
    assert fits(100, 3, 32) == 0
    assert fits(64, 0, 32) == 0


def test_quantizer_refuses_a_shape_that_does_not_tile():
    w = np.zeros((1, 48), np.float32)
    q = np.empty(48, np.int8)
    s = np.empty(2, np.uint16)
    with pytest.raises(nd.ArgumentError):
        _lib.call("ndx_quantize_block_int8", w.ctypes.data_as(ctypes.c_void_p), 0, 1, 48, 32, 1,
                  q.ctypes.data_as(ctypes.c_void_p), s.ctypes.data_as(ctypes.c_void_p))


# ---- shape inference on a device-less graph ---------------------------------------

def test_linear_shapes_and_errors():
    g = Graph(None, DT.BFloat16)
    x = g.Input(DT.BFloat16, [2, 1, 1024, 3072])
    w = g.Input(DT.BFloat16, [12288, 3072])
    y = Ops.Linear(x, w)
    assert y.Shape == (2, 1, 1024, 12288) and y.DataType == DT.BFloat16
    bad = g.Input(DT.BFloat16, [12288, 3000])
    with pytest.raises(nd.ArgumentError, match="inner extents differ"):
        Ops.Linear(x, bad)
    resid = g.Input(DT.Float32, [2, 1, 1024, 12288])
    gate = g.Input(DT.Float32, [2, 1, 1, 12288])
    y = Ops.Linear(x, w, None, 4, gate, resid)
    assert y.DataType == DT.Float32
    with pytest.raises(nd.ArgumentError, match="residual"):
        Ops.Linear(x, w, None, 4, gate, g.Input(DT.Float32, [2, 1, 1000, 12288]))
    w8 = g.Input(DT.Int8, [12288, 3072])
    with pytest.raises(nd.UnsupportedError):
        Ops.Linear(x, w8)


def test_gemm_shape_rule():
    # DmlOps.Gemm (:231-262) and the smoke case of SmokeTest.cs:66-91
    g = Graph(None)
    a = g.Input(DT.Float32, [1, 1, 2, 3])
    b = g.Input(DT.Float32, [1, 1, 3, 4])
    assert Ops.Gemm(a, b).Shape == (1, 1, 2, 4)
    bt = g.Input(DT.Float32, [1, 1, 4, 3])
    assert Ops.Gemm(a, bt, transB=True).Shape == (1, 1, 2, 4)
    with pytest.raises(nd.ArgumentError):
        Ops.Gemm(a, bt)


def test_elementwise_needs_same_shape_and_width():
    g = Graph(None)
    a = g.Input(DT.Float32, [1, 1, 3, 4])
    with pytest.raises(nd.ArgumentError, match="shape"):
        a + g.Input(DT.Float32, [1, 1, 1, 4])
    with pytest.raises(nd.ArgumentError, match="precision"):
        a + g.Input(DT.Float16, [1, 1, 3, 4])
    # broadcasting is a stride-0 view (Layers.Broadcast)
    row = g.Input(DT.Float32, [1, 1, 1, 4])
    assert (a + Layers.Broadcast(row, a.Shape)).Shape == (1, 1, 3, 4)
    with pytest.raises(nd.ArgumentError, match="cannot broadcast"):
        Layers.Broadcast(g.Input(DT.Float32, [1, 1, 2, 4]), [1, 1, 3, 4])
    assert (2.0 * a + 1.0).Shape == (1, 1, 3, 4)


def test_views_stay_inside_their_tensor():
    g = Graph(None)
    x = g.Input(DT.Float32, [1, 4, 2, 3])
    t = Layers.ToTokens(x)
    assert t.Shape == (1, 1, 6, 4)
    assert Layers.ToImage(t, 2, 3).Shape == (1, 4, 2, 3)
    with pytest.raises(nd.ArgumentError):
        Ops.Reinterpret(x, [1, 1, 25, 1])
    with pytest.raises(nd.ArgumentError):
        Ops.Slice(x, [0, 0, 1, 0], [1, 4, 2, 3])
    s = Ops.Slice(x, [0, 1, 0, 0], [1, 2, 2, 3], [1, 1, 1, 1])
    assert s.Shape == (1, 2, 2, 3)
    j = Ops.Join([x, x], 1)
    assert j.Shape == (1, 8, 2, 3)


def test_attention_shapes_and_masks():
    g = Graph(None, DT.BFloat16)
    q = g.Input(DT.BFloat16, [1, 1, 1152, 3072])
    kv = g.Input(DT.BFloat16, [1, 1, 1152, 3072])
    assert Layers.Attend(q, kv, kv, 24).Shape == (1, 1, 1152, 3072)
    with pytest.raises(nd.ArgumentError, match="heads"):
        Layers.Attend(q, kv, kv, 7)
    kl = g.Input(DT.Int32, [1, 1, 1, 1])
    assert Layers.Attend(q, kv, kv, 24, kl, nd.MaskType.KeySequenceLength).Shape == (1, 1, 1152, 3072)
    table = g.Input(DT.Int32, [1, 1, 1152, 1152])
    Layers.Attend(q, kv, kv, 24, Layers.Broadcast(table, [1, 24, 1152, 1152]), nd.MaskType.Boolean)
    with pytest.raises(nd.ArgumentError, match="mask and its type"):
        Ops.MultiheadAttention(q, kv, kv, 24, 0.1, kl, nd.MaskType.NONE)


def test_norm_and_conv_shapes():
    g = Graph(None)
    x = g.Input(DT.Float32, [2, 320, 16, 16])
    w = g.Input(DT.Float32, [640, 320, 3, 3])
    assert Ops.Convolution(x, w, None, [2, 2], [1, 1], [1, 1]).Shape == (2, 640, 8, 8)
    assert Ops.Convolution(x, w, None, [1, 1], [1, 1], [1, 1]).Shape == (2, 640, 16, 16)
    with pytest.raises(nd.ArgumentError, match="groups"):
        Ops.GroupNorm(x, None, None, 33, 1e-5)
    t = g.Input(DT.Float32, [1, 1, 77, 3072])
    sc = g.Input(DT.Float32, [1, 1, 1, 3072])
    assert Transformer.Modulate(t, sc, sc, 1e-6, DT.BFloat16).DataType == DT.BFloat16
    assert Ops.Patchify(g.Input(DT.Float32, [1, 16, 128, 168]), 2).Shape == (1, 1, 5376, 64)


def test_compile_needs_a_device_and_builder_order():
    g = Graph(None)
    x = g.Input(DT.Float32, [1, 1, 2, 2])
    y = x * 2.0
    with pytest.raises(nd.InvalidOperationError):
        nd.CompiledModel(g, [y], None)


def test_host_tensor_widening_and_narrowing():
    # HostTensor.Widen / ConvertTo: bf16 is the top half, exact both ways on
    # representable values; narrowing rounds to nearest even like the oracle.
    vals = np.array([0.1, -2.5, 3.14159, 1e-30, 65504, 7e4], np.float32)
    h = nd.HostTensor.FromFloats(vals)
    b = h.ConvertTo(DT.BFloat16)
    assert np.array_equal(b.Data, oracle.f32_to_bf16_bits(vals))
    assert np.array_equal(b.ToFloats(), (b.Data.astype(np.uint32) << 16).view(np.float32))
    f = h.ConvertTo(DT.Float16)
    with np.errstate(over="ignore"):
        assert np.array_equal(f.Data.view(np.uint16), oracle.f32_to_f16_bits(vals))
    with pytest.raises(nd.ArgumentError):
        nd.HostTensor(DT.Float32, [3], np.zeros(4, np.float32))
