"""Pins the oracle (oracle/oracle.c) before anything is checked against it:
the reference's own known answers (BlockQuantizerTests.cs, CpuMathTests.cs,
TransformerInputsTests.cs, NarrowingLossTests.cs and the CPU references of
Cli/SmokeTest.cs), IEEE conversions from numpy, closed forms, float64 brute
force, and invariants chosen so a dropped term, a wrong sign or index or a
transposed operand fails. CPU only."""

import math
from pathlib import Path

import numpy as np
import pytest

import oracle

GOLDEN = Path(__file__).resolve().parent / "golden" / "quantizer_golden.npz"


def r(seed, *shape, spread=1.0):
    return ((np.random.default_rng(seed).random(shape) - 0.5) * spread).astype(np.float32)


# ---- narrow floats -------------------------------------------------------------

def test_f16_conversion_matches_ieee_round_to_nearest_even():
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * 10,
        np.float32(2.0) ** rng.integers(-30, 17, 2000).astype(np.float32) * rng.random(2000).astype(np.float32),
        np.array([0.0, -0.0, 65504, 65519.99, 65520, 1e9, -1e9, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8, 1e-12,
                  np.inf, -np.inf], np.float32),
        # exact ties between neighbouring halves
        (np.arange(1, 200, dtype=np.float32) * 2 + 1) * np.float32(2.0 ** -11),
    ]).astype(np.float32)
    ours = oracle.f32_to_f16_bits(vals)
    with np.errstate(over="ignore"):
        ref = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, ref)
    back = oracle.f16_bits_to_f32(ref)
    assert np.array_equal(back, ref.view(np.float16).astype(np.float32))


def test_bf16_narrowing_rounds_to_nearest_even():
    vals = np.array([1.0, 1.00390625, 1.005859375, 1.0078125 + 2 ** -9, -3.14159, 1e-40], np.float32)
    bits = oracle.f32_to_bf16_bits(vals)
    # independent: round half to even on the top 16 bits
    u = vals.view(np.uint32).astype(np.uint64)
    ref = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    assert np.array_equal(bits, ref)
    assert bits[1] == 0x3F80  # 1 + 2^-8 is a tie: rounds to the even 1.0


# ---- BlockQuantizer (BlockQuantizerTests.cs) ---------------------------------------

def test_quantizer_matches_independent_golden_vectors():
    g = np.load(GOLDEN)
    for name in ("mixed", "zero", "ties", "big", "small"):
        w = g[f"{name}_w"]
        q, s = oracle.quantize(w, w.shape[0])
        assert np.array_equal(q, g[f"{name}_q"]), name
        assert np.array_equal(s, g[f"{name}_s"]), name


def test_dequantizing_comes_back_within_half_a_step():
    # BlockQuantizerTests.DequantizingComesBackWithinHalfAStep (:19-50)
    rows, cols = 4, 96
    rng = np.random.default_rng(1)
    values = ((rng.random((rows, cols)) * 2 - 1) * np.where(rng.integers(0, 4, (rows, cols)) == 0, 8, 1)).astype(
        np.float32)
    q, s = oracle.quantize(values, rows)
    assert q.dtype == np.int8 and q.shape == (rows, cols)
    assert s.shape == (rows, cols // 32)
    scale = s.view(np.float16).astype(np.float32)
    for row in range(rows):
        for b in range(cols // 32):
            blk = values[row, b * 32:(b + 1) * 32]
            peak = np.abs(blk).max()
            sc = scale[row, b]
            assert abs(sc - peak / 127) <= peak / 127 * 1e-3
            qq = q[row, b * 32:(b + 1) * 32].astype(np.float32)
            assert np.all(np.abs(qq) <= 127)
            assert np.all(np.abs(qq * sc - blk) <= sc * 0.5 + 1e-6)


def test_a_zero_block_has_a_zero_scale():
    # BlockQuantizerTests.AZeroBlockHasAZeroScale (:52-61)
    values = np.zeros((2, 32), np.float32)
    values.reshape(-1)[40] = 1e-9
    q, s = oracle.quantize(values, 2)
    assert np.all(s == 0) and np.all(q == 0)


def test_refuses_a_shape_that_does_not_tile():
    # BlockQuantizerTests.RefusesAShapeThatDoesNotTile (:63-68)
    with pytest.raises(ValueError):
        oracle.quantize(np.zeros((1, 48), np.float32), 1)


def test_per_channel_fp32_scales_are_the_block_rule_with_one_block():
    w = r(3, 8, 64, spread=2)
    q, s = oracle.quantize(w, 8, block=64, fp16_scales=False)
    peak = np.abs(w).max(axis=1)
    assert np.array_equal(s[:, 0], (peak / np.float32(127)).astype(np.float32))
    assert np.array_equal(q, np.clip(np.rint(w * (np.float32(1) / s)), -127, 127).astype(np.int8))


def test_quantization_error_is_bounded_by_half_a_step():
    # NarrowingLossTests.QuantizationErrorIsBoundedByHalfAStep (:79-85)
    values = (np.random.default_rng(1).random((4, 64)) * 2 - 1).astype(np.float32)
    err, energy = oracle.quantization_loss(values, 4)
    assert 0 < math.sqrt(err / energy) < 1 / 127


# ---- CpuMath (CpuMathTests.cs) -----------------------------------------------------

def test_linear_reads_every_float_width_alike():
    # CpuMathTests.LinearReadsEveryFloatWidthAlike (:40-64): weights exact at
    # every width, so the product must match the plain sum to 1e-5.
    outer, inner, rows = 5, 8, 3
    weights = np.array([(i % 7 - 3) * 0.25 for i in range(outer * inner)], np.float32).reshape(outer, inner)
    x = np.sin(np.arange(rows * inner, dtype=np.float32)).reshape(rows, inner)
    bias = np.array([1, 2, 3, 4, 5], np.float32)
    expected = np.zeros((rows, outer), np.float32)
    for m in range(rows):
        for o in range(outer):
            s = np.float32(bias[o])
            for i in range(inner):
                s = np.float32(s + np.float32(x[m, i] * weights[o, i]))
            expected[m, o] = s
    for stored in (weights, weights.astype(np.float16).astype(np.float32),
                   oracle.f32_to_bf16_bits(weights).astype(np.uint32) << 16):
        w = stored if stored.dtype == np.float32 else stored.view(np.float32)
        assert np.allclose(oracle.linear(x, w, bias), expected, atol=1e-5, rtol=0)


def test_dot_uses_four_eight_lane_accumulators():
    # CpuMath.Dot (:311-335): the summation order is fixed; a shape whose
    # partial sums cancel catastrophically tells orders apart.
    n = 70
    a = np.ones(n, np.float32)
    b = np.zeros(n, np.float32)
    b[0], b[8], b[1] = 1e8, -1e8, 1.0  # lane 0 of s0 and of s1 cancel first
    assert oracle.dot(a, b) == 1.0
    x, y = r(5, 1000), r(6, 1000)
    assert abs(oracle.dot(x, y) - float(np.dot(x.astype(np.float64), y.astype(np.float64)))) < 1e-5


def test_linear_against_float64():
    x, w, b = r(1, 7, 96), r(2, 33, 96), r(3, 33)
    ref = x.astype(np.float64) @ w.astype(np.float64).T + b
    assert np.max(np.abs(oracle.linear(x, w, b) - ref)) < 1e-5


def test_layer_norm_and_rms_norm_closed_forms():
    x = r(4, 6, 40, spread=6) + 3
    w, b = r(5, 40) + 1, r(6, 40)
    xd = x.astype(np.float64)
    mean = xd.mean(1, keepdims=True)
    ln = (xd - mean) / np.sqrt(((xd - mean) ** 2).mean(1, keepdims=True) + 1e-5) * w + b
    assert np.max(np.abs(oracle.layer_norm(x, w, b, 1e-5) - ln)) < 1e-5
    rms = xd / np.sqrt((xd ** 2).mean(1, keepdims=True) + 1e-6) * w
    assert np.max(np.abs(oracle.rms_norm(x, w, 1e-6) - rms)) < 1e-5
    # A nearly constant row: the variance is a small difference of large
    # numbers, which the double accumulation keeps (CpuMath.cs:100-101).
    c = np.full((1, 64), 1000.0, np.float32)
    c[0, 0] += 0.5
    out = oracle.layer_norm(c, None, None, 1e-6)
    var = 0.25 * 63 / 64 ** 2
    assert abs(out[0, 0] - (0.5 * 63 / 64) / math.sqrt(var + 1e-6)) < 1e-5


def test_rms_norm_half_smoke_case():
    # SmokeTest.RmsNormHalf (:599-623), fp32 arithmetic
    data = r(5, 24, spread=3).reshape(6, 4)
    weight = np.array([0.5, 1, 1.5, 2], np.float32)
    exp = np.empty_like(data)
    for row in range(6):
        sq = float(np.sum(data[row].astype(np.float64) ** 2))
        scale = np.float32(1 / math.sqrt(sq / 4 + 1e-6))
        exp[row] = data[row] * scale * weight
    assert np.max(np.abs(oracle.rms_norm(data, weight, 1e-6) - exp)) < 1e-6


def test_rope_rotate_half_smoke_case():
    # SmokeTest.RotateHalf (:736-776): feature i pairs with i + dim/2.
    data = r(6, 3, 2, 4, spread=2).reshape(3, 8)
    angles = r(7, 6, spread=6).reshape(3, 2)
    out = oracle.rope(data, 2, np.cos(angles), np.sin(angles))
    exp = np.empty_like(data)
    for t in range(3):
        for h in range(2):
            o = h * 4
            for i in range(2):
                c, s = math.cos(angles[t, i]), math.sin(angles[t, i])
                exp[t, o + i] = data[t, o + i] * c - data[t, o + 2 + i] * s
                exp[t, o + 2 + i] = data[t, o + 2 + i] * c + data[t, o + i] * s
    assert np.max(np.abs(out - exp)) < 1e-5


def test_rope_tables_frequencies():
    c, s = oracle.rope_tables(5, 8, 10000.0)
    for m in range(5):
        for i in range(4):
            f = 1.0 / 10000.0 ** (2 * i / 8)
            assert abs(c[m, i] - math.cos(m * f)) < 1e-6 and abs(s[m, i] - math.sin(m * f)) < 1e-6


def _attention64(q, k, v, heads, allowed=None, add_mask=None):
    rows, width = q.shape
    d = width // heads
    out = np.zeros((rows, width))
    for h in range(heads):
        qs, ks, vs = (t[:, h * d:(h + 1) * d].astype(np.float64) for t in (q, k, v))
        sc = qs @ ks.T / math.sqrt(d)
        if allowed is not None:
            sc = np.where(allowed, sc, -np.inf)
        if add_mask is not None:
            sc = sc + add_mask
        sc = np.exp(sc - sc.max(1, keepdims=True))
        out[:, h * d:(h + 1) * d] = (sc / sc.sum(1, keepdims=True)) @ vs
    return out


def test_multihead_attention_smoke_case():
    # SmokeTest.MultiheadAttention (:337-385): 2 heads of 2 over 3 tokens.
    q, k, v = r(7, 3, 4), r(8, 3, 4), r(9, 3, 4)
    out = oracle.mha(q, k, v, 2)[0]
    assert np.max(np.abs(out - _attention64(q, k, v, 2))) < 1e-6
    assert np.max(np.abs(oracle.attention(q, k, v, 2, 2) - _attention64(q, k, v, 2))) < 1e-6


def test_masked_attention_smoke_cases():
    # SmokeTest.MaskedAttention (:387-485): the -10000 of DirectML equals
    # leaving the key out whenever a row keeps at least one key.
    q, k, v = r(11, 4, 4), r(12, 4, 4), r(13, 4, 4)
    causal = np.tril(np.ones((4, 4), np.int32))
    out = oracle.mha(q, k, v, 2, mask_kind=2, mask=causal.reshape(1, 1, 4, 4))[0]
    assert np.max(np.abs(out - _attention64(q, k, v, 2, allowed=causal.astype(bool)))) < 1e-6
    out = oracle.mha(q, k, v, 2, mask_kind=1, key_len=3)[0]
    allowed = np.tile(np.arange(4) < 3, (4, 1))
    assert np.max(np.abs(out - _attention64(q, k, v, 2, allowed=allowed))) < 1e-6
    # CpuMath.Attention's causal path agrees with the boolean table.
    assert np.max(np.abs(oracle.attention(q, k, v, 2, 2, causal=True) -
                         _attention64(q, k, v, 2, allowed=causal.astype(bool)))) < 1e-6


def test_fully_masked_row_is_the_shifted_softmax():
    # DmlOps.cs:483 adds -10000 rather than excluding keys: a row with
    # every key masked softmaxes the shifted scores, i.e. the unmasked row.
    q, k, v = r(14, 2, 4), r(15, 3, 4), r(16, 3, 4)
    none = np.zeros((2, 3), np.int32)
    out = oracle.mha(q[None], k[None], v[None], 1, mask_kind=2, mask=none.reshape(1, 1, 2, 3))[0]
    # fp32 scores near -10000 keep ~1e-3 of their resolution.
    assert np.all(np.isfinite(out))
    assert np.max(np.abs(out - _attention64(q, k, v, 1))) < 1e-3


def test_grouped_query_attention():
    # CpuMath.Attention (:196-248): query head h reads key head h / group.
    q, k, v = r(17, 5, 8), r(18, 6, 4), r(19, 6, 4)
    out = oracle.attention(q, k, v, 4, 2)
    kk = np.repeat(k.reshape(6, 2, 2), 2, axis=1).reshape(6, 8)
    vv = np.repeat(v.reshape(6, 2, 2), 2, axis=1).reshape(6, 8)
    assert np.max(np.abs(out - _attention64(q, kk, vv, 4))) < 1e-6


def test_activations():
    x = np.linspace(-6, 6, 241).astype(np.float32)
    xd = x.astype(np.float64)
    assert np.max(np.abs(oracle.silu(x) - xd / (1 + np.exp(-xd)))) < 1e-6
    erf = np.array([math.erf(v / math.sqrt(2)) for v in xd])
    # A&S 7.1.26: |error| <= 1.5e-7 of erf (CpuMath.cs:297-298).
    assert np.max(np.abs(oracle.gelu(x) - 0.5 * xd * (1 + erf))) < 6 * 1.5e-7 + 1e-6
    tanh_form = 0.5 * xd * (1 + np.tanh(math.sqrt(2 / math.pi) * (xd + 0.044715 * xd ** 3)))
    assert np.max(np.abs(oracle.gelu_tanh(x) - tanh_form)) < 2e-6
    assert np.max(np.abs(oracle.sigmoid(x) - 1 / (1 + np.exp(-xd)))) < 1e-6
    assert np.max(np.abs(oracle.tanh(x) - np.tanh(xd))) < 1e-6


# ---- Transformer and Qwen-Image inputs (TransformerInputsTests.cs) ------------------

def test_the_sinusoid_is_half_cosines_then_half_sines():
    # TransformerInputsTests.TheSinusoidIsHalfCosinesThenHalfSines (:21-33)
    assert list(oracle.sinusoid(0.0, 8)) == [1, 1, 1, 1, 0, 0, 0, 0]
    at1 = oracle.sinusoid(1.0, 8)
    assert abs(at1[0] - math.cos(1)) < 1e-6
    assert abs(at1[1] - math.cos(0.1)) < 1e-6
    assert abs(at1[4] - math.sin(1)) < 1e-6
    assert abs(at1[7] - math.sin(0.001)) < 1e-6


def test_qwen_rotary_tables_place_text_after_the_image():
    # TransformerInputsTests.QwenImagesRotaryTablesPlaceTextAfterTheImage (:37-69)
    rows, columns, text_length, context_rows = 2, 3, 5, 7
    c, s = oracle.qwen_rope_tables(rows, columns, text_length, context_rows)
    assert c.shape == (rows * columns + context_rows, 64)
    c, s = c.ravel(), s.ravel()
    assert abs(c[0] - math.cos(text_length)) < 1e-6
    assert s[rows * columns * 64] == 0
    assert abs(s[(rows * columns + 3) * 64] - math.sin(3)) < 1e-6
    assert abs(s[0 * 64 + 8] - math.sin(-1)) < 1e-6
    assert abs(s[columns * 64 + 8]) < 1e-6
    assert abs(s[0 * 64 + 36] - math.sin(-2)) < 1e-6
    assert abs(s[2 * 64 + 36]) < 1e-6
    p = rows * columns + 4
    assert abs(s[p * 64 + 8] - math.sin(4)) < 1e-6
    assert abs(s[p * 64 + 36] - math.sin(4)) < 1e-6


def test_the_causal_table_is_a_triangle_closed_over_the_padding():
    # TransformerInputsTests.TheCausalTableIsATriangleClosedOverThePadding (:150-162)
    # and the per-branch tables of :90-127.
    assert list(oracle.causal_table(1, 1)) == [1]
    assert list(oracle.causal_table(2, 4)) == [1, 0, 0, 0, 1, 1, 0, 0, 1, 1, 0, 0, 1, 1, 0, 0]
    assert list(oracle.causal_table(2, 3)) == [1, 0, 0, 1, 1, 0, 1, 1, 0]
    assert list(oracle.causal_table(3, 3)) == [1, 0, 0, 1, 1, 0, 1, 1, 1]


def test_mmdit_rope_tables_frame_at_zero_and_text_unrotated():
    c, s = oracle.mmdit_rope_tables(2, 3, 4)
    qc, qs = oracle.qwen_rope_tables(2, 3, 0, 4)
    assert np.array_equal(c[:6], qc[:6]) and np.array_equal(s[:6], qs[:6])
    assert np.all(c[6:] == 1) and np.all(s[6:] == 0)
    assert np.all(c[:6, :8] == 1)  # frame 0 never turns


# ---- norms, convolution, sampling (SmokeTest.cs) ------------------------------------

def test_group_norm_smoke_case():
    # SmokeTest.GroupNormalization (:208-239): [1, 4, 1, 3] as 2 groups.
    data = np.array([1, 2, 3, 4, 5, 6, 0, 0, 0, 1, 1, 4], np.float32).reshape(1, 4, 1, 3)
    out = oracle.group_norm(data, 2, eps=1e-5).ravel()
    exp = np.empty(12)
    flat = data.ravel().astype(np.float64)
    for g in range(2):
        blk = flat[g * 6:(g + 1) * 6]
        exp[g * 6:(g + 1) * 6] = (blk - blk.mean()) / math.sqrt(blk.var() + 1e-5)
    assert np.max(np.abs(out - exp)) < 1e-6


def test_group_norm_affine_and_silu():
    # SmokeTest.NormalizationVersion2's group norm with per-channel affine (:666-733).
    data = np.array([1, 2, 3, 4, 5, 6, 0, 0, 0, 1, 1, 4], np.float32).reshape(1, 4, 1, 3)
    gamma = np.array([0.5, 2, -1, 1.5], np.float32)
    beta = np.array([0, 1, -2, 0.25], np.float32)
    out = oracle.group_norm(data, 2, gamma, beta, 1e-5).ravel()
    flat = data.ravel().astype(np.float64)
    exp = np.empty(12)
    for g in range(2):
        blk = flat[g * 6:(g + 1) * 6]
        nrm = (blk - blk.mean()) / math.sqrt(blk.var() + 1e-5)
        for i in range(6):
            ch = g * 2 + i // 3
            exp[g * 6 + i] = nrm[i] * gamma[ch] + beta[ch]
    assert np.max(np.abs(out - exp)) < 1e-5
    s = oracle.group_norm(data, 2, gamma, beta, 1e-5, silu=True).ravel()
    assert np.max(np.abs(s - exp / (1 + np.exp(-exp)))) < 1e-5


def test_convolution_smoke_case():
    # SmokeTest.Convolution (:241-281): identity tap and a 3x3 box sum.
    x = np.arange(9, dtype=np.float32).reshape(1, 1, 3, 3)
    f = np.zeros((2, 1, 3, 3), np.float32)
    f[0, 0, 1, 1] = 1
    f[1] = 1
    out = oracle.conv2d(x, f, np.array([0.5, -1], np.float32), 1, 1, 1)
    assert np.array_equal(out[0, 0], x[0, 0] + 0.5)
    xp = np.pad(x[0, 0], 1)
    box = np.array([[xp[i:i + 3, j:j + 3].sum() for j in range(3)] for i in range(3)])
    assert np.array_equal(out[0, 1], box - 1)


def test_convolution_against_float64_with_stride_and_padding():
    x, f, b = r(21, 2, 3, 7, 6), r(22, 4, 3, 3, 3), r(23, 4)
    for stride, pad, pad_end in ((1, 1, 1), (2, 1, 1), (2, 0, 1), (1, 0, 0)):
        out = oracle.conv2d(x, f, b, stride, pad, pad_end)
        xp = np.pad(x.astype(np.float64), ((0, 0), (0, 0), (pad, pad_end + 3), (pad, pad_end + 3)))
        ho = (7 + pad + pad_end - 3) // stride + 1
        wo = (6 + pad + pad_end - 3) // stride + 1
        exp = np.zeros((2, 4, ho, wo))
        for oy in range(ho):
            for ox in range(wo):
                win = xp[:, :, oy * stride:oy * stride + 3, ox * stride:ox * stride + 3]
                exp[:, :, oy, ox] = np.einsum("nchw,ochw->no", win, f.astype(np.float64)) + b
        assert out.shape == exp.shape
        assert np.max(np.abs(out - exp)) < 1e-5


def test_join_upsample_slice_smoke_case():
    # SmokeTest.JoinSliceUpsample (:308-335)
    a = np.array([1, 2, 3, 4], np.float32).reshape(1, 1, 2, 2)
    b = np.array([5, 6, 7, 8], np.float32).reshape(1, 1, 2, 2)
    up = oracle.upsample_nearest(np.concatenate([a, b], 1), 2)[:, :, :3, :3]
    for ch, src in enumerate((a, b)):
        for y in range(3):
            for x in range(3):
                assert up[0, ch, y, x] == src.ravel()[(y // 2) * 2 + x // 2]


def test_modulate_is_the_mixed_precision_blocks_norm():
    # SmokeTest.MixedPrecisionBlock (:778-813): LN(x) * 1.5 + shift is
    # Modulate with scale 0.5.
    x = r(9, 3, 4, spread=4)
    shift = r(10, 4)
    out = oracle.modulate(x, shift, np.full(4, 0.5, np.float32), 1e-6)
    xd = x.astype(np.float64)
    exp = (xd - xd.mean(1, keepdims=True)) / np.sqrt(xd.var(1, keepdims=True) + 1e-6) * 1.5 + shift
    assert np.max(np.abs(out - exp)) < 1e-5


# ---- the MMDiT block composition ----------------------------------------------------

def _tiny_block(seed=0, D=64, H=2, F=96, ni=6, nt=4, T=64):
    g = np.random.default_rng(seed)

    def w(*s, sc=0.2):
        return (g.standard_normal(s) * sc).astype(np.float32)

    def stream():
        d = D // H
        return dict(w_mod=w(6 * D, T), b_mod=w(6 * D), w_qkv=w(3 * D, D), b_qkv=w(3 * D),
                    norm_q=1 + w(d, sc=0.1), norm_k=1 + w(d, sc=0.1), w_o=w(D, D), b_o=w(D),
                    w_fc1=w(F, D), b_fc1=w(F), w_fc2=w(D, F), b_fc2=w(D))

    return w(ni, D, sc=1), w(nt, D, sc=1), w(T, sc=1), stream(), stream()


def _block64(xi, xt, temb, img, txt, H, cos, sin, eps=1e-6):
    """The A14 composition in float64 numpy, written independently of the C."""
    f = lambda a: np.asarray(a, np.float64)
    D = xi.shape[1]
    d = D // H
    st = f(temb) / (1 + np.exp(-f(temb)))
    xs = [f(xi).copy(), f(xt).copy()]
    ws = [img, txt]
    mods, qs, ks, vs = [], [], [], []

    def ln(x):
        m = x.mean(1, keepdims=True)
        return (x - m) / np.sqrt(((x - m) ** 2).mean(1, keepdims=True) + eps)

    def rms(x, w):
        return x / np.sqrt((x ** 2).mean(-1, keepdims=True) + eps) * w

    for x, w in zip(xs, ws):
        mod = f(w["w_mod"]) @ st + f(w["b_mod"])
        mods.append(mod.reshape(6, D))
        h = ln(x) * (1 + mods[-1][1]) + mods[-1][0]
        qkv = h @ f(w["w_qkv"]).T + f(w["b_qkv"])
        n = x.shape[0]
        qs.append(rms(qkv[:, :D].reshape(n, H, d), f(w["norm_q"])).reshape(n, D))
        ks.append(rms(qkv[:, D:2 * D].reshape(n, H, d), f(w["norm_k"])).reshape(n, D))
        vs.append(qkv[:, 2 * D:])
    q, k, v = (np.concatenate(t) for t in (qs, ks, vs))

    def rot(t):
        t = t.reshape(t.shape[0], H, d).copy()
        lo, hi = t[..., :d // 2].copy(), t[..., d // 2:].copy()
        c, s = f(cos)[:, None, :], f(sin)[:, None, :]
        t[..., :d // 2] = lo * c - hi * s
        t[..., d // 2:] = hi * c + lo * s
        return t.reshape(t.shape[0], D)

    a = _attention64(rot(q), rot(k), v, H)
    out, off = [], 0
    for x, w, mod in zip(xs, ws, mods):
        n = x.shape[0]
        x = x + mod[2] * (a[off:off + n] @ f(w["w_o"]).T + f(w["b_o"]))
        h = ln(x) * (1 + mod[4]) + mod[3]
        u = h @ f(w["w_fc1"]).T + f(w["b_fc1"])
        u = 0.5 * u * (1 + np.tanh(math.sqrt(2 / math.pi) * (u + 0.044715 * u ** 3)))
        x = x + mod[5] * (u @ f(w["w_fc2"]).T + f(w["b_fc2"]))
        out.append(x)
        off += n
    return out


def test_mmdit_block_against_float64_composition():
    xi, xt, temb, img, txt = _tiny_block()
    cos, sin = oracle.mmdit_rope_tables(2, 3, 4)
    cos, sin = cos[:, :16], sin[:, :16]  # head size 32: 16 pairs
    yi, yt = oracle.mmdit_block(xi, xt, temb, img, txt, 2, np.ascontiguousarray(cos), np.ascontiguousarray(sin))
    ei, et = _block64(xi, xt, temb, img, txt, 2, cos, sin)
    assert np.max(np.abs(yi - ei)) < 2e-4 * np.max(np.abs(ei))
    assert np.max(np.abs(yt - et)) < 2e-4 * np.max(np.abs(et))


def test_mmdit_block_invariants():
    xi, xt, temb, img, txt = _tiny_block(1)
    cos, sin = oracle.mmdit_rope_tables(2, 3, 4)
    cos, sin = np.ascontiguousarray(cos[:, :16]), np.ascontiguousarray(sin[:, :16])
    # Zero gates (the gate rows of the modulation) leave both streams alone.
    for s in (img, txt):
        for chunk in (2, 5):
            s["w_mod"][chunk * 64:(chunk + 1) * 64] = 0
            s["b_mod"][chunk * 64:(chunk + 1) * 64] = 0
    yi, yt = oracle.mmdit_block(xi, xt, temb, img, txt, 2, cos, sin)
    assert np.array_equal(yi, xi) and np.array_equal(yt, xt)
    # Attention is permutation-equivariant: permuting the image tokens with
    # their rotary rows permutes the result (no mask, no positions lost).
    xi, xt, temb, img, txt = _tiny_block(2)
    perm = np.array([3, 0, 5, 1, 4, 2])
    yi, yt = oracle.mmdit_block(xi, xt, temb, img, txt, 2, cos, sin)
    cp = np.concatenate([cos[:6][perm], cos[6:]])
    sp = np.concatenate([sin[:6][perm], sin[6:]])
    pi, pt = oracle.mmdit_block(xi[perm], xt, temb, img, txt, 2, np.ascontiguousarray(cp), np.ascontiguousarray(sp))
    assert np.max(np.abs(pi - yi[perm])) < 1e-5 and np.max(np.abs(pt - yt)) < 1e-5


# ---- Anima (Models/Anima/AnimaDit.cs) ------------------------------------------------

def test_anima_rotary_tables_leave_the_temporal_pairs_still():
    # TransformerInputsTests.AnimasRotaryTablesLeaveTheTemporalPairsStill (:67-83).
    c, s = oracle.anima_rope_tables(2, 2, 128)
    assert c.shape == (4, 64)
    assert np.all(c[:, :22] == 1) and np.all(s[:, :22] == 0)
    assert abs(s[2, 22] - math.sin(1.0)) <= 1e-6, "row 1, column 0"
    assert abs(s[1, 22 + 21] - math.sin(1.0)) <= 1e-6, "row 0, column 1"
    assert s[1, 22] == 0, "row 0 does not turn with the row"


def test_anima_rotary_frequencies_carry_the_ntk_factor():
    # 21 pairs per spatial axis at 1 / theta^(2k/42), theta = 10000 * 4^(42/40).
    c, s = oracle.anima_rope_tables(5, 7, 128)
    theta = 10000.0 * 4.0 ** (42 / 40)
    freq = 1.0 / theta ** (2.0 * np.arange(21) / 42)
    i, j = 3, 5
    tok = i * 7 + j
    assert np.allclose(c[tok, 22:43], np.cos(i * freq), atol=2e-6)
    assert np.allclose(s[tok, 43:64], np.sin(j * freq), atol=2e-6)
    # A head of 64 features: 20 per spatial axis, 24 temporal.
    c64, s64 = oracle.anima_rope_tables(2, 2, 64)
    assert c64.shape == (4, 32) and np.all(c64[:, :12] == 1) and abs(s64[2, 12] - math.sin(1.0)) <= 1e-6


def test_anima_patch_layouts_against_numpy_transposes():
    C, H, W = 16, 6, 8
    lat = r(40, C, H, W)
    # Patchify: feature c*4 + m*2 + n (AnimaDit.cs:193-219).
    exp = lat.reshape(C, H // 2, 2, W // 2, 2).transpose(1, 3, 0, 2, 4).reshape(-1, C * 4)
    assert np.array_equal(oracle.anima_patchify(lat), exp)
    # Unpatchify: feature (p1*2 + p2)*16 + c (AnimaDit.cs:223-247).
    tok = r(41, (H // 2) * (W // 2), C * 4)
    exp = tok.reshape(H // 2, W // 2, 2, 2, C).transpose(4, 0, 2, 1, 3).reshape(C, H, W)
    assert np.array_equal(oracle.anima_unpatchify(tok, C, H, W), exp)


def _tiny_anima(seed, D=64, heads=2, F=128, R=16, Cw=32, n=6, nc=5):
    g = np.random.default_rng(seed)

    def w(*shape, s=0.2):
        return (g.standard_normal(shape) * s).astype(np.float32)

    p = "blocks.0"
    ws = {}
    for part in ("self_attn", "cross_attn", "mlp"):
        ws[f"{p}.adaln_modulation_{part}.1.weight"] = w(R, D)
        ws[f"{p}.adaln_modulation_{part}.2.weight"] = w(3 * D, R)
    for a, src in (("self_attn", D), ("cross_attn", Cw)):
        ws[f"{p}.{a}.q_proj.weight"] = w(D, D)
        ws[f"{p}.{a}.k_proj.weight"] = w(D, src)
        ws[f"{p}.{a}.v_proj.weight"] = w(D, src)
        ws[f"{p}.{a}.output_proj.weight"] = w(D, D)
        ws[f"{p}.{a}.q_norm.weight"] = 1 + w(D // heads, s=0.1)
        ws[f"{p}.{a}.k_norm.weight"] = 1 + w(D // heads, s=0.1)
    ws[f"{p}.mlp.layer1.weight"] = w(F, D)
    ws[f"{p}.mlp.layer2.weight"] = w(D, F)
    x, temb, lora, ctx = w(n, D, s=1), w(D, s=1), w(3 * D, s=0.5), w(nc, Cw, s=1)
    cos, sin = oracle.anima_rope_tables(2, 3, D // heads)
    return ws, x, temb, lora, ctx, cos, sin


def test_anima_block_invariants():
    D = 64
    ws, x, temb, lora, ctx, cos, sin = _tiny_anima(1)
    # Zero modulation: every gate is 0 and the block is the identity.
    z = {k: (np.zeros_like(v) if ".2.weight" in k and "adaln" in k else v) for k, v in ws.items()}
    y = oracle.anima_block(x, temb, np.zeros_like(lora), ctx, z, 0, 2, cos, sin)
    assert np.array_equal(y, x)
    # The shared term alone: with W2 = 0 the modulation rows are the lora's.
    parts = oracle.anima_modulation(temb, lora, ws["blocks.0.adaln_modulation_mlp.1.weight"],
                                    np.zeros((3 * D, 16), np.float32), 3, D)
    assert all(np.array_equal(parts[i], lora[i * D:(i + 1) * D]) for i in range(3))
    two = oracle.anima_modulation(temb, lora, ws["blocks.0.adaln_modulation_mlp.1.weight"],
                                  np.zeros((2 * D, 16), np.float32), 2, D)
    assert np.array_equal(two[1], lora[D:2 * D])
    # Cross-attention reads the context as keys: permuting its rows changes nothing.
    y = oracle.anima_block(x, temb, lora, ctx, ws, 0, 2, cos, sin)
    yp = oracle.anima_block(x, temb, lora, ctx[[3, 1, 4, 0, 2]], ws, 0, 2, cos, sin)
    assert np.max(np.abs(y - yp)) < 1e-5
    # Self-attention is equivariant: permuting the tokens with their rotary
    # rows permutes the result.
    perm = np.array([4, 0, 5, 2, 1, 3])
    yq = oracle.anima_block(x[perm], temb, lora, ctx, ws, 0, 2, np.ascontiguousarray(cos[perm]),
                            np.ascontiguousarray(sin[perm]))
    assert np.max(np.abs(yq - y[perm])) < 1e-5


def test_anima_mlp_branch_is_exact_gelu():
    """Only the MLP's gate open (1) and shift/scale 0: x + W2 GELU(W1 LN(x)),
    checked in float64 with scipy's erf, which tells the exact GELU from the
    tanh form."""
    from scipy.special import erf
    D = 64
    ws, x, temb, lora, ctx, cos, sin = _tiny_anima(2)
    for part in ("self_attn", "cross_attn", "mlp"):
        ws[f"blocks.0.adaln_modulation_{part}.2.weight"][:] = 0
    lora = np.zeros(3 * D, np.float32)
    # The parts share the lora: a gate of 1 for all three, then close the
    # attention branches by zeroing their output projections.
    lora[2 * D:3 * D] = 1
    ws["blocks.0.self_attn.output_proj.weight"][:] = 0
    ws["blocks.0.cross_attn.output_proj.weight"][:] = 0
    y = oracle.anima_block(x, temb, lora, ctx, ws, 0, 2, cos, sin)
    xd = x.astype(np.float64)
    ln = (xd - xd.mean(1, keepdims=True)) / np.sqrt(xd.var(1, keepdims=True) + 1e-6)
    h = ln @ ws["blocks.0.mlp.layer1.weight"].astype(np.float64).T
    f = 0.5 * h * (1 + erf(h / np.sqrt(2)))
    exp = xd + f @ ws["blocks.0.mlp.layer2.weight"].astype(np.float64).T
    assert np.max(np.abs(y - exp)) < 2e-5 * np.max(np.abs(exp - xd))
