"""The per-layer builder API: Layers (Graph/Layers.cs) and Transformer
(Graph/Transformer.cs), emitting nodes of the HIP graph.

Same names, argument meaning and errors as the reference. Where the
reference composes several DirectML operators that the MI355X path runs as
one kernel (the modulated LayerNorm, the head norm with the rotation, the
gated residual after a projection), the fused operator is used and the
composition it replaces is cited.
"""

from __future__ import annotations

import math
from typing import Optional, Union

import numpy as np

from ._lib import ArgumentError
from .graph import (EPI_GATED_RESIDUAL, EPI_GELU, EPI_GELU_TANH, EPI_NONE, EPI_RESIDUAL, EPI_SILU, EPI_SWIGLU,
                    Expression,
                    MaskType, ModelBuilder, Ops)
from .tensors import HostDataType, HostTensor

WeightLike = Union[HostTensor, Expression]


class Layers:
    """Graph/Layers.cs:11."""

    @staticmethod
    def Broadcast(expression: Expression, shape) -> Expression:
        """Layers.Broadcast (:15-53): view as shape, repeating size-1 axes."""
        source = list(expression.Shape)
        shape = [int(s) for s in shape]
        if source == shape:
            return expression
        if len(source) != len(shape):
            raise ArgumentError(f"cannot broadcast {source} to {shape}: rank differs")
        packed = [1] * len(source)
        for i in range(len(source) - 2, -1, -1):
            packed[i] = packed[i + 1] * source[i + 1]
        strides = []
        for i in range(len(source)):
            if source[i] == shape[i]:
                strides.append(packed[i])
            elif source[i] == 1:
                strides.append(0)
            else:
                raise ArgumentError(f"cannot broadcast {source} to {shape}")
        return Ops.Reinterpret(expression, shape, strides)

    @staticmethod
    def ToTokens(expression: Expression) -> Expression:
        """[N, C, H, W] viewed as [N, 1, H*W, C] (:56-64)."""
        n, c, h, w = expression.Shape
        return Ops.Reinterpret(expression, [n, 1, h * w, c], [c * h * w, c * h * w, 1, h * w])

    @staticmethod
    def ToImage(expression: Expression, height: int, width: int) -> Expression:
        """The inverse of ToTokens (:67-77)."""
        n, _, tokens, c = expression.Shape
        if tokens != height * width:
            raise ArgumentError(f"{tokens} tokens do not fill {height}x{width}")
        return Ops.Reinterpret(expression, [n, c, height, width], [c * tokens, 1, width * c, c])

    @staticmethod
    def ToChannels(expression: Expression) -> Expression:
        s = expression.Shape
        return Ops.Reinterpret(expression, [s[0], s[3], 1, 1])

    @staticmethod
    def Silu(x: Expression) -> Expression:
        return Ops.ActivationSwish(x)

    @staticmethod
    def _constant_type(x: Expression) -> HostDataType:
        """Layers.ConstantType (:96-97): constants at the activation's width."""
        return x.DataType

    @staticmethod
    def _weight(model: ModelBuilder, weight: WeightLike, shape, rows: int) -> Expression:
        if isinstance(weight, Expression):
            return weight
        return model.Weight(weight, shape, rows)

    @staticmethod
    def Conv2d(model: ModelBuilder, x: Expression, weight: WeightLike, bias: Optional[WeightLike], stride: int = 1,
               padding: int = 1, endPadding: Optional[int] = None, residual: Optional[Expression] = None):
        """Layers.Conv2d (:115-127): torch [out, in, kh, kw] filters; residual
        (an addition after the convolution) is fused."""
        if isinstance(weight, HostTensor):
            filters = model.Weight(weight, weight.Shape, weight.Shape[0])
        else:
            filters = weight
        biases = None
        if bias is not None:
            biases = bias if isinstance(bias, Expression) else model.Constant(
                bias, [bias.ElementCount], Layers._constant_type(x))
        end = padding if endPadding is None else endPadding
        return Ops.Convolution(x, filters, biases, [stride, stride], [padding, padding], [end, end], residual)

    @staticmethod
    def Linear(model: ModelBuilder, x: Expression, weight: WeightLike, bias: Optional[WeightLike] = None,
               activation: Optional[str] = None, gate: Optional[Expression] = None,
               residual: Optional[Expression] = None) -> Expression:
        """Layers.Linear (:131-160): y = x W^T (+ bias), torch [out, in]
        weights, the product at x's precision (a narrower weight is widened in
        the kernel), the weight shared across the batch.

        Fused tails: activation 'gelu_tanh' | 'gelu' | 'silu', or 'swiglu'
        (SiLU(gate) * up over a weight whose rows interleave the gate and up
        projections, QwenImageDit.cs:390-406; half the columns out); with
        residual, residual + Cast(y) (or residual + gate * Cast(y) with gate,
        the gated residual of QwenImageDit.cs:421,425), at the residual's
        precision."""
        if isinstance(weight, HostTensor):
            out_features, in_features = weight.Shape[0], weight.Shape[1]
            w = model.Weight(weight, [1, 1, out_features, in_features], out_features)
        else:
            w = weight
        b = None
        if bias is not None:
            b = bias if isinstance(bias, Expression) else model.Constant(bias, [bias.ElementCount],
                                                                         Layers._constant_type(x))
        epi = EPI_NONE
        if residual is not None:
            if activation is not None:
                raise ArgumentError("an activation and a residual do not fuse together")
            epi = EPI_GATED_RESIDUAL if gate is not None else EPI_RESIDUAL
        elif activation is not None:
            epi = {"gelu_tanh": EPI_GELU_TANH, "gelu": EPI_GELU, "silu": EPI_SILU, "swiglu": EPI_SWIGLU}[activation]
        return Ops.Linear(x, w, b, epi, gate, residual)

    @staticmethod
    def GroupNorm(model: ModelBuilder, x: Expression, weight: WeightLike, bias: WeightLike, groups: int,
                  epsilon: float, silu: bool = False) -> Expression:
        """Layers.GroupNorm (:166-185), with an optional SiLU fused after it."""
        c = x.Shape[1]
        if c % groups != 0:
            raise ArgumentError(f"{c} channels do not divide into {groups} groups")
        w = weight if isinstance(weight, Expression) else model.Constant(weight, [c], Layers._constant_type(x))
        b = bias if isinstance(bias, Expression) else model.Constant(bias, [c], Layers._constant_type(x))
        return Ops.GroupNorm(x, w, b, groups, epsilon, silu)

    @staticmethod
    def LayerNorm(*args):
        """LayerNorm(model, x, weight, bias, eps) with a per-feature affine
        (:189-197), or LayerNorm(x, eps) without one (:225-226)."""
        if len(args) == 2:
            x, eps = args
            return Ops.MeanVarianceNormalization(x, [len(x.Shape) - 1], eps)
        model, x, weight, bias, eps = args
        d = x.Shape[-1]
        w = weight if isinstance(weight, Expression) else model.Constant(weight, [d], Layers._constant_type(x))
        b = bias if isinstance(bias, Expression) else model.Constant(bias, [d], Layers._constant_type(x))
        return Ops.MeanVarianceNormalization2(x, [len(x.Shape) - 1], True, eps, w, b)

    @staticmethod
    def RmsNorm(model: ModelBuilder, x: Expression, weight: Optional[WeightLike], epsilon: float) -> Expression:
        """Layers.RmsNorm (:209-221): x / sqrt(mean(x^2) + eps) * weight."""
        axes = [len(x.Shape) - 1]
        if weight is None:
            return Ops.MeanVarianceNormalization2(x, axes, False, epsilon)
        w = weight if isinstance(weight, Expression) else model.Constant(weight, [x.Shape[-1]],
                                                                         Layers._constant_type(x))
        return Ops.MeanVarianceNormalization2(x, axes, False, epsilon, w)

    @staticmethod
    def Cast(x: Expression, dataType: HostDataType) -> Expression:
        return x if x.DataType == dataType else Ops.Cast(x, dataType)

    @staticmethod
    def UpsampleNearest(x: Expression, scale: int = 2) -> Expression:
        return Ops.Upsample2D(x, scale, scale)

    @staticmethod
    def CropTo(x: Expression, height: int, width: int) -> Expression:
        s = x.Shape
        if s[2] == height and s[3] == width:
            return x
        return Ops.Slice(x, [0, 0, 0, 0], [s[0], s[1], height, width], [1, 1, 1, 1])

    @staticmethod
    def Attend(query: Expression, key: Expression, value: Expression, heads: int, mask: Optional[Expression] = None,
               maskType: int = MaskType.NONE) -> Expression:
        """Layers.Attend (:260-279): scale 1/sqrt(d), one fused operator."""
        dim = query.Shape[-1] // heads
        return Ops.MultiheadAttention(query, key, value, heads, 1.0 / math.sqrt(dim), mask,
                                      maskType if mask is not None else MaskType.NONE)


class Transformer:
    """Graph/Transformer.cs:14."""

    @staticmethod
    def Sinusoid(time: float, width: int) -> np.ndarray:
        """Transformer.Sinusoid (:20-32): half cosines then half sines of
        t * 10000^(-i/half), in float32 (CPU side, like the reference)."""
        half = width // 2
        i = np.arange(half, dtype=np.float32)
        freq = np.exp(np.float32(-math.log(10000.0)) * i / np.float32(half), dtype=np.float32)
        angle = (np.float32(time) * freq).astype(np.float32)
        return np.concatenate([np.cos(angle), np.sin(angle)]).astype(np.float32)

    @staticmethod
    def HeadNorm(model: ModelBuilder, x: Expression, weight: WeightLike, heads: int, headDim: int,
                 epsilon: float) -> Expression:
        """Transformer.HeadNorm (:37-43): [1, 1, T, W] viewed as [1, T, H, d]."""
        tokens = x.Shape[2]
        view = Ops.Reinterpret(x, [1, tokens, heads, headDim])
        return Layers.RmsNorm(model, view, weight, epsilon)

    @staticmethod
    def Rotate(heads: Expression, cos: Expression, sin: Expression, headCount: int, headDim: int,
               compute: HostDataType) -> Expression:
        """Transformer.Rotate (:50-64): the rotate-half rotation in fp32."""
        shape = heads.Shape
        half = headDim // 2
        wide = Layers.Cast(heads, HostDataType.Float32)

        def Half(offset):
            return Ops.Slice(wide, [0, 0, 0, offset], [1, shape[1], headCount, half], [1, 1, 1, 1])

        half_shape = [1, shape[1], headCount, half]
        c = Layers.Broadcast(cos, half_shape)
        s = Layers.Broadcast(sin, half_shape)
        low, high = Half(0), Half(half)
        rotated = Ops.Join([low * c - high * s, high * c + low * s], 3)
        return Layers.Cast(rotated, compute)

    @staticmethod
    def HeadNormRotate(model: ModelBuilder, x: Expression, weight: WeightLike, heads: int, epsilon: float,
                       cos: Optional[Expression], sin: Optional[Expression], compute: HostDataType) -> Expression:
        """HeadNorm then Rotate as one kernel, on the packed [.., T, H*d]
        projection (the reference's Flat(Rotate(HeadNorm(x))), :37-68)."""
        d = x.Shape[-1] // heads
        w = None
        if weight is not None:
            w = weight if isinstance(weight, Expression) else model.Constant(weight, [d], x.DataType)
        return Ops.HeadNormRotate(x, w, epsilon, cos, sin, heads, compute)

    @staticmethod
    def Flat(heads: Expression, width: int) -> Expression:
        """[1, T, H, d] back to [1, 1, T, W] (:67-68)."""
        return Ops.Reinterpret(heads, [1, 1, heads.Shape[1], width])

    @staticmethod
    def Modulate(x: Expression, *args) -> Expression:
        """Transformer.Modulate (:72-80): Cast(LayerNorm(x) * (1 + scale) +
        shift, compute) as one kernel. Modulate(x, scale, eps, compute) or
        Modulate(x, shift, scale, eps, compute); scale and shift are rows
        broadcast over the tokens."""
        if len(args) == 3:
            scale, eps, compute = args
            shift = None
        else:
            shift, scale, eps, compute = args
        return Ops.Modulate(x, shift, scale, eps, compute)
