"""The expression graph, its operators and the model builder.

Mirrors Dml/DmlGraph.cs + Dml/DmlExpression.cs (Graph, Expression and its
arithmetic operators), Dml/DmlOps.cs (Ops: each function adds one node and
the library computes the output shape), Dml/DmlCompiledModel.cs
(CompiledModel) and Graph/ModelBuilder.cs (ModelBuilder), over the C ABI.
Every operator runs in libndx.so on the GPU.
"""

from __future__ import annotations

import contextlib
import ctypes
from typing import Optional, Sequence

import numpy as np

from . import _lib
from ._lib import ArgumentError, InvalidOperationError, UnsupportedError, call
from .tensors import Device, DeviceTensor, HostDataType, HostTensor

NONE = -1

# ndx.h enums
UNARY_IDENTITY, UNARY_SIGMOID, UNARY_SILU, UNARY_GELU, UNARY_TANH, UNARY_GELU_TANH = range(6)
BIN_ADD, BIN_SUB, BIN_MUL, BIN_DIV = range(4)
EPI_NONE, EPI_GELU_TANH, EPI_GELU, EPI_SILU, EPI_GATED_RESIDUAL, EPI_RESIDUAL, EPI_SWIGLU = range(7)
PATCH_CHANNEL_FIRST, PATCH_CHANNEL_LAST = 0, 1  # feature order (c, dy, dx) or (dy, dx, c)


class MaskType:
    """MultiheadAttentionMaskType as the graphs use it."""
    NONE = 0
    KeySequenceLength = 1
    Boolean = 2


class Graph:
    """A graph under construction (DmlGraph, Dml/DmlGraph.cs:9). device may
    be None: the graph then infers shapes only."""

    def __init__(self, device: Optional[Device], dataType: HostDataType = HostDataType.Float32,
                 int8Weights: bool = False):
        h = ctypes.c_void_p()
        call("ndx_graph_create", device.handle if device else None, int(dataType), int(int8Weights),
             ctypes.byref(h))
        self._h = h
        self.Device = device
        self.DataType = HostDataType(dataType)

    @property
    def handle(self):
        return self._h

    def _new(self, fn: str, *args) -> "Expression":
        out = ctypes.c_int32()
        call(fn, self._h, *args, ctypes.byref(out))
        return Expression(self, out.value)

    def Input(self, dataType: HostDataType, sizes: Sequence[int]) -> "Expression":
        return self._new("ndx_graph_input", int(dataType), _lib.shape_array(sizes), len(sizes))

    def SetStream(self, stream: int) -> None:
        """The stream (0 or 1) operations emitted from now on run on."""
        call("ndx_graph_set_stream", self._h, int(stream))

    @contextlib.contextmanager
    def Stream(self, stream: int):
        """with graph.Stream(1): ... emits onto the second stream, then back to 0."""
        self.SetStream(stream)
        try:
            yield self
        finally:
            self.SetStream(0)

    def Dispose(self):
        if self._h is not None:
            call("ndx_graph_destroy", self._h)
            self._h = None

    def __del__(self):
        try:
            self.Dispose()
        except Exception:
            pass


def _id(x) -> int:
    return NONE if x is None else x.id


class Expression:
    """An input or the output of an operator node (DmlExpression,
    Dml/DmlExpression.cs:7), with the reference's operator overloads."""

    __slots__ = ("graph", "id")

    def __init__(self, graph: Graph, vid: int):
        self.graph = graph
        self.id = vid

    def _info(self):
        dt, rank = ctypes.c_int32(), ctypes.c_int32()
        shape = (ctypes.c_int64 * 4)()
        call("ndx_value_info", self.graph.handle, self.id, ctypes.byref(dt), shape, ctypes.byref(rank))
        return HostDataType(dt.value), tuple(shape[i] for i in range(rank.value))

    @property
    def Shape(self):
        return self._info()[1]

    @property
    def DataType(self) -> HostDataType:
        return self._info()[0]

    # DmlExpression.cs:37-51
    def __add__(self, o):
        return Ops.Add(self, o) if isinstance(o, Expression) else Ops.Identity(self, 1.0, float(o))

    def __radd__(self, o):
        return Ops.Identity(self, 1.0, float(o))

    def __sub__(self, o):
        return Ops.Subtract(self, o) if isinstance(o, Expression) else Ops.Identity(self, 1.0, -float(o))

    def __rsub__(self, o):
        return Ops.Identity(self, -1.0, float(o))

    def __mul__(self, o):
        return Ops.Multiply(self, o) if isinstance(o, Expression) else Ops.Identity(self, float(o), 0.0)

    def __rmul__(self, o):
        return Ops.Identity(self, float(o), 0.0)

    def __truediv__(self, o):
        return Ops.Divide(self, o) if isinstance(o, Expression) else Ops.Identity(self, 1.0 / float(o), 0.0)

    def __neg__(self):
        return Ops.Identity(self, -1.0, 0.0)

    def __repr__(self):
        dt, shape = self._info()
        return f"<expression {self.id}: {dt.name} {list(shape)}>"


class Ops:
    """Dml/DmlOps.cs: one node per call; output shapes come from the library."""

    @staticmethod
    def _same_graph(*xs):
        g = None
        for x in xs:
            if x is None:
                continue
            if g is None:
                g = x.graph
            elif x.graph is not g:
                raise InvalidOperationError("expression belongs to a different graph")
        return g

    @staticmethod
    def Add(a, b):
        return Ops._same_graph(a, b)._new("ndx_op_binary", a.id, b.id, BIN_ADD)

    @staticmethod
    def Subtract(a, b):
        return Ops._same_graph(a, b)._new("ndx_op_binary", a.id, b.id, BIN_SUB)

    @staticmethod
    def Multiply(a, b):
        return Ops._same_graph(a, b)._new("ndx_op_binary", a.id, b.id, BIN_MUL)

    @staticmethod
    def Divide(a, b):
        return Ops._same_graph(a, b)._new("ndx_op_binary", a.id, b.id, BIN_DIV)

    @staticmethod
    def Identity(x, scale=1.0, bias=0.0):
        return x.graph._new("ndx_op_scale_bias", x.id, float(scale), float(bias))

    @staticmethod
    def Cast(x, dataType: HostDataType):
        return x.graph._new("ndx_op_cast", x.id, int(dataType))

    @staticmethod
    def ActivationSigmoid(x):
        return x.graph._new("ndx_op_unary", x.id, UNARY_SIGMOID)

    @staticmethod
    def ActivationSwish(x):
        return x.graph._new("ndx_op_unary", x.id, UNARY_SILU)

    @staticmethod
    def ActivationGelu(x):
        return x.graph._new("ndx_op_unary", x.id, UNARY_GELU)

    @staticmethod
    def ActivationTanh(x):
        return x.graph._new("ndx_op_unary", x.id, UNARY_TANH)

    @staticmethod
    def ActivationIdentity(x):
        return x.graph._new("ndx_op_unary", x.id, UNARY_IDENTITY)

    @staticmethod
    def ActivationGeluTanh(x):
        return x.graph._new("ndx_op_unary", x.id, UNARY_GELU_TANH)

    @staticmethod
    def Reinterpret(x, sizes, strides=None):
        st = None if strides is None else _lib.shape_array(strides)
        if strides is not None and len(strides) != len(sizes):
            raise ArgumentError("sizes and strides differ in rank")
        return x.graph._new("ndx_op_reinterpret", x.id, _lib.shape_array(sizes), len(sizes), st)

    @staticmethod
    def Slice(x, offsets, sizes, strides=None):
        rank = len(x.Shape)
        if len(offsets) != rank or len(sizes) != rank or (strides is not None and len(strides) != rank):
            raise _lib.ArgumentError(f"a slice of a rank-{rank} tensor takes {rank} offsets, sizes and strides")
        st = None if strides is None else _lib.shape_array(strides)
        return x.graph._new("ndx_op_slice", x.id, _lib.shape_array(offsets), _lib.shape_array(sizes), st)

    @staticmethod
    def Join(inputs, axis: int):
        g = Ops._same_graph(*inputs)
        ids = (ctypes.c_int32 * len(inputs))(*[x.id for x in inputs])
        return g._new("ndx_op_join", ids, len(inputs), axis)

    @staticmethod
    def Gemm(a, b, c=None, transA=False, transB=False, alpha=1.0, beta=1.0):
        g = Ops._same_graph(a, b, c)
        return g._new("ndx_op_gemm", a.id, b.id, _id(c), int(transA), int(transB), float(alpha), float(beta))

    @staticmethod
    def Convolution(x, filter, bias, strides, startPadding, endPadding, residual=None):
        if strides[0] != strides[1] or startPadding[0] != startPadding[1] or endPadding[0] != endPadding[1]:
            raise UnsupportedError("square strides and paddings only")
        g = Ops._same_graph(x, filter, bias, residual)
        return g._new("ndx_op_conv2d", x.id, filter.id, _id(bias), int(strides[0]), int(startPadding[0]),
                      int(endPadding[0]), _id(residual))

    @staticmethod
    def MeanVarianceNormalization(x, axes, epsilon):
        """MVN1 (Dml/DmlOps.cs:305-319): over the last axis it is LayerNorm;
        over axes {2, 3} of [N, C, H, W] each (n, c) plane on its own."""
        rank = len(x.Shape)
        axes = sorted(a % rank for a in axes)
        if axes == [rank - 1]:
            return x.graph._new("ndx_op_layer_norm", x.id, NONE, NONE, float(epsilon))
        if rank == 4 and axes == [2, 3]:
            c = x.Shape[1]
            return x.graph._new("ndx_op_group_norm", x.id, NONE, NONE, int(c), float(epsilon), 0)
        raise UnsupportedError(f"mean-variance normalization over axes {axes}")

    @staticmethod
    def MeanVarianceNormalization2(x, axes, useMean, epsilon, scale=None, bias=None):
        """MVN2 (Dml/DmlOps.cs:327-342): useMean False over the last axis is
        RMSNorm (scale over that axis); useMean True over {2, 3} of [N, G,
        C/G, HW] with a [1, G, C/G, 1] affine is GroupNorm."""
        rank = len(x.Shape)
        axes = sorted(a % rank for a in axes)
        g = Ops._same_graph(x, scale, bias)
        if not useMean and axes == [rank - 1] and bias is None:
            return g._new("ndx_op_rms_norm", x.id, _id(scale), float(epsilon))
        if useMean and axes == [rank - 1]:
            return g._new("ndx_op_layer_norm", x.id, _id(scale), _id(bias), float(epsilon))
        if useMean and rank == 4 and axes == [2, 3]:
            n, groups, per, hw = x.Shape
            flat = Ops.Reinterpret(x, [n, groups * per, 1, hw])
            w = None if scale is None else Ops.Reinterpret(scale, [groups * per])
            b = None if bias is None else Ops.Reinterpret(bias, [groups * per])
            y = g._new("ndx_op_group_norm", flat.id, _id(w), _id(b), int(groups), float(epsilon), 0)
            return Ops.Reinterpret(y, [n, groups, per, hw])
        raise UnsupportedError(f"mean-variance normalization 2 over axes {axes}")

    @staticmethod
    def Upsample2D(x, scaleWidth, scaleHeight):
        if scaleWidth != scaleHeight:
            raise UnsupportedError("square nearest upsampling only")
        return x.graph._new("ndx_op_upsample_nearest", x.id, int(scaleWidth))

    @staticmethod
    def MultiheadAttention(query, key, value, headCount, scale, mask=None, maskType=MaskType.NONE):
        if (mask is None) != (maskType == MaskType.NONE):
            raise ArgumentError("a mask and its type come together")
        g = Ops._same_graph(query, key, value, mask)
        return g._new("ndx_op_attention", query.id, key.id, value.id, int(headCount), float(scale), int(maskType),
                      _id(mask))

    # ---- fused layer operators (no single DmlOps counterpart) -----------------

    @staticmethod
    def Linear(x, w, bias=None, epilogue=EPI_NONE, gate=None, residual=None):
        g = Ops._same_graph(x, w, bias, gate, residual)
        return g._new("ndx_op_linear", x.id, w.id, _id(bias), int(epilogue), _id(gate), _id(residual))

    @staticmethod
    def HeadNormRotate(x, weight, epsilon, cos, sin, heads, outType):
        g = Ops._same_graph(x, weight, cos, sin)
        return g._new("ndx_op_head_norm_rotate", x.id, _id(weight), float(epsilon), _id(cos), _id(sin), int(heads),
                      int(outType))

    @staticmethod
    def Modulate(x, shift, scale, epsilon, outType):
        g = Ops._same_graph(x, shift, scale)
        return g._new("ndx_op_modulate", x.id, _id(shift), scale.id, float(epsilon), int(outType))

    @staticmethod
    def GroupNorm(x, weight, bias, groups, epsilon, silu=False):
        g = Ops._same_graph(x, weight, bias)
        return g._new("ndx_op_group_norm", x.id, _id(weight), _id(bias), int(groups), float(epsilon), int(silu))

    @staticmethod
    def GuidedEulerStep(x, uncond, cond, scalars):
        """ndx_op_guided_euler_step: x + (u + g (c - u)) (sigma_next - sigma),
        scalars = (g, sigma, sigma_next); uncond may be None (no guidance)."""
        g = Ops._same_graph(x, uncond, cond, scalars)
        return g._new("ndx_op_guided_euler_step", x.id, _id(uncond), cond.id, scalars.id)

    @staticmethod
    def ActivationSoftmax(x, scale: float = 1.0):
        """DmlOps.ActivationSoftmax over the last axis (Dml/DmlOps.cs:175-184)
        of scale * x (scale: the alpha of the Gemm that made x)."""
        return x.graph._new("ndx_op_softmax", x.id, float(scale))

    @staticmethod
    def Patchify(x, patch, order=PATCH_CHANNEL_FIRST):
        return x.graph._new("ndx_op_patchify", x.id, int(patch), int(order))

    @staticmethod
    def Unpatchify(x, patch, channels, height, width, order=PATCH_CHANNEL_FIRST):
        return x.graph._new("ndx_op_unpatchify", x.id, int(patch), int(channels), int(height), int(width),
                            int(order))


class CompiledModel:
    """A compiled graph with its weights on the device (DmlCompiledModel,
    Dml/DmlCompiledModel.cs:10)."""

    # The static scratch of DispatchIntoStatic (NDX_STATIC_SCRATCH_BYTES).
    STATIC_SCRATCH_BYTES = 64 << 20

    def __init__(self, graph: Graph, outputs: Sequence[Expression], device: Device):
        if graph.handle is None:
            raise InvalidOperationError("the graph was disposed")
        ids = (ctypes.c_int32 * len(outputs))(*[o.id for o in outputs])
        h = ctypes.c_void_p()
        call("ndx_graph_compile", graph.handle, ids, len(outputs), ctypes.byref(h))
        self._h = h
        self.Device = device
        n_in, n_out, kernels = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
        call("ndx_model_counts", h, ctypes.byref(n_in), ctypes.byref(n_out), ctypes.byref(kernels))
        self.InputCount, self.OutputCount, self.KernelCount = n_in.value, n_out.value, kernels.value

    @property
    def handle(self):
        if self._h is None:
            raise InvalidOperationError("the model was disposed")
        return self._h

    def _sizes(self):
        p, t = ctypes.c_uint64(), ctypes.c_uint64()
        call("ndx_model_sizes", self.handle, ctypes.byref(p), ctypes.byref(t))
        return p.value, t.value

    @property
    def PersistentSize(self) -> int:
        return self._sizes()[0]

    @property
    def TemporarySize(self) -> int:
        return self._sizes()[1]

    def DispatchOnDevice(self, inputs: Sequence[DeviceTensor]) -> list[DeviceTensor]:
        arr = (ctypes.c_void_p * max(len(inputs), 1))(*[t.handle for t in inputs])
        outs = (ctypes.c_void_p * self.OutputCount)()
        call("ndx_model_run", self.handle, arr, len(inputs), outs, self.OutputCount)
        return [DeviceTensor(self.Device, ctypes.c_void_p(o)) for o in outs]

    def DispatchInto(self, inputs: Sequence[DeviceTensor], outputs: Sequence[DeviceTensor]) -> None:
        """Queues one run into existing output tensors without waiting."""
        arr = (ctypes.c_void_p * max(len(inputs), 1))(*[t.handle for t in inputs])
        outs = (ctypes.c_void_p * len(outputs))(*[t.handle for t in outputs])
        call("ndx_model_run_into_async", self.handle, arr, len(inputs), outs, len(outputs))

    def DispatchIntoStatic(self, inputs: Sequence[DeviceTensor], outputs: Sequence[DeviceTensor]) -> None:
        """DispatchInto with the temporaries in the library's static scratch
        (ndx_model_run_into_static_async): allocates nothing; refuses a model
        whose TemporarySize exceeds STATIC_SCRATCH_BYTES."""
        arr = (ctypes.c_void_p * max(len(inputs), 1))(*[t.handle for t in inputs])
        outs = (ctypes.c_void_p * len(outputs))(*[t.handle for t in outputs])
        call("ndx_model_run_into_static_async", self.handle, arr, len(inputs), outs, len(outputs))

    def Dispatch(self, inputs: Sequence[HostTensor]) -> list[HostTensor]:
        device_in = [self.Device.Upload(t) for t in inputs]
        try:
            outs = self.DispatchOnDevice(device_in)
        finally:
            for t in device_in:
                t.Dispose()
        host = [o.Download() for o in outs]
        for o in outs:
            o.Dispose()
        return host

    def SetGraphReplay(self, enabled: bool) -> None:
        """Record DispatchInto's launches as one HIP graph and replay it while
        the same input and output tensors are bound (ndx_model_set_graph_replay)."""
        call("ndx_model_set_graph_replay", self.handle, int(enabled))

    def SetProfiling(self, enabled: bool, family: Optional[str] = None) -> None:
        """Per-kernel timing. family: bracket only that kernel family's
        launches, with no wait per run (for a timed region)."""
        call("ndx_model_set_profile_filter", self.handle, family.encode() if family else None)
        call("ndx_model_set_profiling", self.handle, int(enabled))

    def Profile(self) -> dict:
        """Per kernel family since profiling was enabled: launches, ms,
        algorithmic flops and bytes."""
        out = {}
        i = 0
        buf = ctypes.create_string_buffer(128)
        launches, ms, flops, nbytes = ctypes.c_int64(), ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
        while True:
            st = _lib.lib().ndx_model_profile_entry(self.handle, i, buf, 128, ctypes.byref(launches),
                                                    ctypes.byref(ms), ctypes.byref(flops), ctypes.byref(nbytes))
            if st != 0:
                break
            out[buf.value.decode()] = dict(launches=launches.value, ms=ms.value, flops=flops.value,
                                           bytes=nbytes.value)
            i += 1
        return out

    def Dispose(self):
        if self._h is not None:
            call("ndx_model_release", self._h)
            self._h = None

    def __del__(self):
        try:
            self.Dispose()
        except Exception:
            pass


class ModelBuilder:
    """A graph under construction plus its weights (Graph/ModelBuilder.cs:11).
    Weights are registered with Constant/Weight and carry their data (the
    graph owns them on the device at once); per-run inputs with Placeholder,
    bound in order by Run/RunOnDevice."""

    QuantizeFrom = 1 << 16  # BlockQuantizer.MinimumElements

    def __init__(self, device: Device, dataType: HostDataType = HostDataType.Float32, int8Weights: bool = False):
        self.Graph = Graph(device, dataType, int8Weights)
        self.Device = device
        self._dataType = HostDataType(dataType)
        self.Int8Weights = bool(int8Weights)
        self._placeholders: list[Expression] = []
        self._operator: Optional[CompiledModel] = None

    @property
    def DataType(self) -> HostDataType:
        return self._dataType

    def Constant(self, tensor: HostTensor, shape=None, dataType: Optional[HostDataType] = None) -> Expression:
        """ModelBuilder.Constant (:45-57): converted to dataType (the
        builder's by default) and owned by the graph on the device."""
        dtype = HostDataType(self._dataType if dataType is None else dataType)
        if shape is not None:
            tensor = tensor.Reshape(*shape)
        data = tensor.Data
        return self.Graph._new("ndx_graph_constant", int(dtype), _lib.shape_array(tensor.Shape), len(tensor.Shape),
                               data.ctypes.data_as(ctypes.c_void_p), int(tensor.DataType))

    def Weight(self, tensor: HostTensor, shape, rows: int) -> Expression:
        """ModelBuilder.Weight (:65-88): int8 block-quantised when the builder
        says so and the weight is large and tiles into blocks of 32."""
        tensor = tensor.Reshape(*shape)
        data = tensor.Data
        return self.Graph._new("ndx_graph_weight", _lib.shape_array(tensor.Shape), len(tensor.Shape),
                               data.ctypes.data_as(ctypes.c_void_p), int(tensor.DataType), int(rows))

    def WeightOnDevice(self, tensor: DeviceTensor, rows: int) -> Expression:
        """Weight for data already on the device; the graph takes it over."""
        return self.Graph._new("ndx_graph_weight_device", tensor.take(), int(rows))

    def WeightInt8(self, q: DeviceTensor, scales: DeviceTensor, block: int) -> Expression:
        """A pre-quantised weight (Device.QuantizeInt8's output); the graph
        takes both tensors over."""
        return self.Graph._new("ndx_graph_weight_int8", q.take(), scales.take(), int(block))

    def ConstantOnDevice(self, tensor: DeviceTensor) -> Expression:
        return self.Graph._new("ndx_graph_constant_device", tensor.take())

    def Placeholder(self, shape, dataType: Optional[HostDataType] = None) -> Expression:
        """ModelBuilder.Placeholder (:93-98)."""
        e = self.Graph.Input(self._dataType if dataType is None else dataType, shape)
        self._placeholders.append(e)
        return e

    def Compile(self, outputs: Sequence[Expression]) -> "ModelBuilder":
        """ModelBuilder.Compile (:105-133). The graph is released afterwards:
        the compiled model holds the only copy of the weights."""
        self._operator = CompiledModel(self.Graph, outputs, self.Device)
        return self

    def _require(self) -> CompiledModel:
        if self._operator is None:
            raise InvalidOperationError("Compile() the model before running it")
        return self._operator

    def Run(self, *values: HostTensor) -> list[HostTensor]:
        op = self._require()
        if len(values) != len(self._placeholders):
            raise ArgumentError(f"expected {len(self._placeholders)} inputs, got {len(values)}")
        return op.Dispatch(values)

    def RunOnDevice(self, *values: DeviceTensor) -> list[DeviceTensor]:
        op = self._require()
        if len(values) != len(self._placeholders):
            raise ArgumentError(f"expected {len(self._placeholders)} inputs, got {len(values)}")
        return op.DispatchOnDevice(values)

    @property
    def Compiled(self) -> CompiledModel:
        if self._operator is None:
            raise InvalidOperationError("Compile() the model first")
        return self._operator

    @property
    def TemporarySize(self) -> int:
        return self._operator.TemporarySize if self._operator else 0

    @property
    def PersistentBytes(self) -> int:
        return self._operator.PersistentSize if self._operator else 0

    def Dispose(self):
        if self._operator is not None:
            self._operator.Dispose()
            self._operator = None
        self.Graph.Dispose()
