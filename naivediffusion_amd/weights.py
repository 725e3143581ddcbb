"""Model weights by name, registered once in a ModelBuilder: host arrays
(uploaded through ModelBuilder.Weight, with the int8 quantiser when the
builder has it on) or device tensors (taken over through WeightOnDevice),
plus the stacked projections that the MI355X path runs as one GEMM (q, k, v
of a self-attention; k, v of a cross-attention), stacked once at build time
on the device."""

from __future__ import annotations

import numpy as np

from .graph import CompiledModel, Graph, ModelBuilder, Ops
from .tensors import Device, DeviceTensor, HostDataType, HostTensor


def device_stack(device: Device, tensors, columns: int = 0) -> DeviceTensor:
    """Rows of the given device matrices stacked into one new device tensor
    (one small compiled copy, at build time); with columns > 0 only the
    first `columns` columns of a single matrix."""
    g = Graph(device)
    ins = [g.Input(t.DataType, list(t.Shape)) for t in tensors]
    if columns:
        rows = tensors[0].Shape[0]
        out = Ops.Identity(Ops.Slice(ins[0], [0, 0], [rows, columns]))
    else:
        joined = Ops.Join([Ops.Reinterpret(e, [1, 1] + list(e.Shape)) for e in ins], 2)
        out = Ops.Reinterpret(joined, list(joined.Shape[2:]))
    model = CompiledModel(g, [out], device)
    (res,) = model.DispatchOnDevice(list(tensors))
    model.Dispose()
    g.Dispose()
    return res


class WeightSet:
    """The weights of one model by name (host arrays or device tensors),
    each registered once in a builder; stacks the projections that run as
    one GEMM. Device tensors handed to the builder as weights are taken over
    by it (ModelBuilder.WeightOnDevice)."""

    def __init__(self, model: ModelBuilder, weights: dict, compute: HostDataType, device: Device):
        self.model, self.weights, self.compute, self.device = model, weights, compute, device
        self.cache = {}
        self.owned = []   # device tensors made here, released after compile

    def _register(self, key, w, kind):
        """kind "weight": a matrix at the builder's storage type; "wide": an
        fp32 vector; "norm": a vector at the compute type (the activation
        width it meets, Layers.ConstantType, Graph/Layers.cs:96-97)."""
        m = self.model
        dt = HostDataType.Float32 if kind == "wide" else self.compute
        if isinstance(w, DeviceTensor) and kind == "weight":
            e = m.WeightOnDevice(w, w.Shape[0])
        elif isinstance(w, DeviceTensor) and w.DataType == dt:
            e = m.ConstantOnDevice(w)
        else:
            arr = np.asarray(w.Download().ToFloats() if isinstance(w, DeviceTensor) else w, np.float32)
            if kind == "weight":
                e = m.Weight(HostTensor.FromFloats(arr), arr.shape, arr.shape[0])
            else:
                e = m.Constant(HostTensor.FromFloats(arr), [arr.size], dt)
        self.cache[key] = e
        return e

    def has(self, name: str) -> bool:
        return name in self.weights

    def __call__(self, name: str, kind: str = "weight"):
        if name in self.cache:
            return self.cache[name]
        return self._register(name, self.weights[name], kind)

    def stacked(self, names, kind: str = "weight"):
        """The named tensors stacked along their first axis (matrices row
        after row, vectors end to end), registered as kind."""
        key = "+".join(names)
        if key in self.cache:
            return self.cache[key]
        ws = [self.weights[n] for n in names]
        if all(isinstance(w, DeviceTensor) for w in ws):
            w = device_stack(self.device, ws)
            self.owned.append(w)
        else:
            w = np.concatenate([np.asarray(x.Download().ToFloats() if isinstance(x, DeviceTensor) else x, np.float32)
                                for x in ws], 0)
        return self._register(key, w, kind)

    def columns(self, name, count):
        key = f"{name}[:, :{count}]"
        if key in self.cache:
            return self.cache[key]
        w = self.weights[name]
        if isinstance(w, DeviceTensor):
            w = device_stack(self.device, [w], columns=count)
            self.owned.append(w)
        else:
            w = np.ascontiguousarray(np.asarray(w, np.float32)[:, :count])
        return self._register(key, w, "weight")

    def release(self):
        for t in self.owned:
            t.Dispose()
        self.owned = []
