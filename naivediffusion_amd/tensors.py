"""Host and device tensors, and the device itself.

Mirrors Tensors/HostTensor.cs (HostDataType ordinals, packed bytes, exact
widening, round-to-nearest-even narrowing), Dml/DeviceTensor.cs and the
device surface of Dml/DmlDevice.cs, over the C ABI of libndx.so.
"""

from __future__ import annotations

import ctypes
import enum
from typing import Sequence

import numpy as np

from . import _lib
from ._lib import ArgumentError, call


class HostDataType(enum.IntEnum):
    """Tensors/HostTensor.cs:8-18, same ordinals (the C ABI's dtype codes)."""
    Float32 = 0
    Float16 = 1
    BFloat16 = 2
    UInt32 = 3
    Int32 = 4
    UInt16 = 5
    Int64 = 6
    Int8 = 7


_NP = {
    HostDataType.Float32: np.float32,
    HostDataType.Float16: np.float16,
    HostDataType.BFloat16: np.uint16,  # the raw top halves of float32
    HostDataType.UInt32: np.uint32,
    HostDataType.Int32: np.int32,
    HostDataType.UInt16: np.uint16,
    HostDataType.Int64: np.int64,
    HostDataType.Int8: np.int8,
}


def bytes_per_element(dtype: HostDataType) -> int:
    return np.dtype(_NP[HostDataType(dtype)]).itemsize


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """bfloat16 is the top half of a float32 (HostTensor.cs:178-187): exact."""
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 to bfloat16 bits, rounding to nearest even."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


class HostTensor:
    """A CPU-side tensor: a shape, an element type and packed data
    (Tensors/HostTensor.cs:28). data is a numpy array of the storage type
    (uint16 bits for bfloat16)."""

    def __init__(self, dtype: HostDataType, shape: Sequence[int], data: np.ndarray):
        dtype = HostDataType(dtype)
        shape = tuple(int(s) for s in shape)
        data = np.ascontiguousarray(data, dtype=_NP[dtype])
        if data.size != int(np.prod(shape, dtype=np.int64)):
            raise ArgumentError(f"{data.nbytes} bytes do not fill a {dtype.name} tensor of {list(shape)}")
        self.DataType = dtype
        self.Shape = shape
        self.Data = data.reshape(shape)

    @property
    def ElementCount(self) -> int:
        return int(np.prod(self.Shape, dtype=np.int64))

    @staticmethod
    def FromFloats(values, *shape) -> "HostTensor":
        values = np.asarray(values, np.float32)
        return HostTensor(HostDataType.Float32, shape or values.shape, values)

    @staticmethod
    def FromInt32(values, *shape) -> "HostTensor":
        values = np.asarray(values, np.int32)
        return HostTensor(HostDataType.Int32, shape or values.shape, values)

    def Reshape(self, *shape) -> "HostTensor":
        if int(np.prod(shape)) != self.ElementCount:
            raise ArgumentError(f"cannot view {self.ElementCount} elements as {list(shape)}")
        return HostTensor(self.DataType, shape, self.Data)

    def ToFloats(self) -> np.ndarray:
        """Widened to float32 (HostTensor.ToFloats / Widen, :140-192)."""
        if self.DataType == HostDataType.Float32:
            return self.Data.astype(np.float32, copy=True)
        if self.DataType == HostDataType.Float16:
            return self.Data.astype(np.float32)
        if self.DataType == HostDataType.BFloat16:
            return bf16_to_f32(self.Data)
        raise ArgumentError(f"cannot widen {self.DataType.name} to float32")

    def ConvertTo(self, target: HostDataType) -> "HostTensor":
        """HostTensor.ConvertTo (:110-130): float widths only, round to nearest even."""
        target = HostDataType(target)
        if target == self.DataType:
            return self
        wide = self.ToFloats()
        if target == HostDataType.Float32:
            return HostTensor(target, self.Shape, wide)
        if target == HostDataType.Float16:
            return HostTensor(target, self.Shape, wide.astype(np.float16))
        if target == HostDataType.BFloat16:
            return HostTensor(target, self.Shape, f32_to_bf16(wide))
        raise ArgumentError(f"cannot convert {self.DataType.name} to {target.name}")

    def ToInt32s(self) -> np.ndarray:
        if self.DataType != HostDataType.Int32:
            raise RuntimeError(f"{self.DataType.name} is not int32")
        return self.Data.ravel().copy()

    def __repr__(self):
        return f"<host {self.DataType.name} {list(self.Shape)}>"


class Device:
    """One GPU and its stream (Dml/DmlDevice.cs:15). Synchronous: every call
    that launches work has finished it on return."""

    def __init__(self, adapter_index: int = -1):
        h = ctypes.c_void_p()
        call("ndx_device_create", adapter_index, ctypes.byref(h))
        self._h = h

    @staticmethod
    def Count() -> int:
        n = ctypes.c_int32()
        call("ndx_device_count", ctypes.byref(n))
        return n.value

    @property
    def handle(self):
        if self._h is None:
            raise RuntimeError("the device was disposed")
        return self._h

    @property
    def AdapterName(self) -> str:
        buf = ctypes.create_string_buffer(256)
        call("ndx_device_name", self.handle, buf, 256)
        return buf.value.decode()

    def VideoMemory(self):
        used, budget = ctypes.c_uint64(), ctypes.c_uint64()
        call("ndx_device_memory", self.handle, ctypes.byref(used), ctypes.byref(budget))
        return used.value, budget.value

    def ReleasePooledBuffers(self):
        call("ndx_device_release_pooled", self.handle)

    def Synchronize(self):
        call("ndx_device_synchronize", self.handle)

    def SetFaultInjection(self, kind: int):
        call("ndx_device_set_fault_injection", self.handle, kind)

    def Upload(self, tensor: HostTensor) -> "DeviceTensor":
        """DmlDevice.Upload (:657-689): copies; the host tensor is borrowed."""
        h = ctypes.c_void_p()
        data = tensor.Data
        call("ndx_tensor_upload", self.handle, int(tensor.DataType), _lib.shape_array(tensor.Shape),
             len(tensor.Shape), data.ctypes.data_as(ctypes.c_void_p), data.nbytes, ctypes.byref(h))
        return DeviceTensor(self, h)

    def Empty(self, dtype: HostDataType, shape) -> "DeviceTensor":
        h = ctypes.c_void_p()
        call("ndx_tensor_empty", self.handle, int(dtype), _lib.shape_array(shape), len(shape), ctypes.byref(h))
        return DeviceTensor(self, h)

    def Normal(self, dtype: HostDataType, shape, seed: int, mean: float = 0.0, std: float = 1.0) -> "DeviceTensor":
        """A synthetic tensor of N(mean, std) values made on the device."""
        t = self.Empty(dtype, shape)
        call("ndx_tensor_fill_normal", t.handle, ctypes.c_uint64(seed & (2**64 - 1)), mean, std)
        return t

    def QuantizeInt8(self, weight: "DeviceTensor", block: int = 32,
                     scaleType: HostDataType = HostDataType.Float16) -> tuple:
        """BlockQuantizer.Quantize (Tensors/BlockQuantizer.cs:34-101) on the
        device: weight [rows, cols] -> (q int8 [rows, cols], scales [rows,
        cols / block] of scaleType). block 32 with Float16 scales is the
        reference's format; block = cols with Float32 is per output channel."""
        rows, cols = weight.Shape[0], int(np.prod(weight.Shape[1:]))
        q = self.Empty(HostDataType.Int8, [rows, cols])
        s = self.Empty(scaleType, [rows, cols // block])
        call("ndx_quantize_block_int8_device", weight.handle, int(block), int(scaleType), q.handle, s.handle)
        return q, s

    def Dispose(self):
        if self._h is not None:
            call("ndx_device_destroy", self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.Dispose()


class DeviceTensor:
    """A tensor in device memory (Dml/DeviceTensor.cs:11); Dispose returns it
    to the device's pool."""

    def __init__(self, device: Device, handle):
        self.Device = device
        self._h = handle

    @property
    def handle(self):
        if self._h is None:
            raise RuntimeError("the tensor was disposed")
        return self._h

    def _info(self):
        dt, rank = ctypes.c_int32(), ctypes.c_int32()
        shape = (ctypes.c_int64 * 4)()
        call("ndx_tensor_info", self.handle, ctypes.byref(dt), shape, ctypes.byref(rank))
        return HostDataType(dt.value), tuple(shape[i] for i in range(rank.value))

    @property
    def Shape(self):
        return self._info()[1]

    @property
    def DataType(self) -> HostDataType:
        return self._info()[0]

    def Download(self) -> HostTensor:
        dtype, shape = self._info()
        out = np.empty(shape, _NP[dtype])
        call("ndx_tensor_download", self.handle, out.ctypes.data_as(ctypes.c_void_p), out.nbytes)
        return HostTensor(dtype, shape, out)

    def Dispose(self):
        if self._h is not None:
            call("ndx_tensor_release", self._h)
            self._h = None

    def take(self):
        """Hands the handle over (to a graph that takes ownership)."""
        h, self._h = self._h, None
        return h

    def __del__(self):
        try:
            self.Dispose()
        except Exception:
            pass

    def __repr__(self):
        dtype, shape = self._info()
        return f"<device {dtype.name} {list(shape)}>"
