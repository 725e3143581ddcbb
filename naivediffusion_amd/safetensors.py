"""SafetensorsFile (Weights/SafetensorsFile.cs:22-259) over the library's
mapped reader (ndx_safetensors_*).

The file is mapped read-only and its header checked once, at open; a tensor
is either a window onto the mapping (Read, a read-only numpy view, no copy)
or goes straight to device memory through the library's pinned staging
buffers and is narrowed there (ReadDevice). A window keeps the mapping alive:
Dispose refuses further reads at once, and the file is unmapped when the
last window is gone (the reference leaves a window dangling instead).
"""

from __future__ import annotations

import ctypes
from typing import Dict, List, Optional, Tuple

import numpy as np

from . import _lib
from ._lib import ArgumentError, UnsupportedError
from .tensors import _NP, Device, DeviceTensor, HostDataType, HostTensor


class InvalidDataError(ValueError):
    """InvalidDataException: a file that does not describe itself consistently."""


_DTYPES = {
    "F32": HostDataType.Float32,
    "F16": HostDataType.Float16,
    "BF16": HostDataType.BFloat16,
    "U32": HostDataType.UInt32,
    "I32": HostDataType.Int32,
    "U16": HostDataType.UInt16,
    "I64": HostDataType.Int64,
}


def IsSupportedDataType(dtype: str) -> bool:
    """SafetensorsFile.IsSupportedDataType (:229-240)."""
    return dtype in _DTYPES


def ParseDataType(dtype: str) -> HostDataType:
    """SafetensorsFile.ParseDataType (:242-253)."""
    if dtype not in _DTYPES:
        raise UnsupportedError(f"safetensors dtype {dtype} is not supported")
    return _DTYPES[dtype]


class _Mapping:
    """The open library handle; closed when the file and every window onto
    it are gone."""

    def __init__(self, handle):
        self.handle = handle

    def close(self):
        if self.handle is not None:
            _lib.call("ndx_safetensors_close", self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class SafetensorsFile:
    """A safetensors file, mapped; see the module docstring."""

    def __init__(self, path: str):
        self.Path = str(path)
        h = ctypes.c_void_p()
        try:
            _lib.call("ndx_safetensors_open", self.Path.encode(), ctypes.byref(h))
        except ArgumentError as e:
            raise InvalidDataError(str(e)) from None
        self._map: Optional[_Mapping] = _Mapping(h)
        entries, notes = ctypes.c_int32(), ctypes.c_int32()
        _lib.call("ndx_safetensors_count", h, ctypes.byref(entries), ctypes.byref(notes))
        self._entries: Dict[str, Tuple[str, Tuple[int, ...], int]] = {}
        name, dtype = ctypes.c_char_p(), ctypes.c_char_p()
        shape, rank, size = (ctypes.c_int64 * 8)(), ctypes.c_int32(), ctypes.c_uint64()
        for i in range(entries.value):
            _lib.call("ndx_safetensors_entry", h, i, ctypes.byref(name), ctypes.byref(dtype), shape,
                      ctypes.byref(rank), ctypes.byref(size))
            self._entries[name.value.decode("utf-8")] = (
                dtype.value.decode("utf-8"), tuple(shape[j] for j in range(rank.value)), size.value)
        self._metadata: Dict[str, str] = {}
        key, value = ctypes.c_char_p(), ctypes.c_char_p()
        for i in range(notes.value):
            _lib.call("ndx_safetensors_metadata", h, i, ctypes.byref(key), ctypes.byref(value))
            self._metadata[key.value.decode("utf-8")] = value.value.decode("utf-8")

    def _handle(self):
        if self._map is None:
            raise RuntimeError(f"{self.Path} was disposed")
        return self._map.handle

    @property
    def Keys(self) -> List[str]:
        return list(self._entries)

    @property
    def Metadata(self) -> Dict[str, str]:
        """The string-valued __metadata__ notes (:151-155)."""
        return dict(self._metadata)

    def TryGetInfo(self, name: str):
        """(found, dtype as written, shape) without mapping anything (:160-169)."""
        e = self._entries.get(name)
        if e is None:
            return False, "", ()
        return True, e[0], e[1]

    def Read(self, name: str) -> HostTensor:
        """One tensor as a read-only window onto the mapping (:172-180)."""
        h = self._handle()
        if name not in self._entries:
            raise KeyError(name)
        dtype = ParseDataType(self._entries[name][0])
        shape = self._entries[name][1]
        ptr, size = ctypes.c_void_p(), ctypes.c_uint64()
        _lib.call("ndx_safetensors_data", h, name.encode("utf-8"), ctypes.byref(ptr), ctypes.byref(size))
        if size.value == 0:
            data = np.empty(0, _NP[dtype])
            data.flags.writeable = False
        else:
            window = (ctypes.c_uint8 * size.value).from_address(ptr.value)
            window._mapping = self._map  # the window keeps the mapping alive
            data = np.frombuffer(window, dtype=_NP[dtype])
            data.flags.writeable = False
        if data.size != int(np.prod(shape, dtype=np.int64)):
            raise InvalidDataError(f"the safetensors entry {name}'s bytes do not match its shape and dtype")
        return HostTensor(dtype, shape, data)

    def ReadPrefix(self, prefix: str) -> Dict[str, HostTensor]:
        """Every tensor under prefix, keyed with it stripped (:184-196)."""
        return {k[len(prefix):]: self.Read(k) for k in self._entries if k.startswith(prefix)}

    def ReadDevice(self, name: str, device: Device, dtype: Optional[HostDataType] = None) -> DeviceTensor:
        """One tensor copied into device memory and, for a float tensor,
        narrowed there to dtype (None: as stored) with nearest-even
        rounding: Read followed by HostTensor.ConvertTo (HostTensor.cs:110-130)
        and the upload, without a host copy. More than 4 axes fold into the
        first."""
        h = self._handle()
        if name not in self._entries:
            raise KeyError(name)
        out = ctypes.c_void_p()
        _lib.call("ndx_safetensors_read", h, name.encode("utf-8"), device.handle,
                  -1 if dtype is None else int(dtype), ctypes.byref(out))
        return DeviceTensor(device, out)

    def Dispose(self):
        """Dispose (:198-214): no reads after this; the mapping goes with
        the last window onto it."""
        if self._map is not None:
            m, self._map = self._map, None
            del m

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.Dispose()
