"""Hand-written safetensors files for the tests, laid out as the
reference's fixture writer lays them out (Tests/Fixtures/FakeSafetensors.cs:
45-101): an 8-byte header length, the JSON table, then the tensors with
values in order and the ones without as zeros the file gets by being
extended past them."""

from __future__ import annotations

import json
import struct
from pathlib import Path

import numpy as np

from naivediffusion_amd.tensors import f32_to_bf16

WIDTH = {"F32": 4, "F16": 2, "BF16": 2, "U16": 2, "I32": 4, "U32": 4, "I64": 8, "F8_E4M3": 1, "F8_E5M2": 1,
         "I8": 1}


def encode(dtype: str, values) -> bytes:
    v = np.asarray(values)
    if dtype == "F32":
        return np.ascontiguousarray(v, np.float32).tobytes()
    if dtype == "F16":
        return np.ascontiguousarray(v, np.float32).astype(np.float16).tobytes()
    if dtype == "BF16":
        return f32_to_bf16(np.asarray(v, np.float32)).tobytes()
    return np.ascontiguousarray(v, {"U16": np.uint16, "I32": np.int32, "U32": np.uint32, "I64": np.int64,
                                    "I8": np.int8}[dtype]).tobytes()


def write(path, tensors, metadata=None, header_pad: int = 0) -> str:
    """tensors: (name, shape, dtype, values or None) in any order; values
    are floats for the float types (rounded to nearest even on the way)."""
    header = {}
    if metadata is not None:
        header["__metadata__"] = metadata
    body = bytearray()
    end = 0
    for name, shape, dtype, values in sorted(tensors, key=lambda t: t[3] is None):
        n = int(np.prod(shape, dtype=np.int64)) if len(shape) else 1
        start = end
        end += n * WIDTH[dtype]
        if values is not None:
            data = encode(dtype, np.asarray(values).reshape(-1))
            assert len(data) == n * WIDTH[dtype], name
            body += data
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [start, end]}
    text = json.dumps(header).encode() + b" " * header_pad
    path = str(path)
    with open(path, "wb") as f:
        f.write(struct.pack("<q", len(text)))
        f.write(text)
        f.write(bytes(body))
        f.truncate(8 + len(text) + end)
    return path


def with_header(path, text: bytes) -> str:
    """A file that is only a header: the reference's WithHeader
    (CheckpointInspectorTests.cs:257-263)."""
    Path(path).write_bytes(struct.pack("<q", len(text)) + text)
    return str(path)
