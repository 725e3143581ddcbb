"""naivediffusion_amd: an MI355X (gfx950) backend for NaiveDiffusion's
denoiser forward pass.

The compute runs in libndx.so (hand-written HIP kernels behind the C ABI of
include/ndx.h); this package is the host-side mirror of the reference's
per-layer builder API (Layers, Transformer, ModelBuilder) and device
surface (Device, DeviceTensor, HostTensor), plus the denoiser compositions.
"""

from ._lib import (ArgumentError, DeviceRemovedError, InvalidOperationError, NdxError, OutOfVideoMemoryError,
                   UnsupportedError)
from .graph import CompiledModel, Expression, Graph, MaskType, ModelBuilder, Ops
from .layers import Layers, Transformer
from .tensors import Device, DeviceTensor, HostDataType, HostTensor

__all__ = [
    "ArgumentError", "DeviceRemovedError", "InvalidOperationError", "NdxError", "OutOfVideoMemoryError",
    "UnsupportedError", "CompiledModel", "Expression", "Graph", "MaskType", "ModelBuilder", "Ops", "Layers",
    "Transformer", "Device", "DeviceTensor", "HostDataType", "HostTensor",
]
