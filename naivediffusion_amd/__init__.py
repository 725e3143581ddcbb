"""naivediffusion_amd: an MI355X (gfx950) backend for NaiveDiffusion's
denoiser forward pass.

The compute runs in libndx.so (hand-written HIP kernels behind the C ABI of
include/ndx.h); this package is the host-side mirror of the reference's
per-layer builder API (Layers, Transformer, ModelBuilder, GraphChain) and device
surface (Device, DeviceTensor, HostTensor), plus the denoiser compositions.
"""

from ._lib import (ArgumentError, DeviceRemovedError, InvalidOperationError, NdxError, OutOfVideoMemoryError,
                   UnsupportedError)
from .chain import GraphChain
from .graph import CompiledModel, Expression, Graph, MaskType, ModelBuilder, Ops
from .layers import Layers, Transformer
from .tensors import Device, DeviceTensor, HostDataType, HostTensor

__all__ = [
    "ArgumentError", "DeviceRemovedError", "InvalidOperationError", "NdxError", "OutOfVideoMemoryError",
    "UnsupportedError", "GraphChain", "CompiledModel", "Expression", "Graph", "MaskType", "ModelBuilder", "Ops", "Layers",
    "Transformer", "Device", "DeviceTensor", "HostDataType", "HostTensor",
]
