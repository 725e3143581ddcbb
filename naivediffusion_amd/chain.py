"""GraphChain (Graph/GraphChain.cs): a model written as a sequence of links
with named values carried between them.

The builder API is the reference's — Input, Get, Set, Drop, Cut, Finish,
Run, Current, Shape and the byte counts — so model code written against it
(AnimaDit.Build, UNetModel.Build) reads the same. The reference cuts a model
into several DirectML graphs to keep each persistent resource under 4 GiB and
to stream weights from system memory; with 288 GB of HBM nothing needs
cutting, so here every link lands in one compiled model and Cut only marks
the boundary: the named values are plain expressions, carried tensors never
leave the device, and the weight-streaming tier is a no-op (StreamedBytes 0).
"""

from __future__ import annotations

from typing import Dict, List, Optional, Sequence

from ._lib import ArgumentError, InvalidOperationError
from .graph import Expression, ModelBuilder, Ops
from .tensors import Device, DeviceTensor, HostDataType, HostTensor


class GraphChain:
    """GraphChain.cs:21. residentBudget is accepted for the reference's
    signature and has nothing to decide: every weight is resident."""

    def __init__(self, device: Device, dataType: HostDataType, residentBudget: Optional[int] = None,
                 int8Weights: bool = False):
        self._device = device
        self._dataType = HostDataType(dataType)
        self._model = ModelBuilder(device, dataType, int8Weights)
        self._shapes: Dict[str, List[int]] = {}
        self._types: Dict[str, HostDataType] = {}
        self._declared: Dict[str, HostDataType] = {}
        self._values: Dict[str, Expression] = {}
        self._placeholders: List[str] = []
        self._links = 0
        self._result: Optional[str] = None

    @property
    def Current(self) -> ModelBuilder:
        """The graph under construction (one for the whole chain)."""
        return self._model

    def Input(self, name: str, shape: Sequence[int], dataType: Optional[HostDataType] = None) -> None:
        """A value the caller supplies to Run (GraphChain.cs:86-94); it
        becomes a placeholder when first read."""
        if name in self._declared:
            raise ArgumentError(f"{name} was declared twice")
        dt = HostDataType(dataType) if dataType is not None else self._dataType
        self._declared[name] = dt
        self._shapes[name] = [int(s) for s in shape]
        self._types[name] = dt

    def Get(self, name: str) -> Expression:
        """The value called name (GraphChain.cs:99-110)."""
        if name in self._values:
            return self._values[name]
        if name not in self._shapes:
            raise ArgumentError(f"{name} has not been produced yet")
        placeholder = self._model.Placeholder(self._shapes[name], self._types[name])
        self._values[name] = placeholder
        self._placeholders.append(name)
        return placeholder

    def Shape(self, name: str) -> List[int]:
        return list(self._shapes[name])

    def Set(self, name: str, value: Expression) -> None:
        """Names a value for later links; naming it again replaces it
        (GraphChain.cs:125-138)."""
        if value.graph is not self._model.Graph:
            raise ArgumentError(f"{name} belongs to an earlier link")
        self._values[name] = value
        self._shapes[name] = list(value.Shape)
        self._types[name] = value.DataType

    def Drop(self, name: str) -> None:
        """Nothing after this reads name (GraphChain.cs:142-155)."""
        if name not in self._shapes:
            raise ArgumentError(f"{name} is not a live value")
        del self._shapes[name]
        self._types.pop(name, None)
        self._values.pop(name, None)

    def Cut(self) -> None:
        """Ends a link (GraphChain.cs:160-202): a boundary only."""
        if self._result is not None:
            raise InvalidOperationError("the chain is finished")
        self._links += 1

    def Finish(self, result: str) -> None:
        """Cuts the last link and names the value Run returns (:205-213);
        the whole chain compiles here."""
        self.Cut()
        if result not in self._shapes:
            raise ArgumentError(f"{result} is not a live value at the end")
        out = self.Get(result)
        if result in self._placeholders:
            out = Ops.Identity(out)  # a graph input cannot be a graph output
        self._model.Compile([out])
        self._result = result

    def _ordered(self, inputs: dict) -> list:
        """The inputs in placeholder order, with the reference's checks
        (GraphChain.cs:230-250)."""
        if self._result is None:
            raise InvalidOperationError("Finish() the chain before running it")
        for name in inputs:
            if name not in self._declared:
                raise ArgumentError(f"{name} is not an input of this chain")
        for name in self._placeholders:
            if name not in inputs:
                raise InvalidOperationError(f"{name} was not supplied")
        return [inputs[n] for n in self._placeholders]

    def Run(self, inputs: Dict[str, HostTensor]) -> HostTensor:
        """Feeds the declared inputs (converted to their declared types)
        through the model and returns the result on the host (:218-282)."""
        host = [t.ConvertTo(self._declared[n]) for n, t in zip(self._placeholders, self._ordered(inputs))]
        return self._model.Run(*host)[0]

    def RunOnDevice(self, inputs: Dict[str, DeviceTensor]) -> DeviceTensor:
        """Run with device tensors in and out (the latent stays in HBM)."""
        return self._model.RunOnDevice(*self._ordered(inputs))[0]

    @property
    def PersistentBytes(self) -> int:
        return self._model.PersistentBytes if self._result is not None else 0

    @property
    def StreamedBytes(self) -> int:
        return 0

    @property
    def ResidentBytes(self) -> int:
        return self.PersistentBytes

    @property
    def TemporaryBytes(self) -> int:
        return self._model.TemporarySize if self._result is not None else 0

    @property
    def LinkCount(self) -> int:
        """Links as the reference counts them (cuts made); they compile as one."""
        return self._links

    def Dispose(self) -> None:
        self._model.Dispose()
