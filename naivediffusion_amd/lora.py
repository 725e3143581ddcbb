"""LoRAs and lazily narrowed weights on the way into HBM.

Mirrors Weights/LoraFile.cs (LoraSpec, LoraTower, LoraRows, LoraLayout,
LoraFile, LoraMerge, LoraPatchSet) and Weights/LazyWeights.cs. Matching a
file's pairs to a model's weights is string work and stays on the host, as
in the reference; the fold itself, W' = W + weight * (alpha / rank) * up . down,
runs on the device (ndx_lora_fold) with the reference's order and rounding:
each output row widened to float32, every pair covering it and every rank in
order added as (scale * up[row, r]) * down[r, :], each product and sum
rounded on its own, zero factors skipped, the row narrowed once.
"""

from __future__ import annotations

import ctypes
import os
import re
from dataclasses import dataclass
from typing import Callable, Dict, Iterable, List, Mapping, Optional, Sequence, Tuple

import numpy as np

from . import _lib
from .safetensors import InvalidDataError, SafetensorsFile
from .tensors import Device, DeviceTensor, HostDataType, HostTensor

F32 = HostDataType.Float32
F16 = HostDataType.Float16


@dataclass(frozen=True)
class LoraSpec:
    """LoraSpec (LoraFile.cs:11-57): a file and the multiplier on its delta."""
    Path: str
    Weight: float

    @staticmethod
    def Stamp(loras: Sequence["LoraSpec"]) -> str:
        """A cache key that changes when any LoRA does (:17-31): full path,
        size, write time (.NET ticks) and weight of each non-zero one."""
        parts = []
        for lora in loras:
            if lora.Weight == 0:
                continue
            st = os.stat(lora.Path)
            ticks = st.st_mtime_ns // 100 + 621355968000000000
            parts.append(f"{os.path.abspath(lora.Path)}|{st.st_size}|{ticks}|{str(np.float32(lora.Weight))}")
        return "\n".join(parts)

    @staticmethod
    def Combine(*sources: Iterable["LoraSpec"]) -> List["LoraSpec"]:
        """One list of several, a later entry for the same file replacing the
        earlier one in place (:39-56)."""
        combined: List[LoraSpec] = []
        for source in sources:
            for lora in source:
                same = [i for i, e in enumerate(combined) if os.path.abspath(e.Path) == os.path.abspath(lora.Path)]
                if same:
                    combined[same[0]] = lora
                else:
                    combined.append(lora)
        return combined


@dataclass(frozen=True)
class LoraTower:
    """LoraTower (:68-73): a model a LoRA can change, its kohya prefix, its
    PEFT prefix and the other dotted prefixes it may sit under."""
    Name: str
    Description: str
    KohyaPrefix: str
    PeftPrefix: str
    OtherPeftPrefixes: Tuple[str, ...] = ()

    @property
    def PeftPrefixes(self) -> List[str]:
        return [self.PeftPrefix, *self.OtherPeftPrefixes]


@dataclass(frozen=True)
class LoraRows:
    """LoraRows (:78): Count rows from First on that a LoRA names Name."""
    Name: str
    First: int
    Count: int


class LoraLayout:
    """LoraLayout (:84-148): a family's towers, the kohya prefixes that mark a
    file for another architecture, and the two name patterns."""

    def __init__(self, architecture: str, towers: Sequence[LoraTower], refused: Mapping[str, str]):
        self.Architecture = architecture
        self.Towers = list(towers)
        self.RefusedKohyaPrefixes = dict(refused)
        self._by_kohya = {t.KohyaPrefix: t for t in towers}
        self._by_peft = {p: t for t in towers for p in t.PeftPrefixes}
        self._by_name = {t.Name: t.Description for t in towers}
        kohya = "|".join([re.escape(t.KohyaPrefix) for t in towers] + [re.escape(k) for k in refused])
        peft = "|".join(re.escape(p) for p in self._by_peft if p)
        prefix = f"(?:({peft})\\.)?" if "" in self._by_peft else f"({peft})\\."
        self.KohyaPattern = re.compile(f"^lora_({kohya})_(.+)\\.(lora_down\\.weight|lora_up\\.weight|alpha)$")
        self.PeftPattern = re.compile(
            f"^{prefix}(.+)\\.(lora_A\\.weight|lora_B\\.weight|lora_A\\.default\\.weight|"
            "lora_B\\.default\\.weight|lora_down\\.weight|lora_up\\.weight|alpha)$")

    def ByKohya(self, prefix: str) -> Optional[LoraTower]:
        return self._by_kohya.get(prefix)

    def ByPeft(self, prefix: Optional[str]) -> Optional[LoraTower]:
        return self._by_peft.get(prefix or "")

    def Describe(self, tower: str) -> str:
        return self._by_name.get(tower, tower)


@dataclass
class Module:
    """LoraFile.Module (:171): one layer's pair, windows onto the file, and
    the trainer's alpha (None: alpha = rank)."""
    Down: HostTensor
    Up: HostTensor
    Alpha: Optional[float]


class LoraFile:
    """LoraFile (:155-312): a LoRA's tensors grouped into pairs, filed by
    tower and kohya-style layer name (dots to underscores)."""

    def __init__(self, path: str, layout: LoraLayout):
        self.Path = str(path)
        self._layout = layout
        self._towers: Dict[str, Dict[str, Module]] = {}
        self._file = SafetensorsFile(self.Path)
        try:
            self._index()
        except BaseException:
            self._file.Dispose()
            raise

    @property
    def Name(self) -> str:
        return os.path.splitext(os.path.basename(self.Path))[0]

    def Modules(self, tower: str) -> Dict[str, Module]:
        return dict(self._towers.get(tower, {}))

    def _index(self):
        """LoraFile.Index (:204-309)."""
        downs: Dict[Tuple[str, str], HostTensor] = {}
        ups: Dict[Tuple[str, str], HostTensor] = {}
        alphas: Dict[Tuple[str, str], float] = {}
        unreadable = 0
        L = self._layout
        for key in self._file.Keys:
            if key.endswith(".dora_scale"):
                raise InvalidDataError(
                    f"{self.Name} is a DoRA, which changes the weights' directions rather than adding to them; "
                    "this library applies only LoRA")
            m = L.KohyaPattern.match(key)
            if m:
                prefix = m.group(1)
                if prefix in L.RefusedKohyaPrefixes:
                    raise InvalidDataError(f"{self.Name} {L.RefusedKohyaPrefixes[prefix]}")
                ident = (L.ByKohya(prefix).Name, m.group(2))
                part = {"lora_down.weight": "down", "lora_up.weight": "up"}.get(m.group(3), "alpha")
            else:
                m = L.PeftPattern.match(key)
                if not m:
                    unreadable += 1
                    continue
                ident = (L.ByPeft(m.group(1)).Name, m.group(2).replace(".", "_"))
                part = {"lora_A.weight": "down", "lora_A.default.weight": "down", "lora_down.weight": "down",
                        "lora_B.weight": "up", "lora_B.default.weight": "up",
                        "lora_up.weight": "up"}.get(m.group(3), "alpha")
            if part == "down":
                downs[ident] = self._file.Read(key)
            elif part == "up":
                ups[ident] = self._file.Read(key)
            else:
                alphas[ident] = float(self._file.Read(key).ToFloats().ravel()[0])
        for tower, module in ups:
            if (tower, module) not in downs:
                raise InvalidDataError(f"{self.Name}: {module} has an up matrix but no down matrix")
        for (tower, module), down in downs.items():
            if (tower, module) not in ups:
                raise InvalidDataError(f"{self.Name}: {module} has a down matrix but no up matrix")
            self._towers.setdefault(tower, {})[module] = Module(down, ups[(tower, module)],
                                                                alphas.get((tower, module)))
        if not self._towers:
            arch = self._file.Metadata.get("modelspec.architecture", "")
            trained_for = f"; the file says it is a {arch}, not for {L.Architecture}" if arch else ""
            raise InvalidDataError(
                f"{self.Name} holds no LoRA pairs this library reads for {L.Architecture}; "
                "LoHa, LoKr and full-weight diffs are not supported" + trained_for
                if unreadable > 0 else f"{self.Name} holds no tensors")

    def Dispose(self):
        self._file.Dispose()


def _shape(t) -> Tuple[int, ...]:
    return tuple(t.Shape) if hasattr(t, "Shape") else tuple(t)


def _count(shape) -> int:
    return int(np.prod(shape, dtype=np.int64))


class LoraMerge:
    """LoraMerge (:315-423)."""

    @staticmethod
    def ModuleName(key: str) -> str:
        """The kohya name of a weight key (:333-334)."""
        return key[: -len(".weight")].replace(".", "_")

    @staticmethod
    def Check(weight_shape, module: Module, row_count: int, key: str) -> None:
        """Whether a pair is the shape of the rows it changes (:341-355)."""
        rank = module.Down.Shape[0]
        columns = _count(weight_shape) // weight_shape[0]
        if (module.Down.ElementCount != rank * columns or module.Up.Shape[0] != row_count
                or module.Up.ElementCount != row_count * rank):
            raise InvalidDataError(
                f"the LoRA's {key} is [{', '.join(map(str, module.Up.Shape))}] x "
                f"[{', '.join(map(str, module.Down.Shape))}] but the model's is "
                f"[{', '.join(map(str, weight_shape))}]; the LoRA was trained against a different model")

    @staticmethod
    def Merge(weight: DeviceTensor, patches: Sequence[Tuple[Module, float, int]],
              dtype: Optional[HostDataType] = None) -> DeviceTensor:
        """Merge (:362-420) on the device: a new tensor, the weight plus every
        pair's delta, at dtype (None: the reference's width, Float32 for a
        Float32 weight, else Float16)."""
        device = weight.Device
        shape = weight.Shape
        cols = _count(shape) // shape[0]
        uploaded = []
        try:
            descs = []
            for module, scale, first in patches:
                rank = module.Down.Shape[0]
                down = device.Upload(module.Down.Reshape(rank, cols))
                up = device.Upload(module.Up.Reshape(module.Up.Shape[0], rank))
                uploaded += [down, up]
                descs.append(_lib.LoraPatch(down.handle, up.handle, float(np.float32(scale)), int(first)))
            # More pairs than one launch takes: float32 between the launches
            # holds the row exactly as the single pass would.
            final = dtype if dtype is not None else (F32 if weight.DataType == F32 else F16)
            current = weight
            step = _lib.MAX_LORA_PATCHES
            chunks = [descs[i:i + step] for i in range(0, len(descs), step)] or [[]]
            for i, chunk in enumerate(chunks):
                want = int(final) if i == len(chunks) - 1 else int(F32)
                arr = (_lib.LoraPatch * max(len(chunk), 1))(*chunk)
                out = ctypes.c_void_p()
                _lib.call("ndx_lora_fold", current.handle, ctypes.cast(arr, ctypes.c_void_p), len(chunk), want,
                          ctypes.byref(out))
                if current is not weight:
                    current.Dispose()
                current = DeviceTensor(device, out)
            return current
        finally:
            for t in uploaded:
                t.Dispose()

    @staticmethod
    def Apply(tensors: Dict[str, DeviceTensor], layout: LoraLayout, tower: str, loras: Sequence[LoraSpec],
              aliases: Optional[Callable[[str], Iterable[str]]] = None,
              parts: Optional[Callable[[str], Iterable[LoraRows]]] = None) -> None:
        """Apply (:326-332): every weight any LoRA touches replaced by the
        merged copy (the old device tensor is released)."""
        patches = LoraPatchSet.Prepare(tensors, layout, tower, loras, aliases, parts)
        try:
            for key in list(patches.Keys):
                merged = patches.Apply(key, tensors[key])
                if merged is not tensors[key]:
                    tensors[key].Dispose()
                    tensors[key] = merged
        finally:
            patches.Dispose()


class LoraPatchSet:
    """LoraPatchSet (:427-535): the deltas a set of LoRAs has for one
    model's weights, matched by name, held with their files open."""

    def __init__(self, patches: Dict[str, List[Tuple[Module, float, int]]], files: List[LoraFile]):
        self._patches = patches
        self._files = files

    @staticmethod
    def Prepare(tensors: Mapping[str, object], layout: LoraLayout, tower: str, loras: Sequence[LoraSpec],
                aliases: Optional[Callable[[str], Iterable[str]]] = None,
                parts: Optional[Callable[[str], Iterable[LoraRows]]] = None) -> "LoraPatchSet":
        """Prepare (:445-516). tensors maps each weight key to anything with
        a Shape (a window, a device tensor) or to the shape itself."""
        by_module: Dict[str, Tuple[str, int, int]] = {}
        shapes = {k: _shape(v) for k, v in tensors.items()}
        for key, shape in shapes.items():
            if not key.endswith(".weight") or len(shape) == 0:
                continue
            rows = shape[0]
            by_module[LoraMerge.ModuleName(key)] = (key, 0, rows)
            for alias in (aliases(key) if aliases else ()):
                by_module[LoraMerge.ModuleName(alias)] = (key, 0, rows)
            for part in (parts(key) if parts else ()):
                by_module[LoraMerge.ModuleName(part.Name)] = (key, part.First, part.Count)
        patches: Dict[str, List[Tuple[Module, float, int]]] = {}
        files: List[LoraFile] = []
        try:
            for lora in loras:
                if lora.Weight == 0:
                    continue
                f = LoraFile(lora.Path, layout)
                files.append(f)
                modules = f.Modules(tower)
                found = 0
                for module, pair in modules.items():
                    target = by_module.get(module)
                    if target is None:
                        continue
                    found += 1
                    key, first, count = target
                    LoraMerge.Check(shapes[key], pair, count, key)
                    rank = pair.Down.Shape[0]
                    alpha = np.float32(rank if pair.Alpha is None else pair.Alpha)
                    scale = np.float32(np.float32(lora.Weight) * alpha) / np.float32(rank)
                    patches.setdefault(key, []).append((pair, float(np.float32(scale)), first))
                if modules and found == 0:
                    raise InvalidDataError(
                        f"{f.Name}: none of its {len(modules)} {layout.Describe(tower)} layers exist in this "
                        f"model; it was trained for a different architecture than {layout.Architecture}")
        except BaseException:
            for f in files:
                f.Dispose()
            raise
        return LoraPatchSet(patches, files)

    @property
    def Keys(self) -> List[str]:
        return list(self._patches)

    def Touches(self, key: str) -> bool:
        return key in self._patches

    def Apply(self, key: str, weight: DeviceTensor, dtype: Optional[HostDataType] = None) -> DeviceTensor:
        """A fresh device tensor with the key's deltas folded in, or the
        weight itself when there are none (:520-525)."""
        if key not in self._patches:
            return weight
        return LoraMerge.Merge(weight, self._patches[key], dtype)

    def Dispose(self):
        for f in self._files:
            f.Dispose()
        self._files = []
        self._patches = {}


class LazyWeights(Mapping):
    """LazyWeights (Weights/LazyWeights.cs:17-85) for device memory: a
    checkpoint's tensors under a prefix, each finished only when read, with
    its LoRA deltas folded in and at the width the graphs run at, made on the
    device and owned by the caller (a builder takes it over). The tensors are
    named by their file and prefix instead of host windows, so a tensor no
    LoRA touches goes from the mapping to the device without a host copy."""

    def __init__(self, file: SafetensorsFile, prefix: str, patches: Optional[LoraPatchSet], dataType: HostDataType,
                 device: Device):
        self._file, self._prefix = file, prefix
        self._keys = [k[len(prefix):] for k in file.Keys if k.startswith(prefix)]
        self._key_set = set(self._keys)
        self._patches, self.DataType, self.Device = patches, HostDataType(dataType), device

    def __getitem__(self, key: str) -> DeviceTensor:
        if key not in self:
            raise KeyError(key)
        if self._patches is not None and self._patches.Touches(key):
            stored = self._file.ReadDevice(self._prefix + key, self.Device)
            try:
                return self._patches.Apply(key, stored, self.DataType)
            finally:
                stored.Dispose()
        return self._file.ReadDevice(self._prefix + key, self.Device, self.DataType)

    def Unnarrowed(self, key: str) -> DeviceTensor:
        """The tensor before narrowing: the stored width, or the LoRA merge's
        (LazyWeights.cs:58-62)."""
        stored = self._file.ReadDevice(self._prefix + key, self.Device)
        if self._patches is not None and self._patches.Touches(key):
            try:
                return self._patches.Apply(key, stored)
            finally:
                stored.Dispose()
        return stored

    def Shape(self, key: str) -> Tuple[int, ...]:
        return self._file.TryGetInfo(self._prefix + key)[2]

    def __contains__(self, key) -> bool:
        return key in self._key_set

    def __iter__(self):
        return iter(self._keys)

    def __len__(self) -> int:
        return len(self._keys)

    def Dispose(self):
        """Closes the LoRA files (LazyWeights.cs:80-84); the checkpoint file
        belongs to whoever opened it."""
        if self._patches is not None:
            self._patches.Dispose()
        self._keys, self._key_set = [], set()
