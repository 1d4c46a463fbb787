"""What a candidate kernel arrives as: a `KernelSpec`, and the `RunCase`s it runs.

Mirrors the reference's runner-door contract (kernelverify/runners/spec.py:
`Binding` :79-113, extents :119-140, `LaunchSpec` :150-205, `KernelSpec`
:211-265, `RunCase` :271-342, JSON wire form :348-359) so that a gate
written against that door runs here unchanged.

A spec names its source, its entry point, an ordered list of bindings
(inputs by name, outputs by position, scalar run parameters by name) and the
launch geometry in extents that each case resolves: an int, a run-parameter
name, or a list multiplied together. Shapes and scalar values travel per
case, so one spec serves a whole battery.

Two kinds of source run on MI355X (kernelverify_amd/runners/hip.py):

- HIP C++ source, compiled once per spec with hiprtc for gfx950 and launched
  by `entry_point` with the bindings as kernel arguments in buffer-index
  order (device pointers for tensors, 4-byte values for scalars);
- a pack-library descriptor, ``kvpack:<entry> NAME=value ...``, which runs
  the corresponding libkvpack entry point (kernelverify_amd/runners/library.py)
  with the bindings mapped by name. The pack modules' `kernel_spec()`
  templates are of this kind, with `$NAME` placeholders that `specialize`
  fills.
"""

from __future__ import annotations

import base64
from dataclasses import dataclass, field
from enum import Enum
from typing import Any

import numpy as np

TENSOR_DTYPES = {
    "float32": np.float32,
    "float16": np.float16,
    "int32": np.int32,
    "int64": np.int64,
    "uint32": np.uint32,
}

SCALAR_DTYPES = {
    "uint32": np.uint32,
    "int32": np.int32,
    "float32": np.float32,
    "float16": np.float16,
}

MAX_DIMENSIONS = 3


class SpecError(ValueError):
    """The spec (or a case against it) cannot run as written."""


class BindingKind(str, Enum):
    INPUT = "input"
    OUTPUT = "output"
    SCALAR = "scalar"


@dataclass(frozen=True)
class Binding:
    """One kernel argument; `index` defaults to the binding's position."""

    kind: BindingKind
    name: str = ""
    dtype: str = ""
    index: int | None = None

    def __post_init__(self):
        object.__setattr__(self, "kind", BindingKind(self.kind))
        if self.kind is BindingKind.SCALAR:
            if not self.name:
                raise SpecError("a scalar binding needs the name of a run parameter")
            if self.dtype not in SCALAR_DTYPES:
                raise SpecError(f"scalar {self.name!r} has dtype {self.dtype!r}; "
                                f"expected one of {sorted(SCALAR_DTYPES)}")
        elif self.kind is BindingKind.INPUT and not self.name:
            raise SpecError("an input binding needs the name of an input tensor")

    def to_json(self) -> dict:
        return {"kind": self.kind.value, "name": self.name, "dtype": self.dtype,
                "index": self.index}

    @staticmethod
    def from_json(raw: dict) -> "Binding":
        return Binding(kind=BindingKind(raw["kind"]), name=raw.get("name", ""),
                       dtype=raw.get("dtype", ""), index=raw.get("index"))


def resolve_extent(extent: Any, params: dict, where: str) -> int:
    """An int, a run-parameter name, or a non-empty list multiplied out."""
    if isinstance(extent, bool):
        raise SpecError(f"{where}: {extent!r} is not a valid extent")
    if isinstance(extent, int):
        value = extent
    elif isinstance(extent, str):
        if extent not in params:
            raise SpecError(f"{where}: no run parameter named {extent!r}")
        value = params[extent]
        if isinstance(value, bool) or not isinstance(value, (int, np.integer)):
            raise SpecError(f"{where}: parameter {extent!r} is {value!r}, not an integer")
        value = int(value)
    elif isinstance(extent, (list, tuple)):
        if not extent:
            raise SpecError(f"{where}: an empty product is not a size")
        value = 1
        for part in extent:
            value *= resolve_extent(part, params, where)
    else:
        raise SpecError(f"{where}: {extent!r} is not a valid extent")
    if value < 1:
        raise SpecError(f"{where}: resolved to {value}, which is not a positive size")
    return value


def _extent_json(extent: Any) -> Any:
    return list(extent) if isinstance(extent, tuple) else extent


class LaunchMode(str, Enum):
    #: the grid counts threads; the launch rounds up to whole blocks and the
    #: kernel bounds-checks its tail
    THREADS = "threads"
    #: the grid counts whole blocks (workgroups)
    THREADGROUPS = "threadgroups"


@dataclass(frozen=True)
class LaunchSpec:
    """Grid and block extents; `threadgroup_memory` is dynamic LDS in bytes
    (one entry; HIP has a single dynamic shared-memory segment)."""

    grid: tuple = (1, 1, 1)
    threadgroup: tuple = (1, 1, 1)
    mode: LaunchMode = LaunchMode.THREADS
    threadgroup_memory: tuple = ()

    def __post_init__(self):
        object.__setattr__(self, "mode", LaunchMode(self.mode))
        for name in ("grid", "threadgroup"):
            value = tuple(getattr(self, name))
            if len(value) != MAX_DIMENSIONS:
                raise SpecError(f"{name} must have {MAX_DIMENSIONS} components, got {value!r}")
            object.__setattr__(self, name, value)
        object.__setattr__(self, "threadgroup_memory", tuple(self.threadgroup_memory))

    def resolve(self, params: dict):
        grid = tuple(resolve_extent(e, params, f"grid[{i}]") for i, e in enumerate(self.grid))
        group = tuple(resolve_extent(e, params, f"threadgroup[{i}]")
                      for i, e in enumerate(self.threadgroup))
        memory = tuple(resolve_extent(e, params, f"threadgroup_memory[{i}]")
                       for i, e in enumerate(self.threadgroup_memory))
        return grid, group, memory

    def to_json(self) -> dict:
        return {"grid": [_extent_json(e) for e in self.grid],
                "threadgroup": [_extent_json(e) for e in self.threadgroup],
                "mode": self.mode.value,
                "threadgroup_memory": [_extent_json(e) for e in self.threadgroup_memory]}

    @staticmethod
    def from_json(raw: dict) -> "LaunchSpec":
        return LaunchSpec(grid=tuple(raw["grid"]), threadgroup=tuple(raw["threadgroup"]),
                          mode=LaunchMode(raw.get("mode", LaunchMode.THREADS.value)),
                          threadgroup_memory=tuple(raw.get("threadgroup_memory", ())))


LIBRARY_PREFIX = "kvpack:"


@dataclass(frozen=True)
class KernelSpec:
    """Source plus everything the host needs to launch it."""

    source: str
    entry_point: str
    bindings: tuple = ()
    launch: LaunchSpec = field(default_factory=LaunchSpec)
    name: str = ""

    def __post_init__(self):
        object.__setattr__(self, "bindings", tuple(self.bindings))
        if not self.source.strip():
            raise SpecError("kernel source is empty")
        if not self.entry_point:
            raise SpecError("kernel needs an entry point name")
        if not any(b.kind is BindingKind.OUTPUT for b in self.bindings):
            raise SpecError("a kernel with no output binding has nothing to verify")
        seen: set[int] = set()
        for position, binding in enumerate(self.bindings):
            index = position if binding.index is None else binding.index
            if index < 0:
                raise SpecError(f"buffer index {index} is negative")
            if index in seen:
                raise SpecError(f"buffer index {index} bound twice")
            seen.add(index)

    @property
    def is_library(self) -> bool:
        return self.source.lstrip().startswith(LIBRARY_PREFIX)

    def buffer_index(self, position: int) -> int:
        binding = self.bindings[position]
        return position if binding.index is None else binding.index

    def input_names(self) -> tuple:
        return tuple(b.name for b in self.bindings if b.kind is BindingKind.INPUT)

    def output_count(self) -> int:
        return sum(1 for b in self.bindings if b.kind is BindingKind.OUTPUT)

    def to_json(self) -> dict:
        return {"source": self.source, "entry_point": self.entry_point,
                "bindings": [b.to_json() for b in self.bindings],
                "launch": self.launch.to_json(), "name": self.name}

    @staticmethod
    def from_json(raw: dict) -> "KernelSpec":
        return KernelSpec(source=raw["source"], entry_point=raw["entry_point"],
                          bindings=tuple(Binding.from_json(b) for b in raw.get("bindings", ())),
                          launch=LaunchSpec.from_json(raw["launch"]), name=raw.get("name", ""))


@dataclass(eq=False)
class RunCase:
    """Inputs by name, run parameters (scalars and extents), and one
    ``(shape, dtype)`` per output binding, in binding order."""

    inputs: dict
    params: dict = field(default_factory=dict)
    output_shapes: tuple = ()
    label: str = ""

    def __post_init__(self):
        normalized = []
        for shape, dtype in self.output_shapes:
            shape = tuple(int(d) for d in shape)
            if dtype not in TENSOR_DTYPES:
                raise SpecError(f"output dtype {dtype!r} is not one of {sorted(TENSOR_DTYPES)}")
            if any(d < 1 for d in shape):
                raise SpecError(f"output shape {shape} has a non-positive dimension")
            normalized.append((shape, dtype))
        self.output_shapes = tuple(normalized)
        if not self.output_shapes:
            raise SpecError("a case needs at least one output shape")

    def validate_against(self, spec: KernelSpec) -> None:
        if spec.output_count() != len(self.output_shapes):
            raise SpecError(f"kernel binds {spec.output_count()} outputs, "
                            f"the case describes {len(self.output_shapes)}")
        for name in spec.input_names():
            if name not in self.inputs:
                raise SpecError(f"kernel binds input {name!r}, which the case does not supply")
            if str(np.asarray(self.inputs[name]).dtype) not in TENSOR_DTYPES:
                raise SpecError(f"input {name!r} has dtype {np.asarray(self.inputs[name]).dtype}, "
                                f"expected one of {sorted(TENSOR_DTYPES)}")
        for binding in spec.bindings:
            if binding.kind is BindingKind.SCALAR and binding.name not in self.params:
                raise SpecError(f"kernel binds scalar {binding.name!r}, "
                                "which the case does not supply")
        spec.launch.resolve(self.params)

    def to_json(self) -> dict:
        return {"inputs": {n: array_to_json(a) for n, a in self.inputs.items()},
                "params": self.params,
                "output_shapes": [{"shape": list(s), "dtype": d} for s, d in self.output_shapes],
                "label": self.label}

    @staticmethod
    def from_json(raw: dict) -> "RunCase":
        return RunCase(inputs={n: array_from_json(a) for n, a in raw["inputs"].items()},
                       params=raw.get("params", {}),
                       output_shapes=tuple((tuple(o["shape"]), o["dtype"])
                                           for o in raw.get("output_shapes", ())),
                       label=raw.get("label", ""))


def array_to_json(array: np.ndarray) -> dict:
    contiguous = np.ascontiguousarray(array)
    return {"shape": list(contiguous.shape), "dtype": str(contiguous.dtype),
            "data": base64.b64encode(contiguous.tobytes()).decode()}


def array_from_json(raw: dict) -> np.ndarray:
    flat = np.frombuffer(base64.b64decode(raw["data"]), dtype=np.dtype(raw["dtype"]))
    return flat.reshape(raw["shape"]).copy()
