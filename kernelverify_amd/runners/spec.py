"""The runner door's data model: a `KernelSpec` to run and the `RunCase`s to
run it on.

The names, fields, dtype tables, extents and JSON wire keys are the
reference's runner-door interface (kernelverify/runners/spec.py: `Binding`
:79-113, extents :119-140, `LaunchSpec` :150-205, `KernelSpec` :211-265,
`RunCase` :271-342, wire form :348-359), kept so that a gate written against
that door runs here unchanged. The checks are this build's: each object
collects every problem it finds and raises one `SpecError` listing them all.

A spec is a source text, an entry point, an ordered tuple of bindings
(inputs by name, outputs by position, scalar run parameters by name; each
bound to a kernel-argument slot, its position unless `index` says otherwise)
and a launch shape whose extents a case resolves: an int, the name of a run
parameter, or a list of extents multiplied together.

Sources come in two kinds on MI355X (kernelverify_amd/runners/hip.py):

- HIP C++, compiled per spec with hiprtc for gfx950 and launched by
  `entry_point`, arguments in slot order (device pointers for tensors,
  4-byte words for scalars);
- a pack-library descriptor, ``kvpack:<family> NAME=value ...``, bound by
  name to the matching libkvpack entry point
  (kernelverify_amd/runners/library.py). The pack modules' `kernel_spec()`
  templates are descriptors with `$NAME` holes that `specialize` fills.
"""

from __future__ import annotations

import base64
import math
from dataclasses import dataclass, field
from enum import Enum
from typing import Any

import numpy as np

# dtypes a tensor binding may carry, and those a scalar is passed as (each
# padded to a 4-byte argument word)
TENSOR_DTYPES = {name: getattr(np, name) for name in
                 ("float32", "float16", "int32", "int64", "uint32")}
SCALAR_DTYPES = {name: getattr(np, name) for name in ("uint32", "int32", "float32", "float16")}

MAX_DIMENSIONS = 3
LIBRARY_PREFIX = "kvpack:"


class SpecError(ValueError):
    """A spec, or a case against a spec, that cannot run as written."""


def _raise_if(problems: list[str], what: str) -> None:
    if problems:
        raise SpecError(f"{what}: " + "; ".join(problems))


class BindingKind(str, Enum):
    INPUT = "input"
    OUTPUT = "output"
    SCALAR = "scalar"


@dataclass(frozen=True)
class Binding:
    """One kernel argument. Inputs and scalars are found by `name` in a
    case; outputs by their order among the outputs."""

    kind: BindingKind
    name: str = ""
    dtype: str = ""
    index: int | None = None

    def __post_init__(self):
        object.__setattr__(self, "kind", BindingKind(self.kind))
        problems = []
        if self.kind is not BindingKind.OUTPUT and not self.name:
            problems.append(f"{self.kind.value} bindings are looked up by name, and this one "
                            "has none")
        if self.kind is BindingKind.SCALAR and self.dtype not in SCALAR_DTYPES:
            problems.append(f"{self.dtype!r} is not a scalar dtype "
                            f"({', '.join(SCALAR_DTYPES)})")
        _raise_if(problems, f"binding {self.name or self.kind.value!r}")

    def to_json(self) -> dict:
        return {"kind": self.kind.value, "name": self.name, "dtype": self.dtype,
                "index": self.index}

    @staticmethod
    def from_json(raw: dict) -> "Binding":
        return Binding(BindingKind(raw["kind"]), raw.get("name", ""), raw.get("dtype", ""),
                       raw.get("index"))


def _as_count(value: Any) -> int | None:
    """``value`` as a Python int when it is an integer (bools are not)."""
    if isinstance(value, (bool, np.bool_)):
        return None
    if isinstance(value, (int, np.integer)):
        return int(value)
    return None


def resolve_extent(extent: Any, params: dict, where: str) -> int:
    """A positive size from an extent: an int, a run-parameter name, or a
    non-empty list or tuple of extents multiplied together."""
    if isinstance(extent, str):
        if extent not in params:
            raise SpecError(f"{where}: run parameter {extent!r} is not in this case")
        value = _as_count(params[extent])
        if value is None:
            raise SpecError(f"{where}: run parameter {extent!r} = {params[extent]!r} "
                            "is not an integer")
    elif isinstance(extent, (list, tuple)):
        if len(extent) == 0:
            raise SpecError(f"{where}: an empty list names no size")
        value = math.prod(resolve_extent(part, params, where) for part in extent)
    else:
        value = _as_count(extent)
        if value is None:
            raise SpecError(f"{where}: {extent!r} is neither an integer, a parameter name, "
                            "nor a list of them")
    if value <= 0:
        raise SpecError(f"{where}: sizes must be positive, this one is {value}")
    return value


def _extent_to_json(extent: Any) -> Any:
    return [_extent_to_json(e) for e in extent] if isinstance(extent, (list, tuple)) else extent


class LaunchMode(str, Enum):
    #: the grid counts threads; whole blocks are launched and the kernel
    #: bounds-checks the partial last one
    THREADS = "threads"
    #: the grid counts blocks (workgroups)
    THREADGROUPS = "threadgroups"


@dataclass(frozen=True)
class LaunchSpec:
    """Grid and block extents (three each) and `threadgroup_memory`, the
    dynamic LDS bytes (HIP has one dynamic segment, so at most one entry is
    used)."""

    grid: tuple = (1, 1, 1)
    threadgroup: tuple = (1, 1, 1)
    mode: LaunchMode = LaunchMode.THREADS
    threadgroup_memory: tuple = ()

    def __post_init__(self):
        object.__setattr__(self, "mode", LaunchMode(self.mode))
        problems = []
        for attr in ("grid", "threadgroup", "threadgroup_memory"):
            value = tuple(getattr(self, attr))
            object.__setattr__(self, attr, value)
            if attr != "threadgroup_memory" and len(value) != MAX_DIMENSIONS:
                problems.append(f"{attr} has {len(value)} extents, {MAX_DIMENSIONS} needed")
        _raise_if(problems, "launch")

    def resolve(self, params: dict) -> tuple[tuple, tuple, tuple]:
        """(grid, block, dynamic LDS bytes) as ints for one case."""
        out = []
        for attr in ("grid", "threadgroup", "threadgroup_memory"):
            out.append(tuple(resolve_extent(e, params, f"{attr}[{i}]")
                             for i, e in enumerate(getattr(self, attr))))
        return tuple(out)

    def to_json(self) -> dict:
        return {"grid": _extent_to_json(self.grid),
                "threadgroup": _extent_to_json(self.threadgroup),
                "mode": self.mode.value,
                "threadgroup_memory": _extent_to_json(self.threadgroup_memory)}

    @staticmethod
    def from_json(raw: dict) -> "LaunchSpec":
        return LaunchSpec(tuple(raw["grid"]), tuple(raw["threadgroup"]),
                          LaunchMode(raw.get("mode", "threads")),
                          tuple(raw.get("threadgroup_memory", ())))


@dataclass(frozen=True)
class KernelSpec:
    """A source and everything the host needs to launch it."""

    source: str
    entry_point: str
    bindings: tuple = ()
    launch: LaunchSpec = field(default_factory=LaunchSpec)
    name: str = ""

    def __post_init__(self):
        object.__setattr__(self, "bindings", tuple(self.bindings))
        problems = []
        if not self.source.strip():
            problems.append("the source is blank")
        if not self.entry_point:
            problems.append("no entry point is named")
        if self.output_count() == 0:
            problems.append("no output binding, so nothing could be judged")
        slots = [self.buffer_index(p) for p in range(len(self.bindings))]
        if any(s < 0 for s in slots):
            problems.append(f"negative argument slots {sorted(s for s in slots if s < 0)}")
        repeated = sorted({s for s in slots if slots.count(s) > 1})
        if repeated:
            problems.append(f"argument slots {repeated} are bound more than once")
        _raise_if(problems, f"kernel spec {self.name or self.entry_point!r}")

    @property
    def is_library(self) -> bool:
        """True for a pack-library descriptor, False for HIP source."""
        return self.source.lstrip().startswith(LIBRARY_PREFIX)

    def buffer_index(self, position: int) -> int:
        """The argument slot of the binding at ``position``."""
        index = self.bindings[position].index
        return position if index is None else index

    def input_names(self) -> tuple:
        return tuple(b.name for b in self.bindings if b.kind is BindingKind.INPUT)

    def output_count(self) -> int:
        return [b.kind for b in self.bindings].count(BindingKind.OUTPUT)

    def to_json(self) -> dict:
        return {"source": self.source, "entry_point": self.entry_point,
                "bindings": [b.to_json() for b in self.bindings],
                "launch": self.launch.to_json(), "name": self.name}

    @staticmethod
    def from_json(raw: dict) -> "KernelSpec":
        return KernelSpec(raw["source"], raw["entry_point"],
                          tuple(map(Binding.from_json, raw.get("bindings", ()))),
                          LaunchSpec.from_json(raw["launch"]), raw.get("name", ""))


@dataclass(eq=False)
class RunCase:
    """Input arrays by name, run parameters (scalars and extents) and one
    ``(shape, dtype)`` per output binding, in binding order."""

    inputs: dict
    params: dict = field(default_factory=dict)
    output_shapes: tuple = ()
    label: str = ""

    def __post_init__(self):
        shapes, problems = [], []
        for shape, dtype in self.output_shapes:
            shape = tuple(int(d) for d in shape)
            if dtype not in TENSOR_DTYPES:
                problems.append(f"output dtype {dtype!r} is not one of {', '.join(TENSOR_DTYPES)}")
            if min(shape, default=1) <= 0:
                problems.append(f"output shape {shape} has an empty dimension")
            shapes.append((shape, dtype))
        self.output_shapes = tuple(shapes)
        if not shapes:
            problems.append("it describes no output")
        _raise_if(problems, f"case {self.label!r}")

    def validate_against(self, spec: KernelSpec) -> None:
        """Raise unless this case supplies everything ``spec`` binds and its
        launch extents resolve."""
        problems = []
        if spec.output_count() != len(self.output_shapes):
            problems.append(f"{len(self.output_shapes)} output shapes for "
                            f"{spec.output_count()} output bindings")
        for b in spec.bindings:
            if b.kind is BindingKind.INPUT:
                if b.name not in self.inputs:
                    problems.append(f"input {b.name!r} is missing")
                elif np.asarray(self.inputs[b.name]).dtype.name not in TENSOR_DTYPES:
                    problems.append(f"input {b.name!r} is {np.asarray(self.inputs[b.name]).dtype}, "
                                    "not a tensor dtype")
            elif b.kind is BindingKind.SCALAR and b.name not in self.params:
                problems.append(f"scalar {b.name!r} is missing")
        _raise_if(problems, f"case {self.label!r} against {spec.name or spec.entry_point!r}")
        spec.launch.resolve(self.params)

    def to_json(self) -> dict:
        return {"inputs": {k: array_to_json(v) for k, v in self.inputs.items()},
                "params": self.params,
                "output_shapes": [{"shape": list(s), "dtype": d} for s, d in self.output_shapes],
                "label": self.label}

    @staticmethod
    def from_json(raw: dict) -> "RunCase":
        outs = tuple((tuple(o["shape"]), o["dtype"]) for o in raw.get("output_shapes", ()))
        return RunCase({k: array_from_json(v) for k, v in raw["inputs"].items()},
                       raw.get("params", {}), outs, raw.get("label", ""))


def array_to_json(array: np.ndarray) -> dict:
    """An array as {shape, dtype, data}, data the base64 of its C-order bytes."""
    a = np.ascontiguousarray(array)
    return {"shape": list(a.shape), "dtype": a.dtype.name,
            "data": base64.b64encode(a.tobytes()).decode("ascii")}


def array_from_json(raw: dict) -> np.ndarray:
    data = base64.b64decode(raw["data"])
    return np.frombuffer(data, dtype=raw["dtype"]).reshape(raw["shape"]).copy()
