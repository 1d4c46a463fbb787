"""What a run returns: a status, the output tensors, and the timing samples.

Mirrors kernelverify/runners/result.py (`RunStatus` :67-74, `Timing` :77-117,
`RunResult` :120-149, `DeviceInfo` :152-173). Execution failures are statuses,
never exceptions, so a verifier can tell a broken candidate from a wrong one:

- OK: outputs are there for the oracle.
- COMPILE_ERROR: hiprtc rejected the source (the log is in `detail`).
- LAUNCH_ERROR: the launch or the library call failed (HIP's error string).
- TIMEOUT: the case did not finish inside the runner's wall budget.
- CRASH: the isolated worker died while the case was in flight.
- INVALID_SPEC: the spec or case cannot run as written; nothing ran.
- UNSUPPORTED: no gfx950 device here; never a verdict on the kernel.

`gpu_seconds` are HIP-event intervals around each timed launch on the
runner's stream; `wall_seconds` the host time from launch to completion.
Compare candidates on `gpu_best` (interference only slows a kernel down);
`gpu_spread` says when a number should not be believed.
"""

from __future__ import annotations

import statistics
from dataclasses import dataclass, field
from enum import Enum

from kernelverify_amd.runners.spec import array_from_json, array_to_json


class RunStatus(str, Enum):
    OK = "ok"
    COMPILE_ERROR = "compile_error"
    LAUNCH_ERROR = "launch_error"
    TIMEOUT = "timeout"
    CRASH = "crash"
    INVALID_SPEC = "invalid_spec"
    UNSUPPORTED = "unsupported"


@dataclass(frozen=True)
class Timing:
    gpu_seconds: tuple = ()
    wall_seconds: tuple = ()
    warmup: int = 0

    @property
    def repeats(self) -> int:
        return len(self.gpu_seconds)

    @property
    def gpu_best(self) -> float:
        return min(self.gpu_seconds) if self.gpu_seconds else float("nan")

    @property
    def gpu_median(self) -> float:
        return statistics.median(self.gpu_seconds) if self.gpu_seconds else float("nan")

    @property
    def wall_median(self) -> float:
        return statistics.median(self.wall_seconds) if self.wall_seconds else float("nan")

    @property
    def gpu_spread(self) -> float:
        """Worst over best sample."""
        if not self.gpu_seconds or self.gpu_best <= 0.0:
            return float("nan")
        return max(self.gpu_seconds) / self.gpu_best

    def to_json(self) -> dict:
        return {"gpu_seconds": list(self.gpu_seconds), "wall_seconds": list(self.wall_seconds),
                "warmup": self.warmup}

    @staticmethod
    def from_json(raw: dict) -> "Timing":
        return Timing(gpu_seconds=tuple(raw.get("gpu_seconds", ())),
                      wall_seconds=tuple(raw.get("wall_seconds", ())),
                      warmup=int(raw.get("warmup", 0)))


@dataclass
class RunResult:
    status: RunStatus = RunStatus.OK
    outputs: list = field(default_factory=list)
    timing: Timing | None = None
    detail: str = ""
    label: str = ""

    @property
    def ok(self) -> bool:
        return self.status is RunStatus.OK

    def to_json(self) -> dict:
        return {"status": self.status.value, "outputs": [array_to_json(o) for o in self.outputs],
                "timing": self.timing.to_json() if self.timing is not None else None,
                "detail": self.detail, "label": self.label}

    @staticmethod
    def from_json(raw: dict) -> "RunResult":
        return RunResult(status=RunStatus(raw["status"]),
                         outputs=[array_from_json(o) for o in raw.get("outputs", ())],
                         timing=Timing.from_json(raw["timing"]) if raw.get("timing") else None,
                         detail=raw.get("detail", ""), label=raw.get("label", ""))


@dataclass(frozen=True)
class DeviceInfo:
    """What the runner found: the device, its limits, the library build."""

    name: str = ""
    arch: str = ""
    compute_units: int = 0
    max_threads_per_threadgroup: int = 0
    max_threadgroup_memory: int = 0
    memory_bytes: int = 0
    library: str = ""

    def to_json(self) -> dict:
        return {k: getattr(self, k) for k in DeviceInfo.__annotations__}

    @staticmethod
    def from_json(raw: dict) -> "DeviceInfo":
        return DeviceInfo(**{k: raw[k] for k in raw if k in DeviceInfo.__annotations__})
