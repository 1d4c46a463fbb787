"""The runner door on MI355X: execute a candidate kernel spec over cases and
hand back outputs, a status and timing (reference: kernelverify/runners/).

`HipRunner` runs two kinds of spec: pack-library descriptors (the pack
modules' `kernel_spec()` templates, filled by `specialize`) and HIP C++
source compiled at run time with hiprtc for gfx950. Importing this package
touches no GPU; ask `HipRunner().probe()` whether a device is there.
"""

from kernelverify_amd.runners.compare import CompareReport, compare
from kernelverify_amd.runners.hip import BatchResult, HipRunner
from kernelverify_amd.runners.result import DeviceInfo, RunResult, RunStatus, Timing
from kernelverify_amd.runners.spec import (
    Binding,
    BindingKind,
    KernelSpec,
    LaunchMode,
    LaunchSpec,
    RunCase,
    SpecError,
)
from kernelverify_amd.runners.specialize import specialize

__all__ = [
    "BatchResult",
    "Binding",
    "BindingKind",
    "CompareReport",
    "DeviceInfo",
    "HipRunner",
    "KernelSpec",
    "LaunchMode",
    "LaunchSpec",
    "RunCase",
    "RunResult",
    "RunStatus",
    "SpecError",
    "Timing",
    "compare",
    "specialize",
]
