"""`HipRunner`: the runner door on MI355X (same API as the reference's
`MetalRunner`, kernelverify/runners/metal.py:105-251).

`run(spec, cases)` binds every case, launches it `warmup` times untimed and
`repeats` times timed, and returns one `RunResult` per case in a
`BatchResult`; `run_candidate([(spec, cases), ...])` runs several specs as
one candidate; `probe()` reports the device or None. Nothing here raises
about a candidate: a spec that cannot run is INVALID_SPEC (siblings still
run), a source hiprtc rejects is COMPILE_ERROR for each of its cases, a
failed launch or library status is LAUNCH_ERROR, a case slower than
`case_timeout` is TIMEOUT, and no gfx950 device is UNSUPPORTED.

Each timed repeat is bracketed by HIP events on the runner's own stream
(`gpu_seconds`) and by the host clock from launch to completion
(`wall_seconds`). Outputs are copied back after the last repeat.

`case_timeout` is a host-clock deadline per case, checked while the case's
work is still on the device: the runner polls its stop event
(hipEventQuery) instead of blocking on it, so a kernel that never finishes
is reported as TIMEOUT. Its queue is then still busy, so the runner is
`wedged`: every later case gets TIMEOUT without touching the device, and
the timed-out case's buffers are kept alive (never freed under a kernel
that may still write them). The process cannot reclaim that queue; the
gate drivers exit non-zero when any case timed out, and a caller should
end the process. It is not re-executed in place.

Candidates run in this process, one at a time, on one stream: the kernels
under test are the pack library's and kernels compiled from source here.
The runner does not sandbox a candidate; one that writes outside its
buffers faults the device for this process.
"""

from __future__ import annotations

import time
from dataclasses import dataclass, field

from kernelverify_amd import hip, lib
from kernelverify_amd.runners import library, rtc
from kernelverify_amd.runners.result import DeviceInfo, RunResult, RunStatus, Timing
from kernelverify_amd.runners.spec import KernelSpec, RunCase, SpecError

DEFAULT_CASE_TIMEOUT = 10.0
DEFAULT_WARMUP = 1
DEFAULT_REPEATS = 5


@dataclass
class BatchResult:
    """One result per case, in case order."""

    results: list = field(default_factory=list)
    device: DeviceInfo | None = None
    stderr: str = ""
    compile_options: dict = field(default_factory=dict)

    def __iter__(self):
        return iter(self.results)

    def __len__(self) -> int:
        return len(self.results)

    def __getitem__(self, index):
        return self.results[index]

    @property
    def all_ok(self) -> bool:
        return all(r.ok for r in self.results)


def _validate(spec: KernelSpec, cases) -> str | None:
    try:
        for case in cases:
            case.validate_against(spec)
    except SpecError as error:
        return str(error)
    return None


@dataclass
class HipRunner:
    case_timeout: float = DEFAULT_CASE_TIMEOUT
    warmup: int = DEFAULT_WARMUP
    repeats: int = DEFAULT_REPEATS
    device: int = 0
    # set once a case overran case_timeout with its work still queued
    wedged: str = ""
    _abandoned: list = field(default_factory=list, repr=False)

    # -- device ------------------------------------------------------------
    def probe(self) -> DeviceInfo | None:
        """The gfx950 device this runner uses, or None."""
        if hip.device_count() <= self.device:
            return None
        try:
            import ctypes

            name, arch = ctypes.create_string_buffer(256), ctypes.create_string_buffer(64)
            cu, thr, clk = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
            lds, mem = ctypes.c_size_t(), ctypes.c_size_t()
            status = lib.load().kvp_device_info(self.device, name, 256, arch, 64, ctypes.byref(cu),
                                                ctypes.byref(thr), ctypes.byref(lds),
                                                ctypes.byref(mem), ctypes.byref(clk))
            if status != 0:
                return None
            version = lib.load().kvp_version()
            return DeviceInfo(name=name.value.decode(), arch=arch.value.decode(),
                              compute_units=cu.value, max_threads_per_threadgroup=thr.value,
                              max_threadgroup_memory=lds.value, memory_bytes=mem.value,
                              library=version.decode() if isinstance(version, bytes) else str(version))
        except (lib.LibraryMissing, OSError, hip.HipError):
            return None

    # -- running -----------------------------------------------------------
    def run_one(self, spec: KernelSpec, case: RunCase, **kwargs) -> RunResult:
        return self.run(spec, [case], **kwargs).results[0]

    def run(self, spec: KernelSpec, cases, *, warmup: int | None = None,
            repeats: int | None = None) -> BatchResult:
        return self.run_candidate([(spec, cases)], warmup=warmup, repeats=repeats)[0]

    def run_candidate(self, spec_batches, *, warmup: int | None = None,
                      repeats: int | None = None) -> list:
        warmup = self.warmup if warmup is None else warmup
        repeats = self.repeats if repeats is None else repeats
        batches = [(spec, list(cases)) for spec, cases in spec_batches]
        device = self.probe()
        out = []
        stream = None
        for spec, cases in batches:
            problem = _validate(spec, cases)
            if problem is not None:
                out.append(BatchResult([RunResult(RunStatus.INVALID_SPEC, detail=problem,
                                                  label=c.label) for c in cases], device))
                continue
            if device is None:
                out.append(BatchResult([RunResult(RunStatus.UNSUPPORTED,
                                                  detail="no gfx950 HIP device or libkvpack",
                                                  label=c.label) for c in cases], None))
                continue
            if stream is None:
                stream = hip.Stream()
            options = {} if spec.is_library else {"hiprtc": " ".join(rtc.OPTIONS)}
            out.append(BatchResult(self._run_spec(spec, cases, warmup, repeats, stream), device,
                                   compile_options=options))
        return out

    def _run_spec(self, spec: KernelSpec, cases, warmup: int, repeats: int, stream) -> list:
        module = None
        if not spec.is_library:
            try:
                module = rtc.Module(rtc.compile_source(spec.source, spec.name or "candidate.hip"),
                                    spec.entry_point)
            except rtc.CompileError as error:
                return [RunResult(RunStatus.COMPILE_ERROR, detail=str(error), label=c.label)
                        for c in cases]
            except hip.HipError as error:
                return [RunResult(RunStatus.LAUNCH_ERROR, detail=str(error), label=c.label)
                        for c in cases]
        results = []
        for case in cases:
            if self.wedged:
                results.append(RunResult(RunStatus.TIMEOUT, label=case.label,
                                         detail=f"not run: {self.wedged}"))
                continue
            results.append(self._run_case(spec, module, case, warmup, repeats, stream))
        if module is not None and not self.wedged:
            module.unload()
        elif module is not None:
            self._abandoned.append(module)
        return results

    def _run_case(self, spec, module, case: RunCase, warmup: int, repeats: int,
                  stream) -> RunResult:
        try:
            bound = library.bind(spec, case) if module is None else rtc.BoundKernel(module, spec, case)
        except SpecError as error:
            return RunResult(RunStatus.INVALID_SPEC, detail=str(error), label=case.label)
        except (lib.InvalidArgument, lib.Unsupported) as error:
            status = RunStatus.UNSUPPORTED if isinstance(error, lib.Unsupported) \
                else RunStatus.INVALID_SPEC
            return RunResult(status, detail=str(error), label=case.label)

        def failure(status_code: int) -> RunResult:
            if module is None:
                detail = lib.last_error() or f"library status {status_code}"
                st = RunStatus.UNSUPPORTED if status_code == lib.KVP_UNSUPPORTED else \
                    RunStatus.INVALID_SPEC if status_code == lib.KVP_INVALID else RunStatus.LAUNCH_ERROR
            else:
                detail = hip.runtime().hipGetErrorString(status_code).decode(errors="replace")
                st = RunStatus.LAUNCH_ERROR
            return RunResult(st, detail=detail, label=case.label)

        handle = stream.handle
        deadline = time.perf_counter() + self.case_timeout
        start, stop = hip.Event(), hip.Event()

        def overran() -> RunResult:
            self.wedged = (f"case {case.label!r} ran past case_timeout = {self.case_timeout:g} s "
                           "and its work is still queued on the device")
            self._abandoned.append(bound)
            return RunResult(RunStatus.TIMEOUT, label=case.label,
                             detail=f"still running after {self.case_timeout:g} s")

        for _ in range(warmup):
            code = bound.launch(handle)
            if code:
                return failure(code)
        stop.record(stream)
        if not stop.wait_until(deadline):
            return overran()
        gpu, wall = [], []
        for _ in range(max(repeats, 1)):
            t0 = time.perf_counter()
            start.record(stream)
            code = bound.launch(handle)
            if code:
                return failure(code)
            stop.record(stream)
            if not stop.wait_until(deadline):
                return overran()
            wall.append(time.perf_counter() - t0)
            gpu.append(start.elapsed_ms(stop) * 1e-3)
        outputs = [o.to_host() for o in bound.outputs]
        return RunResult(RunStatus.OK, outputs=outputs, label=case.label,
                         timing=Timing(tuple(gpu), tuple(wall), warmup))
