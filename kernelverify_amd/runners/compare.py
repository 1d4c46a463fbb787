"""Interleaved A/B timing with a noise canary (reference:
kernelverify/runners/compare.py:190-249).

`compare(spec_a, spec_b, cases)` binds every case once per arm, then for
each round times the reference arm (`spec_a`) and the candidate (`spec_b`)
back to back on the same stream. A round whose reference-arm samples spread
wider than `spread_limit` (max / min) is rejected: the machine moved during
it. Speedups use `gpu_best` of the accepted rounds; a report that rejected a
round, or whose arm failed, is not `ok`.
"""

from __future__ import annotations

import statistics
from dataclasses import dataclass, field

from kernelverify_amd import hip
from kernelverify_amd.runners.hip import HipRunner
from kernelverify_amd.runners.spec import KernelSpec, SpecError

DEFAULT_SPREAD_LIMIT = 1.5
DEFAULT_ROUNDS = 5


@dataclass
class RoundSample:
    round_index: int
    ref_best: float
    cand_best: float
    ref_spread: float
    cand_spread: float
    accepted: bool

    @property
    def speedup(self) -> float:
        """Reference time over candidate time; above 1.0 the candidate wins."""
        return self.ref_best / self.cand_best if self.cand_best > 0 else float("nan")


@dataclass
class CaseComparison:
    label: str
    samples: list = field(default_factory=list)

    @property
    def accepted(self) -> list:
        return [s for s in self.samples if s.accepted]

    @property
    def speedup(self) -> float:
        kept = self.accepted
        return statistics.median(s.speedup for s in kept) if kept else float("nan")

    @property
    def rejected_rounds(self) -> int:
        return len(self.samples) - len(self.accepted)


@dataclass
class CompareReport:
    spread_limit: float = DEFAULT_SPREAD_LIMIT
    cases: list = field(default_factory=list)
    failure: str = ""

    @property
    def ok(self) -> bool:
        return not self.failure and bool(self.cases) and all(
            c.rejected_rounds == 0 for c in self.cases)


class _Arm:
    """One spec with its cases bound, timed on demand."""

    def __init__(self, runner: HipRunner, spec: KernelSpec, cases, name: str):
        from kernelverify_amd.runners import library, rtc

        self.name, self.runner = name, runner
        self.module = None
        if not spec.is_library:
            self.module = rtc.Module(rtc.compile_source(spec.source), spec.entry_point)
        self.bound = [library.bind(spec, c) if self.module is None
                      else rtc.BoundKernel(self.module, spec, c) for c in cases]

    def time_case(self, index: int, stream, warmup: int, repeats: int) -> list:
        bound = self.bound[index]
        for _ in range(warmup):
            if bound.launch(stream.handle):
                raise RuntimeError(f"arm {self.name}: launch failed")
        samples = []
        start, stop = hip.Event(), hip.Event()
        for _ in range(max(repeats, 1)):
            start.record(stream)
            if bound.launch(stream.handle):
                raise RuntimeError(f"arm {self.name}: launch failed")
            stop.record(stream)
            stop.synchronize()
            samples.append(start.elapsed_ms(stop) * 1e-3)
        return samples


def compare(spec_a: KernelSpec, spec_b: KernelSpec, cases, *, rounds: int = DEFAULT_ROUNDS,
            warmup: int = 1, repeats: int = 3, spread_limit: float = DEFAULT_SPREAD_LIMIT,
            runner: HipRunner | None = None) -> CompareReport:
    runner = runner or HipRunner()
    cases = list(cases)
    report = CompareReport(spread_limit=spread_limit)
    for spec, name in ((spec_a, "A"), (spec_b, "B")):
        for case in cases:
            try:
                case.validate_against(spec)
            except SpecError as error:
                report.failure = f"arm {name}, case {case.label!r}: {error}"
                return report
    if runner.probe() is None:
        report.failure = "no gfx950 HIP device"
        return report
    try:
        arm_a = _Arm(runner, spec_a, cases, "A (reference)")
        arm_b = _Arm(runner, spec_b, cases, "B (candidate)")
        stream = hip.Stream()
        comparisons = [CaseComparison(label=c.label or f"case {i}") for i, c in enumerate(cases)]
        for r in range(rounds):
            for i in range(len(cases)):
                ref = arm_a.time_case(i, stream, warmup, repeats)
                cand = arm_b.time_case(i, stream, warmup, repeats)
                ref_spread = max(ref) / min(ref) if min(ref) > 0 else float("inf")
                comparisons[i].samples.append(RoundSample(
                    round_index=r, ref_best=min(ref), cand_best=min(cand),
                    ref_spread=ref_spread,
                    cand_spread=max(cand) / min(cand) if min(cand) > 0 else float("inf"),
                    accepted=ref_spread <= spread_limit))
        report.cases = comparisons
    except Exception as error:  # an arm that cannot hold up its half
        report.failure = str(error)
    return report
