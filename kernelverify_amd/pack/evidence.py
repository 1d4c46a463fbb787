"""Structured evidence from a pack gate's verification run (reference:
kernelverify/pack/evidence.py:65-195).

A gate's `verify()` returns a `GateEvidence`; its console banner renders from
it (`render_banner`), and anything downstream (a certificate emitter, a
report) consumes it directly instead of parsing output.

- one `SpecializationEvidence` per compile-time specialization (the unit a
  certificate is issued for), holding one `CaseEvidence` per case: the
  verdict, the error and tolerance behind it, and an advisory sha256 of the
  output bytes (GPU outputs are not bit-stable, so the fingerprint describes
  the certifying run and is never a re-check criterion);
- gate-level `checks` for side conditions that are not kernel verdicts
  (artefact identity, a negative control failing as it must).

`SpecializationEvidence.calls` keeps each case's `RunCase` beside its
verdict; `drop_verified_inputs` empties the inputs of passing cases once
judged, so only failing bytes are retained. No timing is recorded here:
verification may run under contention, and a number recorded in evidence
invites quoting.
"""

from __future__ import annotations

import hashlib
from dataclasses import dataclass, field

import numpy as np

__all__ = [
    "CaseEvidence",
    "GateEvidence",
    "SpecializationEvidence",
    "by_family",
    "input_fingerprints",
    "output_fingerprint",
    "render_banner",
]


def _array_sha256(array) -> str:
    return hashlib.sha256(np.ascontiguousarray(np.asarray(array)).tobytes()).hexdigest()


def output_fingerprint(array) -> str:
    """Advisory sha256 of the output bytes from the certifying run."""
    return _array_sha256(array)


def input_fingerprints(inputs: dict) -> dict:
    """sha256 per input array: which bytes ran, kept for every case."""
    return {name: _array_sha256(array) for name, array in inputs.items()}


@dataclass(frozen=True)
class CaseEvidence:
    """One case's verdict; `err`/`tol` are None when nothing numerical was
    judged (a runner failure, or a boolean check)."""

    label: str
    passed: bool
    err: float | None = None
    tol: float | None = None
    detail: str = ""
    output_sha256: str = ""
    input_sha256: dict = field(default_factory=dict)
    aux: dict = field(default_factory=dict)


@dataclass
class SpecializationEvidence:
    kernel: str        # kernel family, e.g. "kvp_qmv"
    operator: str      # the operator the cases were judged against
    template: dict     # the specialize() substitutions
    threadgroup: tuple = (1, 1, 1)
    cases: list = field(default_factory=list)   # CaseEvidence
    calls: list = field(default_factory=list)   # RunCase, aligned with cases

    @property
    def cases_run(self) -> int:
        return len(self.cases)

    @property
    def cases_passed(self) -> int:
        return sum(1 for c in self.cases if c.passed)

    @property
    def ok(self) -> bool:
        return bool(self.cases) and self.cases_passed == self.cases_run


@dataclass
class GateEvidence:
    gate: str
    policy: str
    seed_protocol: str
    specializations: list = field(default_factory=list)
    checks: list = field(default_factory=list)

    @property
    def cases_run(self) -> int:
        return sum(s.cases_run for s in self.specializations)

    @property
    def cases_passed(self) -> int:
        return sum(s.cases_passed for s in self.specializations)

    @property
    def checks_passed(self) -> bool:
        return all(c.passed for c in self.checks)

    @property
    def ok(self) -> bool:
        return (bool(self.specializations) and all(s.ok for s in self.specializations)
                and self.checks_passed)

    def specialization(self, kernel: str, operator: str, template: dict,
                       threadgroup: tuple) -> SpecializationEvidence:
        """The bucket for `template`, created on first use."""
        for existing in self.specializations:
            if existing.kernel == kernel and existing.template == template:
                return existing
        created = SpecializationEvidence(kernel=kernel, operator=operator, template=dict(template),
                                         threadgroup=tuple(threadgroup))
        self.specializations.append(created)
        return created

    def drop_verified_inputs(self) -> None:
        """Passing cases give up their input arrays (their sha256 stays);
        failing cases keep theirs. Idempotent."""
        for spec in self.specializations:
            for case, call in zip(spec.cases, spec.calls):
                if case.passed and call is not None:
                    call.inputs = {}


def by_family(evidences) -> dict:
    families: dict = {}
    for evidence in evidences:
        for spec in evidence.specializations:
            families.setdefault(spec.kernel, []).append(spec)
    return families


def _case_line(case: CaseEvidence) -> str:
    if case.err is None or case.tol is None:
        verdict = "pass" if case.passed else f"FAIL: {case.detail or 'no verdict'}"
        return f"{case.label}  {verdict}"
    line = (f"{case.label}  err {case.err:9.3e}  tol {case.tol:9.3e}  "
            f"{'pass' if case.passed else 'FAIL'}")
    return line + (f"  ({case.detail})" if case.detail else "")


def render_banner(evidence: GateEvidence, header: str, out=print) -> None:
    """The gate's console banner, rendered from the evidence alone."""
    out(header)
    for check in evidence.checks:
        out(f"  [check] {_case_line(check)}")
    for spec in evidence.specializations:
        joined = " ".join(f"{k}={v}" for k, v in sorted(spec.template.items()))
        out(f"  {spec.kernel} [{joined}] {spec.cases_passed}/{spec.cases_run} passed")
        for case in spec.cases:
            out(f"    {_case_line(case)}")
    verdict = "green" if evidence.ok else "NOT GREEN"
    out(f"  gate {evidence.gate}: {evidence.cases_passed}/{evidence.cases_run} cases, "
        f"checks {'pass' if evidence.checks_passed else 'FAIL'} -> {verdict}")
