"""What a pack gate's ``verify()`` found, as data for its banner and for the
certificate emitter.

The class, field and property names are the reference's gate-evidence
interface (kernelverify/pack/evidence.py:65-195), because the certificate
emitter and its readers consume them; the implementation is this build's.

Shape of the record:

- `GateEvidence`: one gate run, its policy and seed protocol in words, the
  specializations it judged and its side `checks` (boolean facts such as a
  faulted artefact failing as it must);
- `SpecializationEvidence`: one compile-time specialization (the unit a
  certificate is issued for), identified by its kernel family and its
  `specialize()` substitutions, with one `CaseEvidence` per case and, aligned
  with them, the `RunCase` each ran (`calls`);
- `CaseEvidence`: a verdict, the error and tolerance behind it when one was
  computed, sha256 fingerprints of the input and output bytes (outputs are
  not bit-stable across GPU runs, so theirs describes the certifying run
  and is never a re-check criterion), and free-form `aux` numbers.

Passing cases can hand back their input arrays once judged
(`drop_verified_inputs`): their fingerprints stay, and only the bytes of a
failing case are kept for reproduction. Nothing here records time.
"""

from __future__ import annotations

import hashlib
from dataclasses import dataclass, field
from typing import Callable, Iterable, Iterator

import numpy as np

__all__ = [
    "CaseEvidence",
    "GateEvidence",
    "SpecializationEvidence",
    "banner_lines",
    "by_family",
    "input_fingerprints",
    "output_fingerprint",
    "render_banner",
]


def _sha256_of(array) -> str:
    """sha256 of an array's C-order bytes (its dtype and shape are not hashed)."""
    contiguous = np.ascontiguousarray(np.asarray(array))
    return hashlib.sha256(contiguous.tobytes()).hexdigest()


def output_fingerprint(array) -> str:
    """Fingerprint of one output, advisory: it names the certifying run's bytes."""
    return _sha256_of(array)


def input_fingerprints(inputs: dict) -> dict:
    """{input name: fingerprint}, kept for every case whatever its verdict."""
    return {name: _sha256_of(value) for name, value in inputs.items()}


@dataclass(frozen=True)
class CaseEvidence:
    """One case's verdict. ``err``/``tol`` stay None when no comparison was
    made (the runner did not finish, or the entry is a boolean check)."""

    label: str
    passed: bool
    err: float | None = None
    tol: float | None = None
    detail: str = ""
    output_sha256: str = ""
    input_sha256: dict = field(default_factory=dict)
    aux: dict = field(default_factory=dict)

    @property
    def judged(self) -> bool:
        """Whether a numerical comparison stands behind the verdict."""
        return self.err is not None and self.tol is not None

    def describe(self) -> str:
        """One banner line: the label, the numbers when there are any, the verdict."""
        verdict = "ok" if self.passed else "FAILED"
        parts = [self.label]
        if self.judged:
            parts.append(f"err={self.err:.3e} tol={self.tol:.3e}")
        parts.append(verdict)
        if self.detail and (self.judged or not self.passed):
            parts.append(f"[{self.detail}]")
        elif not self.judged and not self.passed:
            parts.append("[no verdict recorded]")
        return "  ".join(parts)


def _count(cases: Iterable[CaseEvidence]) -> tuple[int, int]:
    """(cases, of which passed)."""
    flags = [bool(c.passed) for c in cases]
    return len(flags), sum(flags)


@dataclass
class SpecializationEvidence:
    kernel: str       # kernel family, e.g. "kvp_qmv"
    operator: str     # the oracle operator the cases were judged against
    template: dict    # the specialize() substitutions
    threadgroup: tuple = (1, 1, 1)
    cases: list = field(default_factory=list)   # CaseEvidence, in run order
    calls: list = field(default_factory=list)   # RunCase per case, same order

    @property
    def key(self) -> tuple:
        """Identity within a gate: the family and the substitutions."""
        return (self.kernel, tuple(sorted((str(k), str(v)) for k, v in self.template.items())))

    @property
    def template_text(self) -> str:
        return " ".join(f"{k}={self.template[k]}" for k in sorted(self.template))

    @property
    def cases_run(self) -> int:
        return _count(self.cases)[0]

    @property
    def cases_passed(self) -> int:
        return _count(self.cases)[1]

    @property
    def ok(self) -> bool:
        run, passed = _count(self.cases)
        return run > 0 and run == passed

    def release_passing_inputs(self) -> int:
        """Empty the inputs of every call whose case passed; returns how
        many were emptied."""
        emptied = 0
        for case, call in zip(self.cases, self.calls):
            if case.passed and call is not None and call.inputs:
                call.inputs = {}
                emptied += 1
        return emptied


@dataclass
class GateEvidence:
    gate: str            # e.g. "pack_wide_qmv"
    policy: str          # the gate's case policy, in words a re-checker can follow
    seed_protocol: str   # how a re-checker draws the same inputs
    specializations: list = field(default_factory=list)  # SpecializationEvidence
    checks: list = field(default_factory=list)           # CaseEvidence

    @property
    def cases_run(self) -> int:
        return sum(s.cases_run for s in self.specializations)

    @property
    def cases_passed(self) -> int:
        return sum(s.cases_passed for s in self.specializations)

    @property
    def checks_passed(self) -> bool:
        return _count(self.checks)[0] == _count(self.checks)[1]

    @property
    def ok(self) -> bool:
        specs_green = [s.ok for s in self.specializations]
        return bool(specs_green) and all(specs_green) and self.checks_passed

    def specialization(self, kernel: str, operator: str, template: dict,
                       threadgroup: tuple) -> SpecializationEvidence:
        """The record of (``kernel``, ``template``) in this gate, added the
        first time it is asked for."""
        fresh = SpecializationEvidence(kernel=kernel, operator=operator,
                                       template=dict(template), threadgroup=tuple(threadgroup))
        known = {s.key: s for s in self.specializations}
        if fresh.key in known:
            return known[fresh.key]
        self.specializations.append(fresh)
        return fresh

    def drop_verified_inputs(self) -> None:
        """Passing cases give up their input arrays; failing ones keep them.
        Safe to call more than once."""
        for spec in self.specializations:
            spec.release_passing_inputs()


def by_family(evidences) -> dict:
    """{kernel family: [its SpecializationEvidence across the gates]}, in
    the order the families first appear."""
    families: dict = {}
    for spec in (s for ev in evidences for s in ev.specializations):
        families.setdefault(spec.kernel, []).append(spec)
    return families


def banner_lines(evidence: GateEvidence, header: str) -> Iterator[str]:
    """The gate's console banner, line by line, from the evidence alone."""
    yield header
    for check in evidence.checks:
        yield f"  check  {check.describe()}"
    for spec in evidence.specializations:
        yield (f"  {spec.kernel} {{{spec.template_text}}}: "
               f"{spec.cases_passed} of {spec.cases_run} cases ok")
        for case in spec.cases:
            yield f"      {case.describe()}"
    status = "GREEN" if evidence.ok else "NOT GREEN"
    checks = "ok" if evidence.checks_passed else "FAILED"
    yield (f"  => {evidence.gate} {status}: {evidence.cases_passed} of {evidence.cases_run} "
           f"cases ok, side checks {checks}")


def render_banner(evidence: GateEvidence, header: str,
                  out: Callable[[str], object] = print) -> None:
    for line in banner_lines(evidence, header):
        out(line)
