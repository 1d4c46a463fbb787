"""Verification certificates, schema v2 (reference: kernelverify/report/certificate.py:1-431).

A certificate ships beside a kernel specialization and says exactly what its
verification proves, in blocks that are kept apart on purpose:

- ``byte_bound``: hashes naming WHAT was verified (the translation unit, the
  compile options, the contract and the harness commit). They assert
  nothing about outputs.
- ``protocol_bound``: the verdicts. Re-running the recorded protocol on a
  matching machine reproduces them; output bits are not claimed to
  reproduce, since reduction order, compiler version and clocks move the
  last bits of GPU arithmetic legitimately.
- ``attestation``: every contract clause with HOW it was established,
  numerically by cases or by reading the source; the two are never merged
  into one "verified".
- ``validity``: where the verdicts bind (chip generation, toolchain) and the
  parameter domain the evidence covers.
- ``advisory``: per-case output fingerprints and error margins of the
  certifying run, marked as not reproducible.

Provenance tiers: the reference's three (a translation unit captured from a
framework's generator and validated or not, or one assembled by hand) and
``own-source``: the translation unit is this library's own kernel source,
the bytes built into the shipped ``libkvpack.so`` with the recorded compile
options. Nothing is extracted from a framework, so there is no extraction to
validate and no wrapper standing in for the shipped program.

The JSON layout (keys and block names) is schema 2 of the reference, so a
reader of those certificates reads these.
"""

from __future__ import annotations

import hashlib
import json
from dataclasses import dataclass, field
from pathlib import Path
from typing import Iterable

SCHEMA_VERSION = 2

# How a contract clause was established.
NUMERIC = "numeric-battery"
STRUCTURAL = "source-attestation"
MECHANISMS = (NUMERIC, STRUCTURAL)

# How the verified translation unit was obtained.
EXTRACTED_VALIDATED = "extracted-behaviorally-validated"
EXTRACTED_UNVALIDATED = "extracted-unvalidated"
WRAPPER_ASSEMBLED = "wrapper-assembled"
OWN_SOURCE = "own-source"
PROVENANCE = (EXTRACTED_VALIDATED, EXTRACTED_UNVALIDATED, WRAPPER_ASSEMBLED, OWN_SOURCE)

PROVENANCE_MEANING = {
    EXTRACTED_VALIDATED:
        "captured from the framework's own generator and shown to reproduce the "
        "framework's outputs under this protocol on the recorded toolchain; not "
        "claimed byte-identical to what the framework compiled",
    EXTRACTED_UNVALIDATED:
        "captured from the framework's own generator; the reproduction check has "
        "not run on this toolchain",
    WRAPPER_ASSEMBLED:
        "assembled by hand; it attests the wrapper, not the program a framework ships",
    OWN_SOURCE:
        "the library's own kernel source: the same bytes the shipped libkvpack.so "
        "is built from with the recorded compile options; the hash covers the "
        "kernel sources and the specialization line, not the built binary",
}

# What a source hash cannot reach, stated so that no reader assumes it does.
NOT_ATTESTED = (
    "host-side copies or conversions a caller performs before the call",
    "launch configuration chosen at run time beyond what the sources fix",
    "the compiler's code generation; compile options are recorded beside the "
    "hash, not inside it",
)


def sha256_text(text: str) -> str:
    return hashlib.sha256(text.encode()).hexdigest()


@dataclass(frozen=True)
class ClauseAttestation:
    """One contract clause and the way it was actually established."""

    clause: str
    statement: str
    mechanism: str
    evidence: str
    scope: str = ""

    def __post_init__(self):
        if self.mechanism not in MECHANISMS:
            raise ValueError(f"{self.clause}: mechanism {self.mechanism!r} not in {MECHANISMS}")
        if not self.evidence.strip():
            raise ValueError(f"{self.clause}: an attestation needs its evidence")

    def to_json(self) -> dict:
        body = {"clause": self.clause, "statement": self.statement,
                "mechanism": self.mechanism, "evidence": self.evidence}
        if self.scope:
            body["scope"] = self.scope
        return body


@dataclass(frozen=True)
class PerformanceClaim:
    """A speed ratio, scoped to the range it was measured over; a claim from
    a row that does not bind is published as directional only."""

    ratio: float
    against: str
    scope: str
    binding: bool
    sampling_group: str = ""

    def to_json(self) -> dict:
        return {"ratio": self.ratio, "against": self.against, "scope": self.scope,
                "binding": self.binding, "sampling_group": self.sampling_group,
                "status": ("binding" if self.binding
                           else "directional, pending a certified measurement")}


@dataclass(frozen=True)
class Certificate:
    """What is needed to re-check one specialization's verification claim."""

    kernel_name: str
    operator: str
    translation_unit: str
    extraction_provenance: str
    compile_options: dict
    clauses: tuple
    catalogue_fingerprint: str
    harness_commit: str
    contract_version: str
    tolerance_model: dict
    policy: str
    budget: int
    cases_run: int
    cases_passed: int
    seed_protocol: str
    chip_generation: str
    toolchain: dict
    performance: tuple = ()
    notes: tuple = ()
    kernel_family: str = ""          # certificates of one family emit together or not at all
    domain: dict = field(default_factory=dict)
    advisory_cases: tuple = ()

    def __post_init__(self):
        if self.extraction_provenance not in PROVENANCE:
            raise ValueError(f"provenance {self.extraction_provenance!r} not in {PROVENANCE}")
        if not 0 <= self.cases_passed <= self.cases_run:
            raise ValueError(f"{self.cases_passed} passed of {self.cases_run} run")
        if not self.clauses:
            raise ValueError("a certificate without clause attestations asserts nothing")

    @property
    def family(self) -> str:
        return self.kernel_family or self.kernel_name

    def to_json(self) -> dict:
        body = {
            "schema_version": SCHEMA_VERSION,
            "kernel": self.kernel_name,
            "kernel_family": self.family,
            "byte_bound": _byte_bound(self),
            "protocol_bound": _protocol_bound(self),
            "attestation": _attestation(self),
            "validity": _validity(self),
            "performance": [claim.to_json() for claim in self.performance],
            "notes": list(self.notes),
        }
        if self.advisory_cases:
            body["advisory"] = {
                "_meaning": "advisory, NOT reproducible: fingerprints and margins of "
                            "the certifying run only, never a re-check criterion "
                            "(GPU outputs are not bit-stable)",
                "cases": [dict(case) for case in self.advisory_cases],
            }
        return body

    def dumps(self) -> str:
        return json.dumps(self.to_json(), indent=2)


def _byte_bound(cert: Certificate) -> dict:
    return {
        "_meaning": "these hashes identify WHAT was verified; they assert nothing "
                    "about output values",
        "translation_unit_sha256": sha256_text(cert.translation_unit),
        "catalogue_fingerprint": cert.catalogue_fingerprint,
        "harness_commit": cert.harness_commit,
        "contract_version": cert.contract_version,
        "compile_options": cert.compile_options,
        "extraction_provenance": cert.extraction_provenance,
        "extraction_provenance_meaning": PROVENANCE_MEANING[cert.extraction_provenance],
        "not_attested_by_these_hashes": list(NOT_ATTESTED),
    }


def _protocol_bound(cert: Certificate) -> dict:
    return {
        "_assertion": "re-running the recorded protocol on a machine of the recorded "
                      "chip generation and toolchain reproduces these verdicts; output "
                      "values are NOT asserted to be identical",
        "operator": cert.operator,
        "policy": cert.policy,
        "budget_evaluations_per_operator": cert.budget,
        "cases_run": cert.cases_run,
        "cases_passed": cert.cases_passed,
        "all_passed": cert.cases_passed == cert.cases_run,
        "seed_protocol": cert.seed_protocol,
        "tolerance_model": cert.tolerance_model,
    }


def _attestation(cert: Certificate) -> dict:
    kinds = [c.mechanism for c in cert.clauses]
    return {
        "_meaning": "clauses are established in different ways; one that no case "
                    "can separate is attested from the source or not at all",
        "clauses": [c.to_json() for c in cert.clauses],
        "counts": {"numeric": kinds.count(NUMERIC), "source_attested": kinds.count(STRUCTURAL)},
    }


def _validity(cert: Certificate) -> dict:
    body = {
        "binding_on": {"chip_generation": cert.chip_generation, "toolchain": cert.toolchain},
        "elsewhere": "advisory: another chip generation or toolchain may move numerics "
                     "legitimately; a failure there is a new row to investigate, not a "
                     "refutation",
    }
    if cert.domain:
        body["domain"] = dict(cert.domain)
    return body


def audit(cert: Certificate) -> list[str]:
    """What a reviewer would object to; an empty list means the certificate
    claims no more than its evidence. Run before anything is written."""
    complaints = []
    failed = cert.cases_run - cert.cases_passed
    if failed:
        complaints.append(f"{failed} of {cert.cases_run} cases failed: no certificate is "
                          "issued for a kernel that did not pass")
    if cert.budget and cert.cases_run < cert.budget:
        complaints.append(f"{cert.cases_run} cases run against a stated budget of {cert.budget}")
    if cert.extraction_provenance == WRAPPER_ASSEMBLED:
        complaints.append("wrapper-assembled: this attests a hand-built wrapper, not the "
                          "shipped program, and must not be issued as if it did")
    if cert.extraction_provenance == EXTRACTED_UNVALIDATED:
        complaints.append("the extraction was not validated on this toolchain")
    for claim in cert.performance:
        if not claim.scope:
            complaints.append(f"a {claim.ratio}x speed claim without the range it was "
                              "measured over")
        if claim.binding and not claim.sampling_group:
            complaints.append(f"a binding {claim.ratio}x speed claim without its sampling "
                              "group of interleaved rows")
    if "C1" not in {c.clause for c in cert.clauses}:
        complaints.append("C1 (every intermediate at binary32 or wider) is unattested; "
                          "without it a precision fault would pass as a pass")
    return complaints


def render_markdown(cert: Certificate) -> str:
    """A human summary that states the limits before the claim."""
    out = [f"# Certificate: {cert.kernel_name}", "",
           f"Operator `{cert.operator}`: {cert.cases_passed}/{cert.cases_run} cases passed "
           f"under the recorded policy.", "",
           "## What this asserts", "",
           "Re-running the recorded protocol on a matching machine reproduces these verdicts.",
           "",
           "## What this does not assert", "",
           "That output values are identical: GPU arithmetic is not bit-reproducible.", "",
           "## Contract clauses", "",
           "| Clause | Requirement | Established by | Evidence |", "|---|---|---|---|"]
    for c in cert.clauses:
        how = "cases judged numerically" if c.mechanism == NUMERIC else "reading the source"
        if c.scope:
            how += f" ({c.scope})"
        out.append(f"| {c.clause} | {c.statement} | {how} | {c.evidence} |")
    out.append("")
    if cert.performance:
        out += ["## Speed", "", "| Ratio | Against | Valid for | Status |", "|---|---|---|---|"]
        for p in cert.performance:
            status = p.to_json()["status"]
            out.append(f"| {p.ratio:.2f}x | {p.against} | {p.scope} | {status} |")
        out.append("")
    tools = ", ".join(f"{k} {v}" for k, v in sorted(cert.toolchain.items()))
    out += ["## Validity", "",
            f"Binding on {cert.chip_generation} with {tools}; advisory elsewhere.", ""]
    complaints = audit(cert)
    if complaints:
        out += ["## Audit complaints", ""] + [f"- {c}" for c in complaints] + [""]
    return "\n".join(out).rstrip() + "\n"


@dataclass
class EmitReport:
    written: list = field(default_factory=list)  # paths, in order
    refused: dict = field(default_factory=dict)  # family -> reasons

    @property
    def ok(self) -> bool:
        return not self.refused


def emit(certificates: Iterable[Certificate], directory) -> EmitReport:
    """Write `<kernel>.certificate.json` files, refusing per kernel family:
    every certificate of a family is audited first and a single complaint
    withholds the whole family (named reasons in the report), while other
    families still emit. A directory never holds part of a family."""
    directory = Path(directory)
    directory.mkdir(parents=True, exist_ok=True)
    families: dict = {}
    for cert in certificates:
        families.setdefault(cert.family, []).append(cert)
    report = EmitReport()
    for family, certs in families.items():
        reasons = [f"{cert.kernel_name}: {c}" for cert in certs for c in audit(cert)]
        if reasons:
            report.refused[family] = reasons
            continue
        for cert in certs:
            path = directory / f"{cert.kernel_name}.certificate.json"
            path.write_text(cert.dumps() + "\n")
            report.written.append(path)
    return report
