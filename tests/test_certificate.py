"""Certificate schema, audit and per-family emission (reference:
tests/test_certificate.py, tests/test_emit_pack_certificates.py), and the
emitter's host logic on hand-built gate evidence. CPU only."""

from __future__ import annotations

import hashlib
import json
from pathlib import Path

import pytest

from kernelverify_amd.pack.evidence import CaseEvidence, GateEvidence
from kernelverify_amd.report import (
    NUMERIC,
    OWN_SOURCE,
    SCHEMA_VERSION,
    STRUCTURAL,
    WRAPPER_ASSEMBLED,
    Certificate,
    ClauseAttestation,
    PerformanceClaim,
    audit,
    emit,
    render_markdown,
)
from kernelverify_amd.report.certificate import EXTRACTED_UNVALIDATED
from tests.gates import emit_pack_certificates as E

C1 = ClauseAttestation("C1", "every intermediate at binary32 or wider", STRUCTURAL,
                       "all accumulators fp32 in the source")
C5 = ClauseAttestation("C5", "the specified formula", NUMERIC, "judged against fp64")
CERT_DIR = Path(__file__).resolve().parents[1] / "kernelverify_amd" / "pack" / "certificates"


def make(**over) -> Certificate:
    base = dict(kernel_name="k-BITS4", kernel_family="k", operator="quantized_matmul",
                translation_unit="// source\n", extraction_provenance=OWN_SOURCE,
                compile_options={"flags": ["-O3"]}, clauses=(C1, C5),
                catalogue_fingerprint="none", harness_commit="abc1234", contract_version="v",
                tolerance_model={"K": 4.0}, policy="gate", budget=4, cases_run=4,
                cases_passed=4, seed_protocol="rng(7)", chip_generation="gfx950",
                toolchain={"rocm": "7.2.0"})
    base.update(over)
    return Certificate(**base)


def test_own_source_certificate_is_clean_and_keeps_the_blocks_apart():
    cert = make()
    assert audit(cert) == []
    body = json.loads(cert.dumps())
    assert body["schema_version"] == SCHEMA_VERSION == 2
    assert set(body) >= {"byte_bound", "protocol_bound", "attestation", "validity",
                         "performance", "notes"}
    bb = body["byte_bound"]
    assert bb["translation_unit_sha256"] == hashlib.sha256(b"// source\n").hexdigest()
    assert "nothing about output values" in bb["_meaning"]
    assert "NOT asserted" in body["protocol_bound"]["_assertion"]
    assert body["protocol_bound"]["all_passed"] is True
    assert body["attestation"]["counts"] == {"numeric": 1, "source_attested": 1}
    assert body["kernel_family"] == "k"


@pytest.mark.parametrize("over, needle", [
    (dict(cases_passed=3), "1 of 4 cases failed"),
    (dict(budget=10), "budget of 10"),
    (dict(extraction_provenance=WRAPPER_ASSEMBLED), "wrapper-assembled"),
    (dict(extraction_provenance=EXTRACTED_UNVALIDATED), "not validated"),
    (dict(clauses=(C5,)), "C1"),
    (dict(performance=(PerformanceClaim(1.5, "rocBLAS", "", False),)), "without the range"),
    (dict(performance=(PerformanceClaim(1.5, "rocBLAS", "M 1-4", True),)), "sampling group"),
])
def test_audit_names_each_overclaim(over, needle):
    complaints = audit(make(**over))
    assert any(needle in c for c in complaints), complaints


def test_constructor_refuses_what_cannot_be_a_certificate():
    with pytest.raises(ValueError):
        make(extraction_provenance="guessed")
    with pytest.raises(ValueError):
        make(cases_passed=5)
    with pytest.raises(ValueError):
        make(clauses=())
    with pytest.raises(ValueError):
        ClauseAttestation("C1", "s", "vibes", "e")
    with pytest.raises(ValueError):
        ClauseAttestation("C1", "s", NUMERIC, "  ")


def test_emit_withholds_a_whole_family_and_writes_the_others(tmp_path):
    good = [make(kernel_name="a-BITS4", kernel_family="a"),
            make(kernel_name="a-BITS8", kernel_family="a")]
    bad = [make(kernel_name="b-BITS4", kernel_family="b"),
           make(kernel_name="b-BITS8", kernel_family="b", cases_passed=3)]
    report = emit(good + bad, tmp_path)
    assert sorted(p.name for p in report.written) == ["a-BITS4.certificate.json",
                                                      "a-BITS8.certificate.json"]
    assert list(report.refused) == ["b"] and not report.ok
    assert not (tmp_path / "b-BITS4.certificate.json").exists()


def test_markdown_states_the_limits_and_the_complaints():
    text = render_markdown(make())
    assert "What this does not assert" in text and "Audit complaints" not in text
    assert "Audit complaints" in render_markdown(make(cases_passed=2))


def _evidence(kernel, template, passed=(True, True), checks=()):
    ev = GateEvidence(gate="pack_test", policy="test policy", seed_protocol="rng(1)")
    spec = ev.specialization(kernel, "quantized_matmul", template, (256, 1, 1))
    for i, ok in enumerate(passed):
        spec.cases.append(CaseEvidence(label=f"case {i}", passed=ok, err=1e-3, tol=1e-2,
                                       output_sha256="0" * 64))
    ev.checks.extend(CaseEvidence(label=c, passed=ok) for c, ok in checks)
    return ev


def test_emitter_certifies_per_specialization_and_refuses_per_family(tmp_path):
    qmv = _evidence("kvp_qmv", {"T": "half", "BITS": 4, "M": 1, "R": 2})
    qmv2 = qmv.specialization("kvp_qmv", "quantized_matmul", {"T": "half", "BITS": 8, "M": 1,
                                                              "R": 2}, (256, 1, 1))
    qmv2.cases.append(CaseEvidence(label="x", passed=True, err=0.0, tol=1.0))
    kv = _evidence("kvp_kv_decode", {"T": "half", "BITS": 4, "DH": 128}, passed=(True, False))
    report = E.certify([qmv, kv], tmp_path, commit="abc1234", chip="gfx950")
    names = sorted(p.name for p in report.written)
    assert names == ["kvp_qmv-BITS4-M1-R2.certificate.json", "kvp_qmv-BITS8-M1-R2.certificate.json"]
    assert "kvp_kv_decode" in report.refused
    a, b = (json.loads((tmp_path / n).read_text()) for n in names)
    assert a["byte_bound"]["translation_unit_sha256"] != b["byte_bound"]["translation_unit_sha256"]
    assert a["byte_bound"]["extraction_provenance"] == OWN_SOURCE
    assert "dispatch_boundary" in a["validity"]["domain"]
    assert a["advisory"]["cases"][0]["margin_err_over_tol"] == pytest.approx(0.1)
    manifest = (tmp_path / "MANIFEST.md").read_text()
    assert "BITS4-M1-R2" in manifest and "Refused" in manifest


def test_a_failed_gate_check_refuses_the_family(tmp_path):
    ev = _evidence("kvp_qmv", {"T": "half", "BITS": 4, "M": 1, "R": 2},
                   checks=(("quantizer bytes identical", False),))
    report = E.certify([ev], tmp_path, commit="x", chip="gfx950")
    assert not report.written and "gate check(s) failed" in report.refused["kvp_qmv"][0]


def test_translation_unit_covers_every_family_source():
    ev = _evidence("kvp_kv_decode", {"T": "half", "BITS": 4, "DH": 128})
    tu = E.translation_unit("kvp_kv_decode", ev.specializations[0])
    assert tu.startswith("// kernelverify_amd kvp_kv_decode specialization: BITS=4 DH=128 T=half")
    for rel in (*E.FAMILY_SOURCES["kvp_kv_decode"], E.HEADER):
        assert f"// ---- kernelverify_amd/{rel} ----" in tu
    for family in E.FAMILY_SOURCES:
        assert any(c.clause == "C1" for c in E.clauses_for(family))


def test_committed_certificates_are_whole_and_indexed():
    files = sorted(CERT_DIR.glob("*.certificate.json"))
    if not files:
        pytest.skip("no certificates committed")
    manifest = (CERT_DIR / "MANIFEST.md").read_text()
    for path in files:
        body = json.loads(path.read_text())
        assert body["schema_version"] == 2
        assert body["protocol_bound"]["all_passed"] is True
        assert body["byte_bound"]["extraction_provenance"] == OWN_SOURCE
        assert any(c["clause"] == "C1" for c in body["attestation"]["clauses"])
        assert body["kernel"][len(body["kernel_family"]) + 1:] in manifest
