"""Certificates for the pack kernels, one per specialization, from the three
pack gates' evidence (reference: bench/emit_pack_certificates.py:1-578).

1. Run the gates' `verify()` through `HipRunner` and keep their structured
   evidence (nothing is parsed from output).
2. Per kernel family: any failed case or gate check withholds the family's
   certificates with named reasons, and the other families still emit.
3. One `Certificate` per specialization with gate evidence. Its translation
   unit is the library's own kernel source for that family (provenance
   `own-source`: these are the bytes libkvpack.so is built from, not a
   framework's generated program, so there is no extraction to validate) led
   by a line naming the specialization, so each specialization has its own
   hash. The protocol block names the gate's real policy and case count;
   the clauses say how each was established, including where a source fact
   falls short of the clause; the validity domain states the parameter
   ranges and the routing boundary; per-case margins are advisory.
4. Audit-all-then-write-all per family (`kernelverify_amd.report.emit`), then
   a markdown manifest of everything written and refused.

No timings are recorded: certification may share the GPU, and no
performance claim is made.

    python -m tests.gates.emit_pack_certificates --out DIR [--commit SHA]
"""

from __future__ import annotations

import argparse
import platform
import subprocess
import sys
from pathlib import Path

import numpy as np

from kernelverify_amd import build as kvp_build
from kernelverify_amd.pack import kv_attention, moe_dispatch, routed_windows, wide_qmv
from kernelverify_amd.pack.evidence import GateEvidence, SpecializationEvidence, by_family
from kernelverify_amd.report import (
    NUMERIC,
    OWN_SOURCE,
    STRUCTURAL,
    Certificate,
    ClauseAttestation,
    EmitReport,
    emit,
)
from kernelverify_amd.runners import HipRunner
from oracle.native_ops import K_NATIVE, K_QUANT
from oracle.quant_contract import ENSEMBLE, QUANT_ENSEMBLE_VERSION

PKG = Path(kvp_build.__file__).resolve().parent
ROOT = PKG.parent
CERT_DIR = PKG / "pack" / "certificates"

# The sources each family's kernels and C entry points are compiled from.
FAMILY_SOURCES = {
    wide_qmv.KERNEL_NAME: wide_qmv.KERNEL_SOURCES,
    kv_attention.KERNEL_NAME: ("csrc/kv_decode.hip", "csrc/qmv_core.h", "csrc/common.h"),
    moe_dispatch.ROUTING_NAME: ("csrc/moe.hip", "csrc/qmv_core.h", "csrc/mfma_core.h",
                                "csrc/common.h"),
    moe_dispatch.DISPATCH_NAME: ("csrc/moe.hip", "csrc/qmv_core.h", "csrc/mfma_core.h",
                                 "csrc/common.h"),
}
HEADER = "../include/kvpack.h"

SPEC_KEYS = ("BITS", "DH", "M", "R", "E")


def spec_name(family: str, spec: SpecializationEvidence) -> str:
    keys = [k for k in SPEC_KEYS if k in spec.template]
    return family + "".join(f"-{k}{spec.template[k]}" for k in keys)


def translation_unit(family: str, spec: SpecializationEvidence) -> str:
    """The specialization line, then every source file of the family (and
    the C header they include) with its path."""
    subs = " ".join(f"{k}={v}" for k, v in sorted(spec.template.items()))
    parts = [f"// kernelverify_amd {family} specialization: {subs}\n"]
    for rel in (*FAMILY_SOURCES[family], HEADER):
        parts.append(f"// ---- kernelverify_amd/{rel} ----\n")
        parts.append((PKG / rel).read_text())
    return "".join(parts)


def _hipcc_version() -> str:
    try:
        proc = subprocess.run([kvp_build.HIPCC, "--version"], capture_output=True, text=True,
                              timeout=60)
        for line in proc.stdout.splitlines():
            if "version" in line.lower():
                return line.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    return "unknown"


def compile_options() -> dict:
    flags = [f for f in kvp_build.DEVICE_FLAGS if not f.startswith("-I")] + ["-I<repo>/include"]
    return {"compiler": kvp_build.HIPCC.rsplit("/", 1)[-1], "compiler_version": _hipcc_version(),
            "flags": flags}


def toolchain() -> dict:
    rocm = "unknown"
    info = Path("/opt/rocm/.info/version")
    if info.exists():
        rocm = info.read_text().strip()
    return {"rocm": rocm, "hipcc": _hipcc_version(), "python": platform.python_version(),
            "numpy": np.__version__}


_C5 = ClauseAttestation(
    clause="C5",
    statement="the specified formula, not a defensible relative",
    mechanism=NUMERIC,
    evidence="every case of the protocol block judged against the oracle's fp64 "
             "restatement of the operator within the operator's contract tolerance")


def clauses_for(family: str) -> tuple:
    """C1 from the source (what each accumulator and operand is), C5 from the
    cases, C4 from the source for the kernels that take a softmax."""
    if family == wide_qmv.KERNEL_NAME:
        c1 = ClauseAttestation(
            "C1", "every intermediate at binary32 or wider", STRUCTURAL,
            scope="fp16 activations",
            evidence="csrc/qmv.hip, qmv_core.h, qmv_mfma.hip: the codes enter the dot "
                     "products as exact fp16 values (c * 2^-24) and x as given; v_dot2_f32_f16 "
                     "and v_mfma_f32_16x16x32_f16 accumulate in fp32, and s * dot + b * "
                     "sum(x) is fp32; no fp16 intermediate")
        return (c1, _C5)
    if family == kv_attention.KERNEL_NAME:
        c1 = ClauseAttestation(
            "C1", "every intermediate at binary32 or wider", STRUCTURAL,
            scope="4- and 8-bit matrix-core kernel; the 2- and 3-bit kernel is fp32 throughout",
            evidence="csrc/kv_decode.hip: scores, softmax sums and output accumulators are "
                     "fp32 and the cache codes enter as exact fp16 values; the value-side "
                     "weight x = p * s * 2^E enters the matrix instruction as the sum of two "
                     "fp16 values (hi + lo, about 22 significant bits: within 2^-22 relative "
                     "of its fp32 value), an intermediate two bits short of binary32; every "
                     "product after it is exact and every sum fp32")
        c4 = ClauseAttestation(
            "C4", "exponential sums shifted by their own maximum", STRUCTURAL,
            evidence="csrc/kv_decode.hip: exp2 is taken of s - m with m a running maximum "
                     "that trails the slice maximum by at most 8 (base 2), so no argument "
                     "exceeds 8; the combine rescales every partial by the global maximum "
                     "over the slices and the new entry; the gate's inputs do not provoke "
                     "overflow, so this is read from the source")
        return (c1, c4, _C5)
    if family == moe_dispatch.ROUTING_NAME:
        c1 = ClauseAttestation(
            "C1", "every intermediate at binary32 or wider", STRUCTURAL,
            evidence="csrc/moe.hip: logits (given, or x . router accumulated in fp32), the "
                     "softmax and the renormalised gates are fp32")
        c4 = ClauseAttestation(
            "C4", "exponential sums shifted by their own maximum", STRUCTURAL,
            evidence="csrc/moe.hip route kernels: expf(logit - wave max of the token's "
                     "logits); read from the source, the gate's inputs do not provoke "
                     "overflow")
        return (c1, c4, _C5)
    c1 = ClauseAttestation(
        "C1", "every intermediate at binary32 or wider", STRUCTURAL,
        scope="kvp_moe_dispatch (single linear); the SwiGLU down projection has no gate",
        evidence="csrc/moe.hip: codes exact in fp16, x as given, fp32 dot products, "
                 "fp32 gate-weighted sums in slot order")
    return (c1, _C5)


def contract_version_for(family: str) -> str:
    if family == wide_qmv.KERNEL_NAME:
        return (f"MLX-affine quant contract, ensemble {QUANT_ENSEMBLE_VERSION}, "
                f"K_QUANT={K_QUANT:g} (oracle/quant_contract.py, oracle/native_ops.py)")
    if family == kv_attention.KERNEL_NAME:
        return ("kv_attention contract (oracle/native_ops.py kv_reference / kv_tolerance); "
                f"K_QUANT={K_QUANT:g} borrowed from quantized_matmul, not calibrated over "
                "the KV members")
    return f"moe_dispatch contract (oracle/native_ops.py), K_NATIVE={K_NATIVE:g}"


def tolerance_model_for(family: str) -> dict:
    if family == wide_qmv.KERNEL_NAME:
        return {"anchor": "oracle quantized_matmul fp64 reference", "K_quant": K_QUANT,
                "ensemble_version": QUANT_ENSEMBLE_VERSION, "ensemble": sorted(ENSEMBLE)}
    if family == kv_attention.KERNEL_NAME:
        return {"anchor": "oracle kv_attention fp64 reference", "K_quant": K_QUANT,
                "tolerance": "oracle.native_ops.kv_tolerance"}
    return {"anchor": "oracle moe_dispatch fp64 reference", "K_native": K_NATIVE,
            "tolerance": "oracle.native_ops.moe_tolerance"}


def domain_for(family: str, spec: SpecializationEvidence) -> dict:
    t = spec.template
    if family == wide_qmv.KERNEL_NAME:
        return {"BITS": t["BITS"], "M": t["M"], "R": t["R"],
                "d_in": "any multiple of 64 (gate evidence at 2560 and 4096)",
                "d_out": "any positive count (gate evidence at 2560 and 4096)",
                "dispatch_boundary": routed_windows.dispatch_boundary_prose(t["BITS"], t["M"])}
    if family == kv_attention.KERNEL_NAME:
        return {"BITS": t["BITS"], "DH": t["DH"],
                "T": "0 .. t_stride, no capacity bound (positions split over blocks, "
                     "partials merged by log-sum-exp); gate evidence up to 2048",
                "batch": "any B >= 1, sequences independent",
                "gqa": "n_heads / n_kv_heads in {1, 2, 4, 8}",
                "cache_semantics": "MLX-affine group-64 caches; the step's new_k / new_v "
                                   "enter at full precision"}
    if family == moe_dispatch.ROUTING_NAME:
        return {"E": t["E"], "top_k": "1 .. 8",
                "tie_rule": "ties go to the LOWER index, compared on probabilities"}
    return {"R": t["R"], "BITS": 4, "experts": "MLX-affine 4-bit group-64 expert artefacts",
            "routing_inputs": "(idx, gate) as kvp_moe_route produces them"}


def advisory_for(spec: SpecializationEvidence) -> tuple:
    rows = []
    for case in spec.cases:
        row = {"label": case.label, "output_sha256": case.output_sha256,
               "err": case.err, "tol": case.tol}
        if case.err is not None and case.tol:
            row["margin_err_over_tol"] = round(case.err / case.tol, 6)
        rows.append(row)
    return tuple(rows)


def build_certificate(family: str, spec: SpecializationEvidence, gate: GateEvidence,
                      commit: str, chip: str) -> Certificate:
    return Certificate(
        kernel_name=spec_name(family, spec),
        kernel_family=family,
        operator=spec.operator,
        translation_unit=translation_unit(family, spec),
        extraction_provenance=OWN_SOURCE,
        compile_options=compile_options(),
        clauses=clauses_for(family),
        catalogue_fingerprint="none: no mutation-scored fault catalogue has run against "
                              "this operator",
        harness_commit=commit,
        contract_version=contract_version_for(family),
        tolerance_model=tolerance_model_for(family),
        policy=gate.policy,
        budget=spec.cases_run,
        cases_run=spec.cases_run,
        cases_passed=spec.cases_passed,
        seed_protocol=gate.seed_protocol,
        chip_generation=chip,
        toolchain=toolchain(),
        domain=domain_for(family, spec),
        advisory_cases=advisory_for(spec),
        notes=(f"evidence: the {gate.gate} pack gate ({gate.cases_run} cases, "
               f"{len(gate.checks)} side checks), not a mutation-scored battery",
               "no timings recorded and no performance claim made"),
    )


def write_manifest(certs: list, refused: dict, directory: Path, commit: str) -> Path:
    lines = ["# Pack certificates", "",
             "Written by `python -m tests.gates.emit_pack_certificates` at harness commit "
             f"{commit}: one certificate per kernel specialization with gate evidence, each "
             "with its own translation-unit hash. Provenance `own-source`: the hash covers "
             "the library's own kernel sources. No certificate makes a performance claim.",
             "", "| Family | Specialization | Cases | TU sha256 (prefix) |", "|---|---|---:|---|"]
    for cert in certs:
        tu = cert.to_json()["byte_bound"]["translation_unit_sha256"][:12]
        lines.append(f"| `{cert.family}` | {cert.kernel_name[len(cert.family) + 1:] or '-'} "
                     f"| {cert.cases_passed}/{cert.cases_run} | `{tu}` |")
    if refused:
        lines += ["", "## Refused", ""]
        for family, reasons in sorted(refused.items()):
            lines.append(f"- `{family}`:")
            lines += [f"  - {r}" for r in reasons]
    path = directory / "MANIFEST.md"
    path.write_text("\n".join(lines) + "\n")
    return path


def certify(evidences: list, directory, commit: str, chip: str) -> EmitReport:
    """Evidence to certificates and manifest, withholding per family."""
    directory = Path(directory)
    gate_of = {spec.kernel: ev for ev in evidences for spec in ev.specializations}
    certs, refused = [], {}
    for family, specs in by_family(evidences).items():
        gate = gate_of[family]
        reasons = [f"{spec_name(family, s)}: failed case(s) "
                   f"{[c.label for c in s.cases if not c.passed]}" for s in specs if not s.ok]
        bad_checks = [c.label for c in gate.checks if not c.passed]
        if bad_checks:
            reasons.append(f"gate check(s) failed: {bad_checks}")
        if reasons:
            refused[family] = reasons
            continue
        certs += [build_certificate(family, s, gate, commit, chip) for s in specs]
    report = emit(certs, directory)
    for family, reasons in refused.items():
        report.refused.setdefault(family, []).extend(reasons)
    written = {p.name for p in report.written}
    write_manifest([c for c in certs if f"{c.kernel_name}.certificate.json" in written],
                   report.refused, directory, commit)
    return report


def gate_evidence(runner: HipRunner, out=print) -> list:
    from tests.gates import pack_kv_attention, pack_moe_dispatch, pack_wide_qmv

    return [pack_wide_qmv.verify(runner, out=out), pack_moe_dispatch.verify(runner, out=out),
            pack_kv_attention.verify(runner, out=out)]


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--out", default=str(CERT_DIR))
    ap.add_argument("--commit", default="",
                    help="harness commit (default: git rev-parse --short HEAD)")
    args = ap.parse_args(argv)
    commit = args.commit
    if not commit:
        proc = subprocess.run(["git", "rev-parse", "--short", "HEAD"], capture_output=True,
                              text=True, cwd=str(ROOT))
        commit = proc.stdout.strip() or "unknown"
    runner = HipRunner()
    device = runner.probe()
    chip = "unknown"
    if device is not None:
        chip = f"{device.name} ({device.arch})" if device.name.strip() else device.arch
    report = certify(gate_evidence(runner), args.out, commit, chip)
    print(f"written: {len(report.written)} certificate(s) -> {args.out}", flush=True)
    for family, reasons in sorted(report.refused.items()):
        for reason in reasons:
            print(f"refused {family}: {reason}", flush=True)
    return 0 if report.ok else 1


if __name__ == "__main__":
    sys.exit(main())
