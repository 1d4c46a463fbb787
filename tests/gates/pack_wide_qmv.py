"""The qmv correctness gate through the runner door (reference:
bench/pack_wide_qmv.py:157-245, `verify()`).

Verify-only: every case runs the shipped kernel through `HipRunner` with the
`wide_qmv.kernel_spec()` template specialised per (T, BITS, M, R) and is
judged against the oracle's quantized_matmul reference and tolerance. The
reference's artefact-identity check against `mx.quantize` becomes identity
of the GPU quantizer's bytes (`kvp_quantize_affine`) with the oracle's
canonical quantizer + packer. Timing lives in bench.py, not here.

    python -m tests.gates.pack_wide_qmv        # the full policy; exit 1 unless green
"""

from __future__ import annotations

import sys

import numpy as np

from kernelverify_amd.pack import wide_qmv
from kernelverify_amd.pack.codes import pack_codes
from kernelverify_amd.pack.evidence import CaseEvidence, GateEvidence, input_fingerprints, render_banner
from kernelverify_amd.runners import HipRunner, RunCase, specialize
from oracle.native_ops import K_QUANT
from oracle.quant_contract import QuantContract, canonical_quantize
from oracle.verify import judge_case, qmv_inputs, reference_and_tolerance

SHAPES = [(2560, 2560), (4096, 4096)]
VERIFY_BITS = (2, 3, 4, 8)
VERIFY_M = [1, 4, 5, 6, 8, 11]

GATE_POLICY = (
    "pack-gate fixed-case sweep: 2 matrix shapes at every supported bit width (2, 3, 4, 8) "
    "x M in {1, 4, 5, 6, 8, 11} x {unit, corpus} input scales per (BITS, M) "
    "specialization, judged against the oracle's quantized_matmul reference and "
    "ensemble-floor tolerance; GPU-quantizer bytes checked identical to the canonical "
    "quantizer per (shape, bits)."
)
SEED_PROTOCOL = (
    "weights: np.random.default_rng(7) per (shape, bits), N(0, 0.02) fp16; inputs: "
    "np.random.default_rng(11) per (shape, bits), drawn M-major then {unit x1, corpus "
    "x10} scale, in tests/gates/pack_wide_qmv.py verify()"
)


def weights_for(d_out: int, d_in: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((d_out, d_in)).astype(np.float32) * 0.02).astype(np.float16)


def gpu_quantizer_identical(w: np.ndarray, art, bits: int) -> bool:
    from kernelverify_amd.pack.quant import quantize

    q, s, b = quantize(w, bits)
    return (np.array_equal(q, pack_codes(art.q, bits)) and np.array_equal(s, art.scales)
            and np.array_equal(b, art.biases))


def verify(runner: HipRunner, *, shapes=SHAPES, bits_list=VERIFY_BITS, ms=VERIFY_M,
           artefact_fault=None, out=print) -> GateEvidence:
    """The gate. ``artefact_fault`` (an oracle FAULTS entry) corrupts the
    artefact the kernel reads while the reference keeps the true weights:
    a negative control that must make the gate fail."""
    evidence = GateEvidence(gate="pack_wide_qmv", policy=GATE_POLICY, seed_protocol=SEED_PROTOCOL)
    template = wide_qmv.kernel_spec()
    for d_out, d_in in shapes:
        for bits in bits_list:
            w = weights_for(d_out, d_in, seed=7)
            art = canonical_quantize(w, QuantContract(bits=bits, group_size=64))
            if artefact_fault is None:
                evidence.checks.append(CaseEvidence(
                    label=f"{d_out}x{d_in} {bits}-bit GPU quantizer bytes identical to the "
                          "canonical quantizer",
                    passed=gpu_quantizer_identical(w, art, bits)))
            served = artefact_fault(art) if artefact_fault is not None else art
            packed = pack_codes(served.q, bits)
            shared = input_fingerprints({"w_q": packed, "scales": served.scales,
                                         "biases": served.biases})
            rng = np.random.default_rng(11)
            batches, expected = [], []
            for m in ms:
                grid, block, r = wide_qmv.launch_config(d_out, m, bits, d_in)
                subs = {"T": "half", "BITS": bits, "M": m, "R": r}
                spec_ev = evidence.specialization(wide_qmv.KERNEL_NAME, "quantized_matmul",
                                                  subs, block)
                cases = []
                for tag, scale in (("unit", 1.0), ("corpus", 10.0)):
                    x = (rng.standard_normal((m, d_in)).astype(np.float32)
                         * scale).astype(np.float16)
                    ref, tol = reference_and_tolerance("quantized_matmul", qmv_inputs(x, w, bits))
                    label = f"{bits}-bit M={m} {tag} {d_out}x{d_in}"
                    case = RunCase(inputs={"x": x, "w_q": packed, "scales": served.scales,
                                           "biases": served.biases},
                                   params={"d_in_arg": d_in, "d_out_arg": d_out,
                                           "row_blocks": grid[0]},
                                   output_shapes=[((m, d_out), "float16")], label=label)
                    cases.append(case)
                    spec_ev.calls.append(case)
                    expected.append((spec_ev, label, ref, tol,
                                     {**input_fingerprints({"x": x}), **shared}))
                batches.append((specialize(template, subs), cases))
            results = [r for batch in runner.run_candidate(batches) for r in batch]
            for result, (spec_ev, label, ref, tol, sha) in zip(results, expected):
                judge_case(spec_ev, result, label, ref, tol, input_sha256=sha)
            evidence.drop_verified_inputs()
    render_banner(evidence, f"qmv correctness (runner door, contract K = {K_QUANT:g}):", out=out)
    return evidence


if __name__ == "__main__":
    sys.exit(0 if verify(HipRunner()).ok else 1)
