"""The gate: fp64 reference, tolerance, verdict.

Follows vladmt06/kernelverify ``kernelverify/pack/verify.py:42-149``:
``qmv_inputs`` :61-69, ``moe_inputs`` :72-81, ``kv_inputs`` :84-95,
``reference_and_tolerance`` :98-105, ``judge`` :108-111, ``verify_output``
:114-118, ``judge_case`` :121-149.

Parity: closed form (max-abs at fp64 against a tolerance); pinned by the
"every member passes / every fault fails" tests that the reference runs on
the same functions (``tests/test_pack_verify.py:38-90``).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Sequence

import numpy as np

from oracle.native_ops import NATIVE_OPS
from oracle.quant_contract import QuantArtefact, dequantize


@dataclass(frozen=True)
class _Case:
    """The one field of a battery case the tolerance callables read."""

    dtype: str


@dataclass(frozen=True)
class Verdict:
    ok: bool
    err: float
    tol: float

    def __str__(self) -> str:
        return f"err {self.err:9.3e}  tol {self.tol:9.3e}  {'pass' if self.ok else 'FAIL'}"


def qmv_inputs(x: np.ndarray, w: np.ndarray, bits: int) -> dict:
    """Raw weights, not the artefact: the oracle quantizes them itself."""
    return {"x": x, "w": w, "bits": np.array([bits], dtype=np.int32)}


def moe_inputs(x: np.ndarray, router: np.ndarray,
               expert_artefacts: Sequence[QuantArtefact]) -> dict:
    """A quantized expert judged as the dense expert s*q + b (fp64)."""
    experts = np.stack([dequantize(a, np.float64) for a in expert_artefacts])
    return {"x": x, "router": router, "experts": experts}


def kv_inputs(q, k_cache, v_cache, new_k, new_v, bits: int) -> dict:
    """Raw float caches: the oracle quantizes them itself."""
    return {"q": q, "k_cache": k_cache, "v_cache": v_cache, "new_k": new_k,
            "new_v": new_v, "bits": np.array([bits], dtype=np.int32)}


def reference_and_tolerance(op_name: str, inputs: dict, dtype: str = "float16"):
    op = NATIVE_OPS[op_name]
    ref = op.reference(inputs)
    return ref, float(op.tolerance(_Case(dtype), inputs, ref))


def judge(candidate, ref: np.ndarray, tol: float) -> Verdict:
    err = float(np.max(np.abs(np.asarray(candidate).astype(np.float64) - ref)))
    return Verdict(ok=err <= tol, err=err, tol=tol)


def verify_output(op_name: str, inputs: dict, candidate, dtype: str = "float16") -> Verdict:
    ref, tol = reference_and_tolerance(op_name, inputs, dtype)
    return judge(candidate, ref, tol)


def judge_case(spec_ev, result, label: str, ref, tol: float, aux: dict | None = None,
               input_sha256: dict | None = None):
    """Judge one runner result into gate evidence; a runner that did not
    finish is a failed case carrying its status, and returns None."""
    from kernelverify_amd.pack.evidence import CaseEvidence, output_fingerprint

    prints = {"input_sha256": input_sha256} if input_sha256 else {}
    if not result.ok:
        spec_ev.cases.append(CaseEvidence(label=label, passed=False, tol=tol, **prints,
                                          detail=f"runner {result.status.value}: {result.detail}"))
        return None
    v = judge(result.outputs[0], ref, tol)
    spec_ev.cases.append(CaseEvidence(label=label, passed=v.ok, err=v.err, tol=v.tol,
                                      output_sha256=output_fingerprint(result.outputs[0]),
                                      **prints, **({"aux": aux} if aux is not None else {})))
    return v
