"""The quantized-KV decode correctness gate through the runner door
(reference: bench/pack_kv_attention.py:135-215, `verify()`).

The reference's fixed cases (3 (B, H, T, DH) shapes x bits {4, 8}) with its
input regime (q and new_k at peak 0.6, caches at unit scale), run through
`HipRunner` with `kv_attention.kernel_spec()` specialised per (T, BITS, DH)
and judged against the oracle's kv_attention reference and tolerance. The
artefact check compares the GPU quantizer's cache bytes with the canonical
quantizer's. Added beyond the reference: the two widths it leaves to unit
tests (2, 3) and a T past its 1024 capacity bound.

    python -m tests.gates.pack_kv_attention
"""

from __future__ import annotations

import sys

import numpy as np

from kernelverify_amd.pack import kv_attention
from kernelverify_amd.pack.codes import pack_codes
from kernelverify_amd.pack.evidence import CaseEvidence, GateEvidence, render_banner
from kernelverify_amd.runners import HipRunner, RunCase, specialize
from oracle.inputs import kv_case
from oracle.quant_contract import QuantContract, canonical_quantize
from oracle.verify import judge_case, kv_inputs, reference_and_tolerance

VERIFY_SHAPES = [(1, 8, 512, 128), (4, 2, 64, 64), (1, 4, 300, 128)]
VERIFY_BITS = (4, 8)
EXTRA = [((1, 4, 2048, 128), 4), ((1, 4, 256, 64), 2), ((1, 4, 256, 128), 3)]
# (B, H, T, DH, HKV): grouped-query cases, H / HKV query heads per cache head
GQA = [((1, 8, 256, 128, 2), 4)]

GATE_POLICY = (
    "pack-gate fixed-case sweep: 3 fixed (B, H, T, DH) shapes x bits {4, 8}, plus T = 2048 "
    "(past the reference's 1024 capacity) at 4 bits, one case each at 2 and 3 bits and one "
    "grouped-query case (8 query heads over 2 cache heads, judged on the tiled caches), "
    "judged against the oracle's kv_attention reference and ensemble-floor tolerance; GPU "
    "quantizer cache bytes checked identical to the canonical quantizer per case."
)
SEED_PROTOCOL = (
    "np.random.default_rng(t + bits) per (shape, bits) in oracle.inputs.kv_case(): q and "
    "new_k at peak 0.6, caches and new_v N(0, 1)"
)


def quantize_cache_oracle(cache: np.ndarray, bits: int):
    h, t, dh = cache.shape
    art = canonical_quantize(cache.reshape(h * t, dh), QuantContract(bits=bits, group_size=64))
    return (pack_codes(art.q, bits).reshape(h, t, -1), art.scales.reshape(h, t, -1),
            art.biases.reshape(h, t, -1))


def gpu_cache_identical(cache: np.ndarray, bits: int, parts) -> bool:
    from kernelverify_amd.pack.quant import quantize_cache

    got = quantize_cache(cache, bits)
    return all(np.array_equal(g.reshape(p.shape), p) for g, p in zip(got, parts))


def case_arrays(b, h, t, dh, bits, hkv=None):
    """(q, k cache, v cache, new_k, new_v) the kernel reads, and the kv_inputs the
    oracle judges by: a grouped-query case's caches and new entries hold HKV
    heads, and the oracle reads them tiled to H heads (query head h reads
    cache head h // (H / HKV); tests/test_oracle_kv_gqa.py pins the tiling)."""
    q, kc, vc, nk, nv = kv_case(b, h, t, dh, seed=t + bits)
    hkv = hkv or h
    kc, vc, nk, nv = kc[:hkv], vc[:hkv], nk[:, :hkv], nv[:, :hkv]
    r = h // hkv
    judged = kv_inputs(q, np.repeat(kc, r, axis=0), np.repeat(vc, r, axis=0),
                       np.repeat(nk, r, axis=1), np.repeat(nv, r, axis=1), bits)
    return (q, kc, vc, nk, nv), judged


def verify(runner: HipRunner, *, cases=None, out=print) -> GateEvidence:
    evidence = GateEvidence(gate="pack_kv_attention", policy=GATE_POLICY,
                            seed_protocol=SEED_PROTOCOL)
    template = kv_attention.kernel_spec()
    plan = cases if cases is not None else (
        [(s, bits) for s in VERIFY_SHAPES for bits in VERIFY_BITS] + EXTRA + GQA)
    grouped: dict = {}
    for shape, bits in plan:
        b, h, t, dh = shape[:4]
        hkv = shape[4] if len(shape) > 4 else h
        (q, kc, vc, nk, nv), judged = case_arrays(b, h, t, dh, bits, hkv)
        k_parts, v_parts = quantize_cache_oracle(kc, bits), quantize_cache_oracle(vc, bits)
        label = f"B={b} H={h} T={t} DH={dh} {bits}-bit" + (f" HKV={hkv}" if hkv != h else "")
        evidence.checks.append(CaseEvidence(
            label=f"{label} GPU quantizer cache bytes identical to the canonical quantizer",
            passed=gpu_cache_identical(kc, bits, k_parts)))
        ref, tol = reference_and_tolerance("kv_attention", judged)
        subs = {"T": "half", "BITS": bits, "DH": dh}
        if (bits, dh) not in grouped:
            grouped[(bits, dh)] = (specialize(template, subs), [], [])
        _, group_cases, exp = grouped[(bits, dh)]
        spec_ev = evidence.specialization(kv_attention.KERNEL_NAME, "kv_attention", subs,
                                          (256, 1, 1))
        case = RunCase(inputs={"q": q, "k_wq": k_parts[0], "k_scales": k_parts[1],
                               "k_biases": k_parts[2], "v_wq": v_parts[0],
                               "v_scales": v_parts[1], "v_biases": v_parts[2],
                               "new_k": nk, "new_v": nv},
                       params={"b_rows": b, "n_heads": h, "t_cached": t, "n_kv_heads": hkv,
                               "t_stride": t},
                       output_shapes=[((b, h, dh), "float16")], label=label)
        group_cases.append(case)
        spec_ev.calls.append(case)
        exp.append((spec_ev, label, ref, tol))
    batches = [(spec, cs) for spec, cs, _ in grouped.values()]
    expected = [e for _, _, exp in grouped.values() for e in exp]
    results = [r for batch in runner.run_candidate(batches) for r in batch]
    for result, (spec_ev, label, ref, tol) in zip(results, expected):
        judge_case(spec_ev, result, label, ref, tol)
    evidence.drop_verified_inputs()
    render_banner(evidence, "kv correctness (runner door, kv_attention contract):", out=out)
    return evidence


if __name__ == "__main__":
    sys.exit(0 if verify(HipRunner()).ok else 1)
