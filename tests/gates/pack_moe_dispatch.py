"""The MoE routing + dispatch correctness gate through the runner door
(reference: bench/pack_moe_dispatch.py:106-233, `verify()`).

The reference's 3 (n_tokens, d_model, n_experts, d_ffn) shapes x {normal,
constant_rows} input modes: routing runs `routing_spec()` (specialised per
E) and is judged bit-exact against the contract's top-2-by-probability rule
with ties to the lower index (outside near-tie rows, where fp32 exp may
round apart); dispatch runs `dispatch_spec()` on the routed indices and
gates and is judged against the oracle's moe_dispatch reference and
tolerance over the exact dequantized experts.

    python -m tests.gates.pack_moe_dispatch
"""

from __future__ import annotations

import sys

import numpy as np

from kernelverify_amd.pack import moe_dispatch as moe
from kernelverify_amd.pack.codes import pack_codes
from kernelverify_amd.pack.evidence import CaseEvidence, GateEvidence, output_fingerprint, render_banner
from kernelverify_amd.runners import HipRunner, RunCase, specialize
from oracle.extensions import near_tie_rows
from oracle.inputs import moe_case
from oracle.native_kernels import _topk_by_prob
from oracle.quant_contract import QuantContract, canonical_quantize
from oracle.verify import judge_case, moe_inputs, reference_and_tolerance

VERIFY_SHAPES = [(1, 512, 16, 256), (8, 512, 16, 256), (4, 256, 8, 128)]
TOP_K = 2

GATE_POLICY = (
    "pack-gate fixed-case sweep: 3 (n_tokens, d_model, n_experts, d_ffn) shapes x {normal, "
    "constant_rows} input modes; routing judged bit-exact against the contract's "
    "top-2-by-probability with ties to the lower index (near-tie rows excepted), dispatch "
    "judged against the oracle's moe_dispatch reference and tolerance over the exact "
    "dequantized experts."
)
SEED_PROTOCOL = (
    "np.random.default_rng(n_tokens * 31 + len(mode)) per (shape, mode) in "
    "oracle.inputs.moe_case(); constant_rows repeats one column so every logit ties"
)


def quantize_experts(experts: np.ndarray, bits: int = 4):
    arts = [canonical_quantize(w, QuantContract(bits=bits, group_size=64)) for w in experts]
    return (np.stack([pack_codes(a.q, bits) for a in arts]), np.stack([a.scales for a in arts]),
            np.stack([a.biases for a in arts]), arts)


def verify(runner: HipRunner, *, out=print) -> GateEvidence:
    evidence = GateEvidence(gate="pack_moe_dispatch", policy=GATE_POLICY,
                            seed_protocol=SEED_PROTOCOL)
    metas = []
    for n, d, e, d_ffn in VERIFY_SHAPES:
        for mode in ("normal", "constant_rows"):
            x, router, experts = moe_case(n, d, e, d_ffn, seed=n * 31 + len(mode), mode=mode)
            packed, scales, biases, arts = quantize_experts(experts)
            ref, tol = reference_and_tolerance("moe_dispatch", moe_inputs(x, router, arts))
            metas.append(dict(mode=mode, n=n, d=d, e=e, d_ffn=d_ffn, x=x, router=router,
                              packed=packed, scales=scales, biases=biases, ref=ref, tol=tol,
                              label=f"{mode} n={n} E={e}"))
    by_e: dict = {}
    for i, m in enumerate(metas):
        by_e.setdefault(m["e"], []).append(i)
    batches, routing_evs = [], {}
    for e, order in by_e.items():
        _, block = moe.routing_launch(metas[order[0]]["n"])
        routing_evs[e] = evidence.specialization(moe.ROUTING_NAME, "moe_dispatch", {"E": e}, block)
        cases = [RunCase(inputs={"x": metas[i]["x"], "router": metas[i]["router"]},
                         params={"d_in_arg": metas[i]["d"], "n_tokens": metas[i]["n"]},
                         output_shapes=[((metas[i]["n"], TOP_K), "uint32"),
                                        ((metas[i]["n"], TOP_K), "float32")],
                         label=f"routing {metas[i]['label']}") for i in order]
        routing_evs[e].calls.extend(cases)
        batches.append((specialize(moe.routing_spec(), {"E": e}), cases))
    for order, batch in zip(by_e.values(), runner.run_candidate(batches)):
        for i, result in zip(order, batch):
            metas[i]["route"] = result

    dispatch_cases, dispatch_meta = [], []
    dispatch_ev = None
    for m in metas:
        route, e = m["route"], m["e"]
        label = f"routing {m['label']}"
        if not route.ok:
            routing_evs[e].cases.append(CaseEvidence(
                label=label, passed=False, detail=f"runner {route.status.value}: {route.detail}"))
            continue
        idx, gate = route.outputs
        logits = m["x"].astype(np.float32) @ m["router"].astype(np.float32).T
        probs = np.exp(logits - logits.max(-1, keepdims=True))
        probs /= probs.sum(-1, keepdims=True)
        want = _topk_by_prob(probs, TOP_K, tie_high=False)
        clean = ~near_tie_rows(logits, TOP_K, ulps=16)
        exact = bool(np.array_equal(idx.astype(np.int64)[clean], want[clean]))
        routing_evs[e].cases.append(CaseEvidence(
            label=label, passed=exact, output_sha256=output_fingerprint(idx),
            detail="" if exact else "top-2 indices differ from the tie-to-lower-index rule",
            aux={"routing_exact": exact, "near_tie_rows": int((~clean).sum())}))
        grid, block, rows = moe.dispatch_launch(m["d_ffn"], m["n"])
        subs = {"T": "half", "R": rows}
        dispatch_ev = evidence.specialization(moe.DISPATCH_NAME, "moe_dispatch", subs, block)
        case = RunCase(inputs={"x": m["x"], "idx": idx, "gate": gate, "w_q": m["packed"],
                               "scales": m["scales"], "biases": m["biases"]},
                       params={"d_in_arg": m["d"], "d_out_arg": m["d_ffn"],
                               "row_blocks": grid[0], "n_tokens": m["n"]},
                       output_shapes=[((m["n"], m["d_ffn"]), "float16")],
                       label=f"dispatch {m['label']}")
        dispatch_ev.calls.append(case)
        dispatch_cases.append(case)
        dispatch_meta.append(m)
    if dispatch_cases:
        spec = specialize(moe.dispatch_spec(), dict(dispatch_ev.template))
        for m, result in zip(dispatch_meta, runner.run(spec, dispatch_cases)):
            judge_case(dispatch_ev, result, f"dispatch {m['label']}", m["ref"], m["tol"])
    evidence.drop_verified_inputs()
    render_banner(evidence, "moe correctness (runner door, moe_dispatch contract):", out=out)
    return evidence


if __name__ == "__main__":
    sys.exit(0 if verify(HipRunner()).ok else 1)
