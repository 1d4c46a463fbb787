"""A mutation battery for MoE routing: faulty routers through the MoE gate's
own cases (tests/gates/pack_moe_dispatch.py), scored by whether the gate
catches each (reference: the moe_dispatch entries of the mutation catalogue,
kernelverify/mutation/catalogue.py:166-179, whose six faults these are).

Every mutant is one run-time compiled HIP router (one wave per token: fp32
logits, softmax over all experts, top-2 by probability, renormalised gates)
with one fault switched on by a macro; the control has none and must pass.
Its indices and gates then go through the library's dispatch, as the gate's
routing outputs do, and are judged by the gate's two rules:

- routing: indices bit-exact against top-2 with ties to the lower index, on
  the rows that are not near-ties (oracle.extensions.near_tie_rows, 16 ulps);
- dispatch: the library's gather-qmv on those indices and gates within the
  moe_dispatch contract tolerance of the oracle's reference.

A mutant is CAUGHT when either rule fails on some case. The tie-break fault
expresses only on the constant_rows inputs, where every row is a near-tie
and only the dispatch rule can see it. Softmax over the chosen logits equals
the renormalised full softmax exactly, so that mutant is an expected escape.

    python -m tests.gates.battery_moe      # prints the table; exit 1 if the control fails
"""

from __future__ import annotations

import sys

import numpy as np

from kernelverify_amd.pack import moe_dispatch as moe
from kernelverify_amd.runners import (
    Binding,
    BindingKind,
    HipRunner,
    KernelSpec,
    LaunchMode,
    LaunchSpec,
    RunCase,
    specialize,
)
from oracle.extensions import near_tie_rows
from oracle.inputs import moe_case
from oracle.native_kernels import _topk_by_prob
from oracle.verify import moe_inputs, reference_and_tolerance
from tests.gates.pack_moe_dispatch import TOP_K, VERIFY_SHAPES, quantize_experts

MAX_E = 64

TEMPLATE = r"""
#ifndef LOGIT
#define LOGIT(v) (v)
#endif
#ifndef BETTER
#define BETTER(a, b) ((a) > (b))
#endif
#ifndef K_EFF
#define K_EFF 2
#endif
#ifndef OUT_IDX
#define OUT_IDX(e) (e)
#endif
#ifndef RENORM
#define RENORM 1
#endif
#ifndef TOPK_SOFTMAX
#define TOPK_SOFTMAX 0
#endif
__device__ float wave_sum64(float v) {
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ float wave_max64(float v) {
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
extern "C" __global__ void moe_route_mutant(const _Float16* x, const _Float16* router,
                                            unsigned* idx, float* gate, unsigned d_in) {
  __shared__ float lg[E];
  __shared__ float p[E];
  const unsigned t = blockIdx.x, lane = threadIdx.x;
  const _Float16* xr = x + (size_t)t * d_in;
  float mx = -__builtin_inff();
  for (unsigned e = lane; e < E; e += 64) {
    const _Float16* rr = router + (size_t)e * d_in;
    float s = 0.0f;
    for (unsigned d = 0; d < d_in; ++d) s += (float)xr[d] * (float)rr[d];
    lg[e] = LOGIT(s);
    mx = fmaxf(mx, lg[e]);
  }
  mx = wave_max64(mx);
  float l = 0.0f;
  for (unsigned e = lane; e < E; e += 64) {
    p[e] = expf(lg[e] - mx);
    l += p[e];
  }
  l = wave_sum64(l);
  for (unsigned e = lane; e < E; e += 64) p[e] /= l;
  __syncthreads();
  if (lane != 0) return;
  unsigned chosen[TOP_K];
  float w[TOP_K];
  for (unsigned k = 0; k < K_EFF; ++k) {
    int best = -1;
    for (unsigned e = 0; e < E; ++e) {
      bool taken = false;
      for (unsigned j = 0; j < k; ++j) taken |= chosen[j] == e;
      if (!taken && (best < 0 || BETTER(p[e], p[best]))) best = (int)e;
    }
    chosen[k] = (unsigned)best;
    w[k] = TOPK_SOFTMAX ? expf(lg[best] - lg[chosen[0]]) : p[best];
  }
  float sum = 0.0f;
  for (unsigned k = 0; k < K_EFF; ++k) sum += w[k];
  for (unsigned k = 0; k < TOP_K; ++k) {
    const bool live = k < K_EFF;
    const float g = live ? ((RENORM || TOPK_SOFTMAX) ? w[k] / sum : w[k]) : 0.0f;
    idx[(size_t)t * TOP_K + k] = OUT_IDX(live ? chosen[k] : chosen[0]);
    gate[(size_t)t * TOP_K + k] = g;
  }
}
"""

# name -> (macro definitions, what the fault is)
MUTANTS = {
    "control": ("", "no fault: fp32 logits, full softmax, top-2 ties low, renormalised"),
    "not-renormalised": ("#define RENORM 0\n", "top-k weights left unnormalised"),
    "expert-offset": ("#define OUT_IDX(e) (((e) + 1) % E)\n", "expert index off by one"),
    "fp16-logits": ("#define LOGIT(v) ((float)(_Float16)(v))\n",
                    "router logits rounded to fp16"),
    "top-1": ("#define K_EFF 1\n", "top-1 routing where the contract says top-2"),
    "ties-high": ("#define BETTER(a, b) ((a) >= (b))\n",
                  "tie-break to the higher index (expresses only where logits tie)"),
    "softmax-after-topk": ("#define TOPK_SOFTMAX 1\n",
                           "softmax over the chosen logits (equivalent: expected to escape)"),
}


def mutant_spec(name: str, n_experts: int) -> KernelSpec:
    defs, _ = MUTANTS[name]
    assert 2 <= TOP_K <= n_experts <= MAX_E
    return KernelSpec(
        source=f"#define E {n_experts}\n#define TOP_K {TOP_K}\n" + defs + TEMPLATE,
        entry_point="moe_route_mutant",
        name=f"moe-route-mutant-{name}-E{n_experts}",
        bindings=(Binding(BindingKind.INPUT, "x"), Binding(BindingKind.INPUT, "router"),
                  Binding(BindingKind.OUTPUT), Binding(BindingKind.OUTPUT),
                  Binding(BindingKind.SCALAR, "d_in_arg", "uint32")),
        launch=LaunchSpec(grid=("n_tokens", 1, 1), threadgroup=(64, 1, 1),
                          mode=LaunchMode.THREADGROUPS),
    )


def cases():
    """The MoE gate's plan (same shapes, modes and seeds), grouped by E."""
    grouped: dict = {}
    for n, d, e, d_ffn in VERIFY_SHAPES:
        for mode in ("normal", "constant_rows"):
            x, router, experts = moe_case(n, d, e, d_ffn, seed=n * 31 + len(mode), mode=mode)
            packed, scales, biases, arts = quantize_experts(experts)
            ref, tol = reference_and_tolerance("moe_dispatch", moe_inputs(x, router, arts))
            logits = x.astype(np.float32) @ router.astype(np.float32).T
            probs = np.exp(logits - logits.max(-1, keepdims=True))
            probs /= probs.sum(-1, keepdims=True)
            grouped.setdefault(e, []).append(dict(
                label=f"{mode} n={n} E={e}", n=n, d=d, d_ffn=d_ffn, x=x, router=router,
                packed=packed, scales=scales, biases=biases, ref=ref, tol=tol,
                want=_topk_by_prob(probs, TOP_K, tie_high=False),
                clean=~near_tie_rows(logits, TOP_K, ulps=16)))
    return grouped


def _route_case(m) -> RunCase:
    return RunCase(inputs={"x": m["x"], "router": m["router"]},
                   params={"d_in_arg": m["d"], "n_tokens": m["n"]},
                   output_shapes=[((m["n"], TOP_K), "uint32"), ((m["n"], TOP_K), "float32")],
                   label=f"routing {m['label']}")


def _dispatch_case(m, idx, gate) -> tuple:
    grid, _, rows = moe.dispatch_launch(m["d_ffn"], m["n"])
    case = RunCase(inputs={"x": m["x"], "idx": idx, "gate": gate, "w_q": m["packed"],
                           "scales": m["scales"], "biases": m["biases"]},
                   params={"d_in_arg": m["d"], "d_out_arg": m["d_ffn"], "row_blocks": grid[0],
                           "n_tokens": m["n"]},
                   output_shapes=[((m["n"], m["d_ffn"]), "float16")],
                   label=f"dispatch {m['label']}")
    return specialize(moe.dispatch_spec(), {"T": "half", "R": rows}), case


def _index_range_ok(idx, n_experts) -> bool:
    """The library's dispatch rejects an index past E; the gate would report
    that as a failed case, and so does the battery."""
    return bool(np.all(idx.astype(np.int64) < n_experts))


def run_battery(runner: HipRunner | None = None) -> dict:
    """{mutant: {"caught": bool, "by": [rules], "worst_err_over_tol": float,
    "failed": [labels]}}; worst_err_over_tol is the dispatch rule's."""
    runner = runner or HipRunner(repeats=1)
    plan = cases()
    table = {}
    for name in MUTANTS:
        worst, failed, by = 0.0, [], set()
        for e, metas in plan.items():
            routed = runner.run(mutant_spec(name, e), [_route_case(m) for m in metas]).results
            for m, res in zip(metas, routed):
                if not res.ok:
                    failed.append(f"routing {m['label']}: {res.status.value}")
                    by.add("runner")
                    worst = float("inf")
                    continue
                idx, gate = res.outputs
                clean = m["clean"]
                if not np.array_equal(idx.astype(np.int64)[clean], m["want"][clean]):
                    failed.append(f"routing {m['label']}")
                    by.add("routing")
                if not _index_range_ok(idx, e):
                    failed.append(f"dispatch {m['label']}: index out of range")
                    by.add("dispatch")
                    continue
                spec, case = _dispatch_case(m, idx, gate)
                out = runner.run(spec, [case]).results[0]
                if not out.ok:
                    failed.append(f"dispatch {m['label']}: {out.status.value}")
                    by.add("dispatch")
                    worst = float("inf")
                    continue
                err = float(np.max(np.abs(out.outputs[0].astype(np.float64) - m["ref"])))
                worst = max(worst, err / m["tol"])
                if not err <= m["tol"]:
                    failed.append(f"dispatch {m['label']}")
                    by.add("dispatch")
        table[name] = {"caught": bool(failed), "by": sorted(by), "worst_err_over_tol": worst,
                       "failed": failed}
    return table


def main() -> int:
    table = run_battery()
    print(f"{'mutant':20s} {'verdict':8s} {'rule':17s} worst err/tol  fault")
    for name, row in table.items():
        verdict = "caught" if row["caught"] else ("pass" if name == "control" else "ESCAPED")
        rule = "+".join(row["by"]) or "-"
        print(f"{name:20s} {verdict:8s} {rule:17s} {row['worst_err_over_tol']:12.3g}  "
              f"{MUTANTS[name][1]}")
    faults = [n for n in MUTANTS if n != "control"]
    print(f"caught {sum(table[n]['caught'] for n in faults)} of {len(faults)} mutants; control "
          f"{'passes' if not table['control']['caught'] else 'FAILS'}")
    return 1 if table["control"]["caught"] else 0


if __name__ == "__main__":
    sys.exit(main())
