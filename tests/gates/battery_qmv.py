"""A mutation battery for the qmv operator: faulty kernels through the qmv
gate's own cases, scored by whether the gate catches each (reference: the
battery / mutation catalogue kernelverify/mutation/catalogue.py:133-182,
extended to the pack operators as TODOS.md:163-170 asks).

Every mutant is one run-time compiled HIP candidate (one thread per output)
with one fault switched on by a macro; the control has none and must pass.
A mutant is CAUGHT when at least one case's error exceeds the contract
tolerance of `oracle.verify.reference_and_tolerance`; an escaped mutant is a
fault the gate cannot see at these inputs, reported as such, not hidden.

    python -m tests.gates.battery_qmv      # prints the table; exit 1 if the control fails
"""

from __future__ import annotations

import sys

import numpy as np

from kernelverify_amd.pack.codes import pack_codes
from kernelverify_amd.runners import (
    Binding,
    BindingKind,
    HipRunner,
    KernelSpec,
    LaunchMode,
    LaunchSpec,
    RunCase,
)
from oracle.quant_contract import QuantContract, canonical_quantize
from oracle.verify import qmv_inputs, reference_and_tolerance

TEMPLATE = r"""
#ifndef ACC
#define ACC float
#endif
#ifndef SCALE_GROUP
#define SCALE_GROUP(g, groups) (g)
#endif
#ifndef BIAS_TERM
#define BIAS_TERM(b, xs) ((b) * (xs))
#endif
#ifndef CODE
#define CODE(c) (c)
#endif
#ifndef XI
#define XI(i, d_in) (i)
#endif
#ifndef GROUP_ROUND
#define GROUP_ROUND(v) (v)
#endif
extern "C" __global__ void qmv_mutant(const _Float16* x, const unsigned* w_q,
                                      const _Float16* scales, const _Float16* biases,
                                      _Float16* out, unsigned d_in, unsigned d_out) {
  const unsigned row = blockIdx.x * blockDim.x + threadIdx.x;
  const unsigned m = blockIdx.y;
  if (row >= d_out) return;
  const unsigned groups = d_in / 64, words = d_in * BITS / 32;
  const unsigned* wr = w_q + (size_t)row * words;
  ACC acc = 0;
  for (unsigned g = 0; g < groups; ++g) {
    ACC dot = 0, xs = 0;
    for (unsigned j = 0; j < 64; ++j) {
      const unsigned i = g * 64 + j, bit = i * BITS, w = bit / 32, sh = bit % 32;
      unsigned long long pair = wr[w];
      if (w + 1 < words) pair |= (unsigned long long)wr[w + 1] << 32;
      const unsigned c = CODE((unsigned)(pair >> sh) & ((1u << BITS) - 1u));
      const ACC xv = (ACC)(float)x[(size_t)m * d_in + XI(i, d_in)];
      dot += xv * (ACC)(float)c;
      xs += xv;
    }
    const float s = (float)scales[(size_t)row * groups + SCALE_GROUP(g, groups)];
    const float b = (float)biases[(size_t)row * groups + g];
    acc += (ACC)GROUP_ROUND(s * (float)dot + BIAS_TERM(b, (float)xs));
  }
  out[(size_t)m * d_out + row] = (_Float16)(float)acc;
}
"""

# name -> (macro definitions, what the fault is)
MUTANTS = {
    "control": ("", "no fault: the operator's formula in fp32"),
    "fp16-accumulate": ("#define ACC _Float16\n",
                        "every sum (dot, sum(x), the row total) in fp16 (clause C1)"),
    "drop-bias": ("#define BIAS_TERM(b, xs) 0.0f\n", "the bias * sum(x) term dropped"),
    "wrong-group-scale": ("#define SCALE_GROUP(g, groups) (((g) + 1) % (groups))\n",
                          "each group takes the next group's scale"),
    "complemented-codes": ("#define CODE(c) (((1u << BITS) - 1u) - (c))\n",
                           "codes read as their complement (stream orientation)"),
    "shifted-activations": ("#define XI(i, d_in) (((i) + 1) % (d_in))\n",
                            "activation index off by one"),
    "fp16-group-partials": ("#define GROUP_ROUND(v) ((float)(_Float16)(v))\n",
                            "each group's partial rounded to fp16 before the fp32 sum"),
}

SHAPE = (512, 1024)
BITS = (4, 8)
MS = (1, 4)
SCALES = (("unit", 1.0), ("corpus", 10.0))


def mutant_spec(name: str, bits: int) -> KernelSpec:
    defs, _ = MUTANTS[name]
    return KernelSpec(
        source=f"#define BITS {bits}\n" + defs + TEMPLATE,
        entry_point="qmv_mutant",
        name=f"qmv-mutant-{name}-{bits}bit",
        bindings=(Binding(BindingKind.INPUT, "x"), Binding(BindingKind.INPUT, "w_q"),
                  Binding(BindingKind.INPUT, "scales"), Binding(BindingKind.INPUT, "biases"),
                  Binding(BindingKind.OUTPUT),
                  Binding(BindingKind.SCALAR, "d_in_arg", "uint32"),
                  Binding(BindingKind.SCALAR, "d_out_arg", "uint32")),
        launch=LaunchSpec(grid=("row_blocks", "m_rows", 1), threadgroup=(64, 1, 1),
                          mode=LaunchMode.THREADGROUPS),
    )


def cases(bits: int):
    """The qmv gate's case recipe (tests/gates/pack_wide_qmv.py) at one shape."""
    d_out, d_in = SHAPE
    rng_w = np.random.default_rng(7)
    w = (rng_w.standard_normal((d_out, d_in)).astype(np.float32) * 0.02).astype(np.float16)
    art = canonical_quantize(w, QuantContract(bits=bits, group_size=64))
    packed = pack_codes(art.q, bits)
    rng = np.random.default_rng(11)
    out = []
    for m in MS:
        for tag, scale in SCALES:
            x = (rng.standard_normal((m, d_in)).astype(np.float32) * scale).astype(np.float16)
            ref, tol = reference_and_tolerance("quantized_matmul", qmv_inputs(x, w, bits))
            case = RunCase(inputs={"x": x, "w_q": packed, "scales": art.scales,
                                   "biases": art.biases},
                           params={"d_in_arg": d_in, "d_out_arg": d_out,
                                   "row_blocks": (d_out + 63) // 64, "m_rows": m},
                           output_shapes=[((m, d_out), "float16")],
                           label=f"{bits}-bit M={m} {tag} {d_out}x{d_in}")
            out.append((case, ref, tol))
    return out


def run_battery(runner: HipRunner | None = None) -> dict:
    """{mutant: {"caught": bool, "worst_err_over_tol": float, "failed": [labels]}}."""
    runner = runner or HipRunner(repeats=1)
    table = {}
    per_bits = {bits: cases(bits) for bits in BITS}
    for name in MUTANTS:
        worst, failed = 0.0, []
        for bits, recipe in per_bits.items():
            results = runner.run(mutant_spec(name, bits), [c for c, _, _ in recipe]).results
            for res, (case, ref, tol) in zip(results, recipe):
                if not res.ok:
                    failed.append(f"{case.label}: {res.status.value}")
                    worst = float("inf")
                    continue
                err = float(np.max(np.abs(res.outputs[0].astype(np.float64) - ref)))
                worst = max(worst, err / tol)
                if not err <= tol:
                    failed.append(case.label)
        table[name] = {"caught": bool(failed), "worst_err_over_tol": worst, "failed": failed}
    return table


def main() -> int:
    table = run_battery()
    print(f"{'mutant':24s} {'verdict':8s} worst err/tol  fault")
    for name, row in table.items():
        verdict = "caught" if row["caught"] else ("pass" if name == "control" else "ESCAPED")
        print(f"{name:24s} {verdict:8s} {row['worst_err_over_tol']:12.3g}  {MUTANTS[name][1]}")
    faults = [n for n in MUTANTS if n != "control"]
    caught = sum(table[n]["caught"] for n in faults)
    print(f"caught {caught} of {len(faults)} mutants; control "
          f"{'passes' if not table['control']['caught'] else 'FAILS'}")
    return 1 if table["control"]["caught"] else 0


if __name__ == "__main__":
    sys.exit(main())
