"""A mutation battery for quantized-KV decode attention: faulty kernels through
the KV gate's own cases (tests/gates/pack_kv_attention.py), scored by
whether the gate catches each (reference: the kv seam of the mutation
catalogue, kernelverify/mutation/catalogue.py:133-182).

Every mutant is one run-time compiled HIP candidate, one wave per (sequence,
query head) over the T + 1 softmax, with one fault switched on by a macro;
the control has none and must pass. CAUGHT means at least one case's error
exceeds the kv_attention contract tolerance. An escaped mutant is a fault
these cases cannot see, reported, not hidden: the gate's inputs are small
enough that an unshifted softmax never overflows (clause C4 is therefore
attested from source).

    python -m tests.gates.battery_kv       # prints the table; exit 1 if the control fails
"""

from __future__ import annotations

import sys

import numpy as np

from kernelverify_amd.runners import (
    Binding,
    BindingKind,
    HipRunner,
    KernelSpec,
    LaunchMode,
    LaunchSpec,
    RunCase,
)
from oracle.verify import reference_and_tolerance
from tests.gates.pack_kv_attention import (
    EXTRA,
    GQA,
    VERIFY_BITS,
    VERIFY_SHAPES,
    case_arrays,
    quantize_cache_oracle,
)

MAX_T = 2048

TEMPLATE = r"""
#ifndef SHIFT
#define SHIFT(m) (m)
#endif
#ifndef HEAD_MAP
#define HEAD_MAP(h, r, hkv) ((h) / (r))
#endif
#ifndef T_SOFT
#define T_SOFT(t) ((t) + 1)
#endif
#ifndef V_BIAS
#define V_BIAS(b) (b)
#endif
#ifndef V_POS
#define V_POS(t, T) (t)
#endif
#ifndef SCORE_SCALE
#define SCORE_SCALE(dh) (1.0f / sqrtf((float)(dh)))
#endif
#ifndef SACC
#define SACC float
#endif
__device__ float code_at(const unsigned* row, unsigned d) {
  const unsigned bit = d * BITS, w = bit / 32, sh = bit % 32;
  unsigned long long pair = row[w];
  if ((bit + BITS + 31) / 32 > w + 1) pair |= (unsigned long long)row[w + 1] << 32;
  return (float)((unsigned)(pair >> sh) & ((1u << BITS) - 1u));
}
__device__ float wave_sum64(float v) {
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ float wave_max64(float v) {
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
extern "C" __global__ void kv_mutant(const _Float16* q, const unsigned* k_wq,
                                     const _Float16* k_s, const _Float16* k_b,
                                     const unsigned* v_wq, const _Float16* v_s,
                                     const _Float16* v_b, const _Float16* new_k,
                                     const _Float16* new_v, _Float16* out, unsigned n_heads,
                                     unsigned t_cached, unsigned n_kv_heads, unsigned t_stride) {
  __shared__ float p[MAX_T + 1];
  const unsigned z = blockIdx.z, b = z / n_heads, h = z % n_heads, lane = threadIdx.x;
  const unsigned hk = HEAD_MAP(h, n_heads / n_kv_heads, n_kv_heads);
  const unsigned T = t_cached, words = DH * BITS / 32, groups = DH / 64;
  const _Float16* qh = q + (size_t)z * DH;
  const _Float16* nk = new_k + ((size_t)b * n_kv_heads + hk) * DH;
  const _Float16* nv = new_v + ((size_t)b * n_kv_heads + hk) * DH;
  const float scale = SCORE_SCALE(DH);
  float mx = -__builtin_inff();
  for (unsigned t = lane; t < T + 1; t += 64) {
    SACC s = 0;
    if (t < T) {
      const size_t r = (size_t)hk * t_stride + t;
      for (unsigned d = 0; d < DH; ++d) {
        const float kv = (float)k_s[r * groups + d / 64] * code_at(k_wq + r * words, d) +
                         (float)k_b[r * groups + d / 64];
        s += (SACC)((float)qh[d] * kv);
      }
    } else {
      for (unsigned d = 0; d < DH; ++d) s += (SACC)((float)qh[d] * (float)nk[d]);
    }
    p[t] = (float)s * scale;
    mx = fmaxf(mx, p[t]);
  }
  mx = SHIFT(wave_max64(mx));
  float l = 0.0f;
  for (unsigned t = lane; t < T + 1; t += 64) {
    p[t] = t < T_SOFT(T) ? expf(p[t] - mx) : 0.0f;
    l += p[t];
  }
  l = wave_sum64(l);
  __syncthreads();
  for (unsigned d = lane; d < DH; d += 64) {
    float o = 0.0f;
    for (unsigned t = 0; t < T; ++t) {
      const size_t r = (size_t)hk * t_stride + V_POS(t, T);
      o += p[t] * ((float)v_s[r * groups + d / 64] * code_at(v_wq + r * words, d) +
                   V_BIAS((float)v_b[r * groups + d / 64]));
    }
    o += p[T] * (float)nv[d];
    out[(size_t)z * DH + d] = (_Float16)(o / l);
  }
}
"""

MUTANTS = {
    "control": ("", "no fault: the T + 1 softmax in fp32"),
    "no-max-shift": ("#define SHIFT(m) 0.0f\n", "exponentials of unshifted scores (clause C4)"),
    "new-entry-dropped": ("#define T_SOFT(t) (t)\n", "the step's own entry left out of the softmax"),
    "v-bias-dropped": ("#define V_BIAS(b) 0.0f\n", "the V groups' bias dropped"),
    "v-position-shifted": ("#define V_POS(t, T) (((t) + 1) % (T))\n",
                           "values read one position late"),
    "scale-1-over-dh": ("#define SCORE_SCALE(dh) (1.0f / (float)(dh))\n",
                        "scores scaled by 1 / DH, not 1 / sqrt(DH)"),
    "fp16-scores": ("#define SACC _Float16\n", "score dot products accumulated in fp16 (C1)"),
    "gqa-modulo": ("#define HEAD_MAP(h, r, hkv) ((h) % (hkv))\n",
                   "query head h reads KV head h mod HKV, not h / G"),
}


def mutant_spec(name: str, bits: int, dh: int) -> KernelSpec:
    defs, _ = MUTANTS[name]
    return KernelSpec(
        source=f"#define BITS {bits}\n#define DH {dh}\n#define MAX_T {MAX_T}\n" + defs + TEMPLATE,
        entry_point="kv_mutant",
        name=f"kv-mutant-{name}-{bits}bit-dh{dh}",
        bindings=tuple(Binding(BindingKind.INPUT, n) for n in (
            "q", "k_wq", "k_scales", "k_biases", "v_wq", "v_scales", "v_biases", "new_k",
            "new_v")) + (Binding(BindingKind.OUTPUT),) + tuple(
            Binding(BindingKind.SCALAR, n, "uint32")
            for n in ("n_heads", "t_cached", "n_kv_heads", "t_stride")),
        launch=LaunchSpec(grid=(1, 1, ["b_rows", "n_heads"]), threadgroup=(64, 1, 1),
                          mode=LaunchMode.THREADGROUPS),
    )


def cases():
    """The KV gate's plan (same shapes, widths and seeds), grouped by (bits, DH)."""
    plan = [(s, bits) for s in VERIFY_SHAPES for bits in VERIFY_BITS] + EXTRA + GQA
    grouped: dict = {}
    for shape, bits in plan:
        b, h, t, dh = shape[:4]
        hkv = shape[4] if len(shape) > 4 else h
        assert t <= MAX_T
        (q, kc, vc, nk, nv), judged = case_arrays(b, h, t, dh, bits, hkv)
        k_parts, v_parts = quantize_cache_oracle(kc, bits), quantize_cache_oracle(vc, bits)
        ref, tol = reference_and_tolerance("kv_attention", judged)
        case = RunCase(inputs={"q": q, "k_wq": k_parts[0], "k_scales": k_parts[1],
                               "k_biases": k_parts[2], "v_wq": v_parts[0],
                               "v_scales": v_parts[1], "v_biases": v_parts[2],
                               "new_k": nk, "new_v": nv},
                       params={"b_rows": b, "n_heads": h, "t_cached": t, "n_kv_heads": hkv,
                               "t_stride": t},
                       output_shapes=[((b, h, dh), "float16")],
                       label=f"B={b} H={h} T={t} DH={dh} HKV={hkv} {bits}-bit")
        grouped.setdefault((bits, dh), []).append((case, ref, tol))
    return grouped


def run_battery(runner: HipRunner | None = None) -> dict:
    runner = runner or HipRunner(repeats=1)
    plan = cases()
    table = {}
    for name in MUTANTS:
        worst, failed = 0.0, []
        for (bits, dh), recipe in plan.items():
            results = runner.run(mutant_spec(name, bits, dh), [c for c, _, _ in recipe]).results
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
    print(f"{'mutant':20s} {'verdict':8s} worst err/tol  fault")
    for name, row in table.items():
        verdict = "caught" if row["caught"] else ("pass" if name == "control" else "ESCAPED")
        print(f"{name:20s} {verdict:8s} {row['worst_err_over_tol']:12.3g}  {MUTANTS[name][1]}")
    faults = [n for n in MUTANTS if n != "control"]
    print(f"caught {sum(table[n]['caught'] for n in faults)} of {len(faults)} mutants; control "
          f"{'passes' if not table['control']['caught'] else 'FAILS'}")
    return 1 if table["control"]["caught"] else 0


if __name__ == "__main__":
    sys.exit(main())
