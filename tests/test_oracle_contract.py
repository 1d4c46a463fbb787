"""Pins of the oracle's CPU control paths, their fault seams and the MoE
tolerances (oracle/floor.py, oracle/native_kernels.py, oracle/native_ops.py
``moe_reference``/``moe_tolerance``, oracle/extensions.py
``moe_linear_reference``/``moe_linear_tolerance``).

What fixes each of them independently of its own formula:

- ``max_abs_error`` / ``floored_tolerance``: known answers (empty input,
  a planted difference, broadcasting, the max of the two terms).
- The three CPU controls (``quantized_matmul``, ``kv_attention``,
  ``moe_dispatch``) agree with the fp64 references at the reference's own
  bounds (vladmt06/kernelverify ``tests/test_native_ops.py:37-42``: qmm
  < 5e-2; ``:115-122``: kv < 5e-3; ``:57-75``: moe < 1e-4), pass their own
  ensemble tolerance over a sampled case set (``:190-204``), and every
  non-equivalent seam is rejected by that tolerance on at least one sampled
  case (``:78-100``); the two equivalent seams (softmax after top-k, ties to
  the higher index on continuous draws) stay equivalent (``:170-187``).
- ``moe_reference``: an independent torch fp64 restatement of the routing
  contract (softmax, ``torch.sort(stable=True)``, renormalise, combine), in
  place of the reference's MLX cross-check, which needs Apple hardware.
- ``moe_tolerance`` and ``moe_linear_tolerance``: their members pass, and
  planted mistakes (one slot's gate dropped, gates not applied, a wrong
  expert, a transposed expert, the combine accumulated in fp16) exceed them.
- ``moe_linear_reference``: a closed form on experts that dequantize to
  scaled permutation matrices (a transposed expert or a wrong index fails
  it), and equality with ``moe_reference`` on the same routing.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.extensions import artefact_from_arrays, moe_linear_reference, moe_linear_tolerance
from oracle.floor import floored_tolerance, max_abs_error
from oracle.native_kernels import (
    kv_attention,
    moe_dispatch,
    quantized_matmul,
    quantized_matmul_artefact,
)
from oracle.native_ops import (
    MOE_MEMBERS,
    NATIVE_OPS,
    moe_reference,
    moe_tolerance,
    qmm_reference_artefact,
    qmm_tolerance_artefact,
    route_probs,
)
from oracle.quant_contract import QuantContract, canonical_quantize, dequantize
from oracle.verify import _Case


# ---------------------------------------------------------------------------
# the verdict formula
# ---------------------------------------------------------------------------
def test_max_abs_error_known_answers():
    assert max_abs_error(np.zeros(0), np.zeros(0)) == 0.0
    assert max_abs_error(np.array([1.0, 2.0, 3.0]), np.array([1.0, 2.5, 2.0])) == 1.0
    assert max_abs_error(np.float16(1.0), np.array([[1.0, 0.25]])) == 0.75
    assert max_abs_error(np.array([-4.0]), np.array([4.0])) == 8.0


def test_floored_tolerance_is_the_max_of_its_two_terms():
    ref = np.array([1.0, -2.0])
    members = [ref + 0.01, ref - 0.03]
    assert floored_tolerance(0.5, 4.0, iter(members), ref) == 0.5
    assert floored_tolerance(0.05, 4.0, iter(members), ref) == pytest.approx(0.12, rel=1e-12)


# ---------------------------------------------------------------------------
# the reference test suite's input makers (tests/test_native_ops.py:25-39, 103-111)
# ---------------------------------------------------------------------------
def qmm_case(rng, b=2, d_in=256, d_out=32, bits=4, dtype=np.float16, x_scale=1.0):
    x = (rng.standard_normal((b, d_in)) * x_scale).astype(dtype)
    w = (rng.standard_normal((d_out, d_in)).astype(np.float32) * 0.05).astype(dtype)
    return {"x": x, "w": w, "bits": np.array([bits], dtype=np.int32)}


def kv_case(rng, b=2, h=2, t=64, dh=64, bits=4, dtype=np.float16):
    return {
        "q": (rng.standard_normal((b, h, dh)).astype(np.float32) * 0.2).astype(dtype),
        "k_cache": (rng.standard_normal((h, t, dh)).astype(np.float32) * 3).astype(dtype),
        "v_cache": (rng.standard_normal((h, t, dh)).astype(np.float32) * 3).astype(dtype),
        "new_k": (rng.standard_normal((b, h, dh)).astype(np.float32) * 0.2).astype(dtype),
        "new_v": (rng.standard_normal((b, h, dh)).astype(np.float32) * 3).astype(dtype),
        "bits": np.array([bits], dtype=np.int32),
    }


def moe_case(rng, b=4, d=64, e=8, d_out=32, dtype=np.float32, constant_router=False):
    router = (rng.standard_normal((e, d)) * 0.05).astype(dtype)
    if constant_router:
        router = np.repeat(router[:1], e, axis=0)
    return {
        "x": rng.standard_normal((b, d)).astype(dtype),
        "router": router,
        "experts": (rng.standard_normal((e, d_out, d)) * 0.05).astype(dtype),
    }


# ---------------------------------------------------------------------------
# the controls against the fp64 references, at the reference's bounds
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("bits", [2, 3, 4, 8])
def test_qmm_control_agrees_with_the_contract_reference(bits):
    inputs = qmm_case(np.random.default_rng(3 + bits), bits=bits)
    ref = NATIVE_OPS["quantized_matmul"].reference(inputs)
    out = quantized_matmul(inputs).astype(np.float64)
    assert np.max(np.abs(out - ref)) < 5e-2
    # the control is also a legitimate fp16 implementation: inside its own gate
    assert np.max(np.abs(out - ref)) <= NATIVE_OPS["quantized_matmul"].tolerance(
        _Case("float16"), inputs, ref)


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
def test_qmm_artefact_control_is_the_control_on_a_given_artefact(bits):
    """``quantized_matmul_artefact`` (the bench's CPU baseline) on the
    canonical artefact is bit-identical to the quantizing control, and is
    inside the contract on directly drawn codes (config 1's form)."""
    rng = np.random.default_rng(40 + bits)
    inputs = qmm_case(rng, b=3, d_in=512, d_out=48, bits=bits)
    art = canonical_quantize(inputs["w"], QuantContract(bits=bits, group_size=64))
    assert np.array_equal(quantized_matmul_artefact(inputs["x"], art), quantized_matmul(inputs))
    q = rng.integers(0, 1 << bits, size=(96, 512)).astype(np.int32)
    s = np.abs(rng.standard_normal((96, 8)) * 0.02).astype(np.float16)
    bb = (rng.standard_normal((96, 8)) * 0.01).astype(np.float16)
    drawn = artefact_from_arrays(q, s, bb, bits)
    x = rng.standard_normal((2, 512)).astype(np.float16)
    ref = qmm_reference_artefact(x, drawn)
    out = quantized_matmul_artefact(x, drawn).astype(np.float64)
    assert np.max(np.abs(out - ref)) <= qmm_tolerance_artefact("float16", x, drawn, ref)
    # and the dequantized weights really are s * q + b of the drawn arrays
    want = s.astype(np.float64).repeat(64, 1) * q + bb.astype(np.float64).repeat(64, 1)
    assert np.array_equal(dequantize(drawn, np.float64), want)


@pytest.mark.parametrize("bits", [4, 8])
def test_kv_control_agrees_with_the_reference(bits):
    inputs = kv_case(np.random.default_rng(11 + bits), bits=bits)
    ref = NATIVE_OPS["kv_attention"].reference(inputs)
    out = kv_attention(inputs).astype(np.float64)
    assert np.max(np.abs(out - ref)) < 5e-3


def _torch_moe(x, router, experts, k):
    """The routing contract restated with torch primitives in fp64: softmax
    over every expert, the k most probable by a stable descending sort (ties
    to the lower index), renormalised, then the weighted sum of x @ W_e^T."""
    xt = torch.from_numpy(x.astype(np.float64))
    logits = xt @ torch.from_numpy(router.astype(np.float64)).T
    probs = torch.softmax(logits, dim=-1)
    top = torch.sort(probs, dim=-1, descending=True, stable=True).indices[:, :k]
    w = torch.gather(probs, 1, top)
    w = w / w.sum(dim=-1, keepdim=True)
    ex = torch.from_numpy(experts.astype(np.float64))
    out = torch.zeros(x.shape[0], experts.shape[1], dtype=torch.float64)
    for t in range(x.shape[0]):
        for s in range(k):
            out[t] += w[t, s] * (ex[int(top[t, s])] @ xt[t])
    return out.numpy(), top.numpy()


@pytest.mark.parametrize("k", [1, 2, 4])
def test_moe_reference_is_the_torch_restatement(k):
    inputs = moe_case(np.random.default_rng(5 + k), b=6, d=96, e=12, d_out=40)
    want, _ = _torch_moe(inputs["x"], inputs["router"], inputs["experts"], k)
    ref = moe_reference(inputs, k)
    assert np.max(np.abs(ref - want)) <= 1e-12 * np.max(np.abs(want))


def test_moe_control_agrees_with_the_reference():
    """The reference's bound for its MLX cross-check (tests/test_native_ops.py:75)."""
    inputs = moe_case(np.random.default_rng(2))
    ref = moe_reference(inputs)
    assert np.max(np.abs(moe_dispatch(inputs).astype(np.float64) - ref)) < 1e-4


# ---------------------------------------------------------------------------
# controls pass their own gate; every seam is rejected somewhere
# ---------------------------------------------------------------------------
def _sampled_cases(op_name):
    """A small fixed sample of each operator's battery space
    (NATIVE_OPS[op].meta dims x dtypes x input scales) at the reference test
    suite's draw scales."""
    rng = np.random.default_rng({"quantized_matmul": 1, "kv_attention": 2, "moe_dispatch": 3}[op_name])
    cases = []
    if op_name == "quantized_matmul":
        shapes = [(4, 1024, 64, 4, "float32", 1.0), (1, 448, 16, 3, "float16", 1.0),
                  (4, 128, 64, 8, "float16", 10.0), (2, 1024, 32, 2, "float32", 10.0),
                  (4, 448, 64, 4, "float16", 1.0)]
        for b, d_in, d_out, bits, dtype, scale in shapes:
            cases.append((dtype, qmm_case(rng, b, d_in, d_out, bits, np.dtype(dtype), scale)))
    elif op_name == "kv_attention":
        for b, h, t, dh, bits, dtype in [(1, 2, 512, 128, 4, "float32"), (4, 8, 64, 64, 8, "float16"),
                                         (4, 2, 512, 64, 8, "float32"), (1, 8, 64, 128, 4, "float16")]:
            cases.append((dtype, kv_case(rng, b, h, t, dh, bits, np.dtype(dtype))))
    else:
        for b, d, e, d_out, dtype, const in [(8, 512, 16, 256, "float32", False),
                                             (1, 100, 4, 32, "float16", False),
                                             (8, 64, 16, 32, "float16", False),
                                             (4, 100, 16, 256, "float32", True)]:
            cases.append((dtype, moe_case(rng, b, d, e, d_out, np.dtype(dtype), const)))
    return cases


CONTROLS = {"quantized_matmul": quantized_matmul, "kv_attention": kv_attention,
            "moe_dispatch": moe_dispatch}


@pytest.mark.parametrize("op_name", sorted(CONTROLS))
def test_controls_pass_their_gate_on_every_sampled_case(op_name):
    op = NATIVE_OPS[op_name]
    for dtype, inputs in _sampled_cases(op_name):
        ref = op.reference(inputs)
        tol = op.tolerance(_Case(dtype), inputs, ref)
        out = CONTROLS[op_name](inputs)
        assert out.shape == ref.shape and np.all(np.isfinite(out))
        assert max_abs_error(out, ref) <= tol, (op_name, dtype)


# (operator, seam) pairs the reference's catalogue lists as non-equivalent
# (kernelverify/mutation/catalogue.py:133-179)
SEAMS = [
    ("quantized_matmul", {"scales_rotated": True}),
    ("quantized_matmul", {"nibble_swapped": True}),
    ("quantized_matmul", {"bias_dropped": True}),
    ("quantized_matmul", {"group_size_halved": True}),
    ("quantized_matmul", {"dequant_dtype": "float16"}),
    ("quantized_matmul", {"accum_dtype": "float16"}),
    ("quantized_matmul", {"accum_dtype": "float16-seq"}),
    ("kv_attention", {"scores_dtype": "float16"}),
    ("kv_attention", {"accum_dtype": "float16"}),
    ("kv_attention", {"accum_dtype": "float16-seq"}),
    ("kv_attention", {"k_scales_rotated": True}),
    ("kv_attention", {"v_bias_dropped": True}),
    ("kv_attention", {"new_entry_skipped": True}),
    ("kv_attention", {"dhead_scale_dropped": True}),
    ("moe_dispatch", {"renormalize": False}),
    ("moe_dispatch", {"expert_offset": 1}),
    ("moe_dispatch", {"gate_dtype": "float16"}),
    ("moe_dispatch", {"k_offset": -1}),
]


@pytest.fixture(scope="module")
def judged_cases():
    """Each sampled case with its fp64 reference and tolerance, built once."""
    out = {}
    for op_name in CONTROLS:
        op = NATIVE_OPS[op_name]
        rows = []
        for dtype, inputs in _sampled_cases(op_name):
            ref = op.reference(inputs)
            rows.append((inputs, ref, op.tolerance(_Case(dtype), inputs, ref)))
        out[op_name] = rows
    return out


@pytest.mark.parametrize("op_name,seam", SEAMS, ids=[f"{o}-{s}" for o, s in SEAMS])
def test_every_seam_is_rejected_on_some_sampled_case(judged_cases, op_name, seam):
    control = CONTROLS[op_name]
    errs = []
    for inputs, ref, tol in judged_cases[op_name]:
        faulty = control(inputs, **seam)
        moved = not np.array_equal(faulty, control(inputs))
        rejected = (faulty.shape != ref.shape or not np.all(np.isfinite(faulty))
                    or max_abs_error(faulty, ref) > tol)
        errs.append((moved, rejected))
        if rejected:
            break
    assert any(r for _, r in errs), f"{op_name} {seam} passes every sampled case"
    assert any(m for m, _ in errs)


def test_equivalent_seams_stay_equivalent():
    """Softmax over the chosen logits is the renormalised full softmax; ties
    to the higher index differ only where logits tie exactly."""
    inputs = moe_case(np.random.default_rng(7))
    base = moe_dispatch(inputs).astype(np.float64)
    np.testing.assert_allclose(moe_dispatch(inputs, softmax_topk_order=True), base, atol=1e-5)
    np.testing.assert_allclose(moe_dispatch(inputs, tie_high=True), base, atol=0)
    tied = moe_case(np.random.default_rng(7), constant_router=True)
    assert not np.array_equal(moe_dispatch(tied, tie_high=True), moe_dispatch(tied))


# ---------------------------------------------------------------------------
# moe_tolerance: members pass, planted mistakes fail
# ---------------------------------------------------------------------------
def _moe_mistake(inputs, kind, k=2):
    """The routing contract with one planted mistake, in fp64."""
    x = inputs["x"].astype(np.float64)
    experts = inputs["experts"].astype(np.float64)
    top, w = route_probs(x @ inputs["router"].astype(np.float64).T, k, np.float64)
    out = np.zeros((x.shape[0], experts.shape[1]))
    for t in range(x.shape[0]):
        for s in range(k):
            e = int(top[t, s])
            if kind == "slot-dropped" and s == k - 1:
                continue
            if kind == "wrong-expert":
                e = (e + 1) % experts.shape[0]
            we = experts[e].T if kind == "transposed" else experts[e]
            g = 1.0 if kind == "gates-not-applied" else w[t, s]
            out[t] += g * (we @ x[t])
    if kind == "fp16-combine":
        out = np.zeros((x.shape[0], experts.shape[1]), dtype=np.float16)
        for t in range(x.shape[0]):
            for s in range(k):
                out[t] += (w[t, s] * (experts[int(top[t, s])] @ x[t])).astype(np.float16)
    return out


@pytest.mark.parametrize("dtype", ["float16", "float32"])
def test_moe_tolerance_admits_its_members_and_rejects_planted_mistakes(dtype):
    inputs = moe_case(np.random.default_rng(21), b=8, d=128, e=16, d_out=128, dtype=np.dtype(dtype))
    ref = moe_reference(inputs)
    tol = moe_tolerance(_Case(dtype), inputs, ref)
    for fn in MOE_MEMBERS.values():
        assert max_abs_error(fn(inputs), ref) <= tol
    kinds = ["slot-dropped", "gates-not-applied", "wrong-expert", "transposed"]
    if dtype == "float32":
        kinds.append("fp16-combine")  # inside fp16 rounding at an fp16 output, by design
    for kind in kinds:
        assert max_abs_error(_moe_mistake(inputs, kind), ref) > tol, (kind, dtype)


# ---------------------------------------------------------------------------
# moe_linear_reference / moe_linear_tolerance (routing given, any k)
# ---------------------------------------------------------------------------
D = 64


def _perm_expert(shift: int, scale: float):
    """Rows j = scale * e_{(j + shift) % D}: code 1, scale, bias 0."""
    q = np.zeros((D, D), dtype=np.int32)
    q[np.arange(D), (np.arange(D) + shift) % D] = 1
    return artefact_from_arrays(q, np.full((D, 1), scale, np.float16),
                                np.zeros((D, 1), np.float16), 4)


SHIFTS, AMPS = (3, 10, 17, 29, 41), (0.5, 1.25, 2.0, 0.75, 1.5)


def test_moe_linear_reference_closed_form_on_permutation_experts():
    arts = [_perm_expert(s, a) for s, a in zip(SHIFTS, AMPS)]
    x = np.random.default_rng(9).standard_normal((4, D)).astype(np.float16)
    idx = np.array([[0, 3, 4], [2, 2, 1], [4, 0, 1], [1, 3, 2]])
    gate = np.array([[0.5, 0.25, 0.25], [0.375, 0.125, 0.5], [0.75, 0.125, 0.125],
                     [0.0625, 0.5, 0.4375]], dtype=np.float32)
    x64 = x.astype(np.float64)
    want = np.zeros((4, D))
    for t in range(4):
        for s in range(3):
            e = idx[t, s]
            want[t] += gate[t, s] * AMPS[e] * np.roll(x64[t], -SHIFTS[e])
    got = moe_linear_reference(x, idx, gate, arts)
    assert np.max(np.abs(got - want)) <= 1e-12 * np.max(np.abs(want))
    transposed = [artefact_from_arrays(a.q.T.copy(), a.scales, a.biases, 4) for a in arts]
    for wrong in (moe_linear_reference(x, idx, gate, transposed),
                  moe_linear_reference(x, (idx + 1) % 5, gate, arts)):
        assert np.max(np.abs(wrong - want)) > 1e-2 * np.max(np.abs(want))


def _drawn_linear(seed, n=6, d=128, e=8, d_out=96, k=4, bits=4, dtype=np.float16):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, d)).astype(dtype)
    arts = [canonical_quantize((rng.standard_normal((d_out, d)) * 0.05).astype(np.float16),
                               QuantContract(bits=bits, group_size=64)) for _ in range(e)]
    logits = rng.standard_normal((n, e))
    top, w = route_probs(logits, k, np.float64)
    return x, logits, top, w, arts


def test_moe_linear_reference_is_moe_reference_on_the_same_routing():
    x, logits, top, w, arts = _drawn_linear(4)
    dense = np.stack([dequantize(a, np.float64) for a in arts])
    want = moe_reference({"x": x, "logits": logits, "experts": dense}, k=4)
    got = moe_linear_reference(x, top, w, arts)
    assert np.max(np.abs(got - want)) <= 1e-12 * np.max(np.abs(want))


def _linear_mistake(x, idx, gate, arts, kind):
    out = np.zeros((x.shape[0], arts[0].q.shape[0]))
    k = idx.shape[1]
    for t in range(x.shape[0]):
        for s in range(k):
            if kind == "slot-dropped" and s == k - 1:
                continue
            e = int(idx[t, s])
            if kind == "wrong-expert":
                e = (e + 1) % len(arts)
            wd = dequantize(arts[e], np.float64)
            g = 1.0 if kind == "gates-not-applied" else float(gate[t, s])
            if kind == "bias-dropped":
                wd = wd - dequantize(arts[e], np.float64) + (
                    arts[e].scales.astype(np.float64).repeat(64, 1) * arts[e].q)
            out[t] += g * (wd @ x[t].astype(np.float64))
    if kind == "fp16-combine":
        out = np.zeros((x.shape[0], arts[0].q.shape[0]), dtype=np.float16)
        for t in range(x.shape[0]):
            for s in range(k):
                y = float(gate[t, s]) * (dequantize(arts[int(idx[t, s])], np.float64)
                                         @ x[t].astype(np.float64))
                out[t] += y.astype(np.float16)
    return out


@pytest.mark.parametrize("dtype", ["float16", "float32"])
def test_moe_linear_tolerance_admits_fp32_and_rejects_planted_mistakes(dtype):
    x, _, top, w, arts = _drawn_linear(6, dtype=np.dtype(dtype))
    gate = w.astype(np.float32)
    ref = moe_linear_reference(x, top, gate, arts)
    tol = moe_linear_tolerance(dtype, x, top, gate, arts, ref)
    # a legitimate fp32 evaluation in another order (BLAS over the stacked slots)
    y = np.stack([[dequantize(arts[int(top[t, s])], np.float32) @ x[t].astype(np.float32)
                   for s in range(top.shape[1])] for t in range(x.shape[0])])
    blas = np.einsum("ts,tsd->td", gate, y).astype(np.dtype(dtype))
    assert max_abs_error(blas, ref) <= tol
    kinds = ["slot-dropped", "gates-not-applied", "wrong-expert", "bias-dropped"]
    if dtype == "float32":
        kinds.append("fp16-combine")
    for kind in kinds:
        assert max_abs_error(_linear_mistake(x, top, gate, arts, kind), ref) > tol, (kind, dtype)
