"""Pins of the SwiGLU expert oracle (oracle.extensions.swiglu_reference and
swiglu_tolerance), which the reference has no counterpart for.

- Closed form: experts whose dequantized gate, up and down matrices are
  scaled permutation matrices (a P, b Q, c R, distinct per expert). The MLP
  then reduces elementwise to out[i] = sum_s g_s c silu(a x[p(r(i))]) b
  x[q(r(i))], with silu(z) = z / (1 + e^-z) per element. A transposed
  operand, swapped gate/up roles or a wrong expert index each fails it.
- Invariants on drawn weights: slot order, linearity in the gates, one
  expert taken twice, zero gates.
- The tolerance: the three fp32 members pass, and planted mistakes in the
  oracle (sigmoid for silu, no up projection, swapped roles, gates dropped,
  the next expert) each exceed it.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle.extensions import artefact_from_arrays, swiglu_reference, swiglu_tolerance
from oracle.quant_contract import QuantContract, canonical_quantize, dequantize

D = 64  # one group per row: d_model = d_ffn = 64


def _perm_artefact(perm: np.ndarray, scale: float, bits: int = 4):
    """Rows j = scale * e_{perm[j]}: code 1 at column perm[j], scale, bias 0."""
    q = np.zeros((D, D), dtype=np.int32)
    q[np.arange(D), perm] = 1
    return artefact_from_arrays(q, np.full((D, 1), scale, np.float16),
                                np.zeros((D, 1), np.float16), bits)


def _shift(k):
    return (np.arange(D) + k) % D


def _closed_form_experts():
    """Expert e: gate a_e P, up b_e Q, down c_e R with P, Q, R cyclic shifts
    (none an involution, so a transpose shows)."""
    scales = [(0.5, 1.25, 0.75), (1.5, 0.25, 2.0), (0.75, 2.5, 0.5)]
    gate_arts, up_arts, down_arts = [], [], []
    for e, (a, b, c) in enumerate(scales):
        gate_arts.append(_perm_artefact(_shift(1 + e), a))
        up_arts.append(_perm_artefact(_shift(5 + 2 * e), b))
        down_arts.append(_perm_artefact(_shift(11 + 3 * e), c))
    return scales, gate_arts, up_arts, down_arts


def _closed_form(x, idx, gate, scales):
    out = np.zeros((x.shape[0], D))
    for t in range(x.shape[0]):
        for s in range(idx.shape[1]):
            e = int(idx[t, s])
            a, b, c = scales[e]
            for i in range(D):
                j = (i + 11 + 3 * e) % D                   # down row i reads h[j]
                z = a * float(x[t, (j + 1 + e) % D])       # gate row j reads x[j + 1 + e]
                u = b * float(x[t, (j + 5 + 2 * e) % D])   # up row j reads x[j + 5 + 2e]
                out[t, i] += float(gate[t, s]) * c * (z / (1.0 + math.exp(-z))) * u
    return out


def test_reference_is_the_closed_form_on_permutation_experts():
    scales, g_arts, u_arts, d_arts = _closed_form_experts()
    x = np.random.default_rng(0).standard_normal((3, D)).astype(np.float16)
    idx = np.array([[0, 2], [1, 0], [2, 2]])
    gate = np.array([[0.625, 0.375], [0.5, 0.5], [0.25, 0.75]], dtype=np.float32)
    ref = swiglu_reference(x, idx, gate, g_arts, u_arts, d_arts)
    want = _closed_form(x, idx, gate, scales)
    assert np.max(np.abs(ref - want)) <= 1e-12 * np.max(np.abs(want))


def test_closed_form_separates_the_plausible_mistakes():
    """The closed form is not blind: transposed experts and swapped roles
    move the output far beyond rounding."""
    scales, g_arts, u_arts, d_arts = _closed_form_experts()
    x = np.random.default_rng(1).standard_normal((2, D)).astype(np.float16)
    idx, gate = np.array([[0, 1], [2, 0]]), np.array([[0.5, 0.5], [0.5, 0.5]], np.float32)
    want = _closed_form(x, idx, gate, scales)
    transposed = [artefact_from_arrays(a.q.T.copy(), a.scales, a.biases, 4) for a in g_arts]
    for wrong in (swiglu_reference(x, idx, gate, transposed, u_arts, d_arts),
                  swiglu_reference(x, idx, gate, u_arts, g_arts, d_arts),
                  swiglu_reference(x, (idx + 1) % 3, gate, g_arts, u_arts, d_arts)):
        assert np.max(np.abs(wrong - want)) > 1e-2 * np.max(np.abs(want))


def _drawn(n=4, e=5, d_model=128, d_ffn=64, bits=4, seed=3):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, d_model)).astype(np.float16)
    arts = {}
    for name, shape in (("gate", (d_ffn, d_model)), ("up", (d_ffn, d_model)),
                        ("down", (d_model, d_ffn))):
        arts[name] = [canonical_quantize((rng.standard_normal(shape) * 0.05).astype(np.float16),
                                         QuantContract(bits=bits, group_size=64))
                      for _ in range(e)]
    idx = np.stack([rng.choice(e, size=2, replace=False) for _ in range(n)])
    g = rng.random((n, 2)).astype(np.float32) + 0.1
    return x, idx, (g / g.sum(1, keepdims=True)).astype(np.float32), arts


def test_invariants_slot_order_linearity_repeats_and_zero():
    x, idx, gate, arts = _drawn()
    A = (arts["gate"], arts["up"], arts["down"])
    ref = swiglu_reference(x, idx, gate, *A)
    scale = np.max(np.abs(ref))
    swapped = swiglu_reference(x, idx[:, ::-1].copy(), gate[:, ::-1].copy(), *A)
    assert np.max(np.abs(swapped - ref)) <= 1e-12 * scale
    doubled = swiglu_reference(x, idx, (gate * 2).astype(np.float32), *A)
    assert np.max(np.abs(doubled - 2 * ref)) <= 1e-12 * scale
    twice = np.stack([idx[:, 0], idx[:, 0]], axis=1)
    dyadic = (np.round(gate * 64) / 64).astype(np.float32)  # the fp32 sum is exact
    split = swiglu_reference(x, twice, dyadic, *A)
    whole = swiglu_reference(x, twice, np.stack([dyadic.sum(1), np.zeros(len(x))], 1)
                             .astype(np.float32), *A)
    assert np.max(np.abs(split - whole)) <= 1e-12 * np.max(np.abs(whole))
    assert not np.any(swiglu_reference(x, idx, np.zeros_like(gate), *A))


def _mistake(x, idx, gate, arts, kind):
    """A planted mistake in the oracle's own formula (fp64, CPU)."""
    out = np.zeros((x.shape[0], arts["down"][0].q.shape[0]))
    for t in range(x.shape[0]):
        for s in range(idx.shape[1]):
            e = int(idx[t, s])
            if kind == "next-expert":
                e = (e + 1) % len(arts["gate"])
            wg, wu, wd = (dequantize(arts[m][e], np.float64) for m in ("gate", "up", "down"))
            g, u = wg @ x[t].astype(np.float64), wu @ x[t].astype(np.float64)
            if kind == "sigmoid":
                h = u / (1.0 + np.exp(-g))
            elif kind == "no-up":
                h = g / (1.0 + np.exp(-g))
            elif kind == "swapped-roles":
                h = u / (1.0 + np.exp(-u)) * g
            else:
                h = g / (1.0 + np.exp(-g)) * u
            w = 1.0 if kind == "gates-dropped" else float(gate[t, s])
            out[t] += w * (wd @ h)
    return out


@pytest.mark.parametrize("dtype", ["float16", "float32"])
def test_tolerance_admits_fp32_and_rejects_planted_mistakes(dtype):
    from oracle.extensions import SWIGLU_MEMBERS, _swiglu_member

    x, idx, gate, arts = _drawn(seed=5)
    A = (arts["gate"], arts["up"], arts["down"])
    ref = swiglu_reference(x, idx, gate, *A)
    tol = swiglu_tolerance(dtype, x, idx, gate, *A, ref)
    for kw in SWIGLU_MEMBERS.values():
        member = _swiglu_member(x.astype(dtype), idx, gate, *A, **kw).astype(np.float64)
        assert np.max(np.abs(member - ref)) <= tol
    for kind in ("sigmoid", "no-up", "swapped-roles", "gates-dropped", "next-expert"):
        err = np.max(np.abs(_mistake(x, idx, gate, arts, kind) - ref))
        assert err > tol, (kind, err, tol)
