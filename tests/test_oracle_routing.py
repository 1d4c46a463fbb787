"""Pins of the MoE routing and permutation oracles (oracle.native_ops.route_probs,
oracle.native_kernels._topk_by_prob, oracle.extensions.route_topk and
permute_by_expert) against what the definitions fix independently:

- top-k by probability with ties to the lower index: brute force (Python's
  sorted on (-p, index)) and torch's stable sort, on rows with exact ties;
  ties to the higher index likewise on (-p, -index);
- the softmax: a known answer (logits 0, ln 2, ln 3 give 1/6, 2/6, 3/6),
  shift invariance, and renormalised gates that sum to one in the top-k's
  probability ratios;
- the permutation: brute force (sorted on (expert, flat index)) and the
  counting-sort offsets;
- moe_reference (routing then combine): a closed form on constant router
  rows and permutation-matrix experts.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle.extensions import permute_by_expert, route_topk
from oracle.native_kernels import _topk_by_prob
from oracle.native_ops import route_probs


def _tied_probs(rng, n, e):
    """Probability rows drawn from a few levels, so exact ties are common."""
    levels = rng.integers(0, 4, size=(n, e)).astype(np.float64)
    p = np.exp(levels)
    return p / p.sum(1, keepdims=True)


@pytest.mark.parametrize("k", [1, 2, 8, 16])
def test_topk_is_the_brute_force_and_the_stable_sort(k):
    rng = np.random.default_rng(k)
    probs = _tied_probs(rng, 40, 16)
    low = _topk_by_prob(probs, k, tie_high=False)
    high = _topk_by_prob(probs, k, tie_high=True)
    for r, row in enumerate(probs):
        want_low = sorted(range(16), key=lambda i: (-row[i], i))[:k]
        want_high = sorted(range(16), key=lambda i: (-row[i], -i))[:k]
        assert list(low[r]) == want_low and list(high[r]) == want_high
    by_torch = torch.sort(-torch.from_numpy(probs), dim=1, stable=True).indices[:, :k].numpy()
    assert np.array_equal(low, by_torch)


def test_constant_rows_route_to_the_first_k_either_way():
    probs = np.full((3, 8), 1 / 8)
    assert np.array_equal(_topk_by_prob(probs, 3), np.tile([0, 1, 2], (3, 1)))
    assert np.array_equal(_topk_by_prob(probs, 3, tie_high=True), np.tile([7, 6, 5], (3, 1)))


def test_softmax_known_answer_and_shift_invariance():
    logits = np.array([[0.0, math.log(2.0), math.log(3.0)]])
    top, gate = route_probs(logits, 3, np.float64)
    assert list(top[0]) == [2, 1, 0]
    assert np.allclose(gate[0], [3 / 6, 2 / 6, 1 / 6], rtol=1e-15, atol=0)
    rng = np.random.default_rng(2)
    x = rng.standard_normal((20, 32))
    t1, g1 = route_probs(x, 4, np.float64)
    t2, g2 = route_probs(x + 7.25, 4, np.float64)
    assert np.array_equal(t1, t2) and np.allclose(g1, g2, rtol=1e-13, atol=0)


def test_route_topk_gates_are_renormalised_probability_ratios():
    rng = np.random.default_rng(4)
    logits = rng.standard_normal((25, 64)).astype(np.float32)
    idx, gate = route_topk(logits, 8)
    assert idx.shape == gate.shape == (25, 8) and gate.dtype == np.float32
    l64 = logits.astype(np.float64)
    for r in range(25):
        assert list(idx[r]) == sorted(range(64), key=lambda i: (-l64[r, i], i))[:8]
        chosen = l64[r, idx[r]]
        want = np.exp(chosen - chosen.max())
        want /= want.sum()  # softmax restricted to the chosen: the renormalised gates
        assert np.allclose(gate[r], want, rtol=2e-6, atol=0)
    assert np.allclose(gate.sum(1), 1.0, rtol=0, atol=1e-6)


@pytest.mark.parametrize("n,k,e", [(1, 2, 8), (7, 3, 5), (33, 8, 16), (12, 4, 64)])
def test_permutation_is_the_brute_force_stable_sort(n, k, e):
    idx = np.random.default_rng(n * k).integers(0, e, size=(n, k))
    offsets, perm = permute_by_expert(idx, e)
    flat = idx.reshape(-1)
    assert list(perm) == sorted(range(n * k), key=lambda i: (flat[i], i))
    counts = [int((flat == x).sum()) for x in range(e)]
    assert list(offsets) == [sum(counts[:x]) for x in range(e + 1)]


def test_moe_reference_closed_form_on_permutation_experts():
    """Constant router rows make every logit equal: routing is experts 0 and
    1 (ties low) at gates 1/2 each. Experts a_e P_e (P_e a cyclic shift by
    s_e) then give out[i] = (a_0 x[i + s_0] + a_1 x[i + s_1]) / 2."""
    from oracle.native_ops import moe_reference

    d, e = 64, 4
    shifts, amps = (3, 10, 17, 29), (0.5, 1.25, 2.0, 0.75)
    experts = np.zeros((e, d, d))
    for j in range(e):
        experts[j, np.arange(d), (np.arange(d) + shifts[j]) % d] = amps[j]
    x = np.random.default_rng(9).standard_normal((3, d)).astype(np.float16)
    router = np.full((e, d), 0.03125, dtype=np.float16)
    out = moe_reference({"x": x, "router": router, "experts": experts})
    x64 = x.astype(np.float64)
    want = 0.5 * (amps[0] * np.roll(x64, -shifts[0], axis=1)
                  + amps[1] * np.roll(x64, -shifts[1], axis=1))
    assert np.max(np.abs(out - want)) <= 1e-12 * np.max(np.abs(want))
    transposed = experts.transpose(0, 2, 1).copy()
    wrong = moe_reference({"x": x, "router": router, "experts": transposed})
    assert np.max(np.abs(wrong - want)) > 1e-2 * np.max(np.abs(want))
