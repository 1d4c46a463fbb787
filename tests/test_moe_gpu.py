"""MoE routing, permutation and expert dispatch on the GPU against the CPU oracle.

Mirrors the reference's kernel tests (tests/test_pack_moe_dispatch.py:64-124)
and gate (bench/pack_moe_dispatch.py:122-233: VERIFY_SHAPES x {normal,
constant_rows}), at the reference's k = 2 and at BASELINE config 5's
top-8 of 128 with the SwiGLU expert MLP.

Bit-exact claims: top-k indices on every row (each seed is checked to hold
no row whose k-th and (k+1)-th probabilities sit within 64 fp32 ulps, where
an exp rounded apart from numpy's could reorder them:
``oracle.extensions.near_tie_rows``), constant-row ties ([0 .. k-1]
exactly), and the token permutation (offsets and order).
Gates: within 1e-5 of the contract (tests/test_pack_moe_dispatch.py:79-87).
Outputs: the oracle's fp64 reference and ensemble-floor tolerance.
"""

import numpy as np
import pytest

from kernelverify_amd import lib
from kernelverify_amd.pack import moe_dispatch as moe
from kernelverify_amd.pack.codes import pack_codes
from oracle.extensions import (
    moe_linear_reference,
    moe_linear_tolerance,
    near_tie_rows,
    permute_by_expert,
    route_topk,
    swiglu_reference,
    swiglu_tolerance,
)
from oracle.inputs import moe_case
from oracle.native_ops import _moe_route
from oracle.quant_contract import QuantContract, canonical_quantize, dequantize
from oracle.verify import judge, moe_inputs, verify_output

pytestmark = pytest.mark.gpu

VERIFY_SHAPES = [(1, 512, 16, 256), (8, 512, 16, 256), (4, 256, 8, 128)]


def quantize_experts(experts: np.ndarray, bits: int):
    """Oracle artefacts per expert + the kernel layout (product packer)."""
    arts = [canonical_quantize(w, QuantContract(bits=bits, group_size=64)) for w in experts]
    packed = np.stack([pack_codes(a.q, bits) for a in arts])
    return packed, np.stack([a.scales for a in arts]), np.stack([a.biases for a in arts]), arts


# ---------------------------------------------------------------------------
# routing
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("n,e,k", [(32, 128, 8), (8, 16, 2), (5, 64, 4), (3, 1024, 32)])
def test_route_logits_matches_the_contract(n, e, k):
    """Every row judged: indices exact (array_equal over all rows, as
    tests/test_pack_moe_dispatch.py:62-66), gates within 1e-5."""
    logits = np.random.default_rng(n * e + k).standard_normal((n, e)).astype(np.float32)
    # no row of this seed has its k-th and (k+1)-th probabilities within 64
    # fp32 ulps, so an exp rounded apart from numpy's cannot reorder them
    assert not near_tie_rows(logits, k, ulps=64).any()
    idx, gate = moe.route(logits, k)
    want_idx, want_gate = route_topk(logits, k)
    assert np.array_equal(idx.astype(np.int64), want_idx)
    assert np.max(np.abs(gate - want_gate)) < 1e-5
    assert np.allclose(gate.sum(axis=-1), 1.0, atol=1e-6)


@pytest.mark.parametrize("n", [1, 8, 32])
def test_config5_routing_exact_over_seeds(n):
    """BASELINE config 5 (128 experts, top-8, logits ~ N(0, 1)) over 16 seeds
    per batch size: every index of every row equals the contract's."""
    for seed in range(16):
        logits = np.random.default_rng(1000 * n + seed).standard_normal((n, 128)).astype(np.float32)
        assert not near_tie_rows(logits, 8, ulps=64).any(), seed
        idx, gate = moe.route(logits, 8)
        want_idx, want_gate = route_topk(logits, 8)
        assert np.array_equal(idx.astype(np.int64), want_idx), seed
        assert np.max(np.abs(gate - want_gate)) < 1e-5, seed


def test_ties_go_to_the_lower_index():
    """Constant rows tie every logit: the chosen set is [0 .. k-1] exactly."""
    logits = np.full((4, 128), 0.25, dtype=np.float32)
    idx, gate = moe.route(logits, 8)
    assert np.array_equal(idx, np.tile(np.arange(8, dtype=np.uint32), (4, 1)))
    assert np.allclose(gate, 1.0 / 8, atol=1e-7)


def test_reference_routing_from_x_k2():
    """The reference kernel's own form: logits = x @ router^T, k = 2, every
    row exact (tests/test_pack_moe_dispatch.py:62-66)."""
    x, router, _ = moe_case(8, 512, 16, 256, seed=2)
    idx, gate = moe.route(x=x, router=router, k=2)
    _, want_idx, want_gate = _moe_route({"x": x, "router": router}, np.float32, k=2)
    logits = x.astype(np.float32) @ router.astype(np.float32).T
    # the GPU sums x . router in another order than BLAS; no row of this seed
    # is within 256 ulps of a tie, so that cannot reorder a choice
    assert not near_tie_rows(logits, 2, ulps=256).any()
    assert np.array_equal(idx.astype(np.int64), want_idx)
    assert np.max(np.abs(gate - want_gate)) < 1e-5


def test_constant_rows_from_x_route_low():
    x, router, _ = moe_case(4, 256, 8, 128, seed=2, mode="constant_rows")
    idx, _ = moe.route(x=x, router=router, k=2)
    assert np.array_equal(idx.astype(int), np.tile([0, 1], (4, 1)))


# ---------------------------------------------------------------------------
# permutation
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("n,k,e,mode", [(32, 8, 128, "random"), (1, 8, 128, "random"),
                                        (64, 8, 16, "skewed"), (200, 8, 128, "random"),
                                        (7, 3, 5, "random")])
def test_permute_is_the_stable_counting_sort(n, k, e, mode):
    rng = np.random.default_rng(n + k + e)
    if mode == "skewed":
        idx = np.minimum(rng.geometric(0.5, (n, k)) - 1, e - 1).astype(np.uint32)
    else:
        idx = np.stack([rng.choice(e, k, replace=False) for _ in range(n)]).astype(np.uint32)
    offsets, perm = moe.permute_host(idx, e)
    want_off, want_perm = permute_by_expert(idx, e)
    assert np.array_equal(offsets, want_off)
    assert np.array_equal(perm, want_perm)


# ---------------------------------------------------------------------------
# single-linear dispatch (the reference's contract)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("shape", VERIFY_SHAPES)
@pytest.mark.parametrize("mode", ["normal", "constant_rows"])
def test_reference_gate_k2(shape, mode):
    """The reference gate's cases: route from x, dispatch 4-bit experts,
    judged by NATIVE_OPS['moe_dispatch'] over the dequantized experts."""
    n, d, e, d_ffn = shape
    x, router, experts = moe_case(n, d, e, d_ffn, seed=n * 31 + len(mode), mode=mode)
    packed, scales, biases, arts = quantize_experts(experts, 4)
    idx, gate = moe.route(x=x, router=router, k=2)
    out = moe.dispatch_host(x, idx, gate, packed, scales, biases, bits=4)
    v = verify_output("moe_dispatch", moe_inputs(x, router, arts), out)
    assert v.ok, v


@pytest.mark.parametrize("bits", [4, 2])
def test_dispatch_slot_naming_no_expert_adds_nothing(bits):
    """A slot whose index is n_experts or more contributes zero (as in
    kvp_moe_swiglu): the output equals the reference with that slot's gate
    zeroed, and a token with no valid slot is zero."""
    rng = np.random.default_rng(90 + bits)
    n, d, e, k, d_out = 4, 256, 8, 3, 96
    x = rng.standard_normal((n, d)).astype(np.float16)
    experts = (rng.standard_normal((e, d_out, d)) * 0.02).astype(np.float16)
    packed, scales, biases, arts = quantize_experts(experts, bits)
    idx, gate = route_topk(rng.standard_normal((n, e)).astype(np.float32), k)
    idx = idx.astype(np.uint32)
    bad = idx.copy()
    bad[1, 2] = e
    bad[3, :] = np.uint32(0xFFFFFFFF)
    out = moe.dispatch_host(x, bad, gate, packed, scales, biases, bits=bits, out_dtype="float32")
    assert not np.any(out[3])
    fixed, g0 = idx.copy(), gate.copy()
    fixed[1, 2], g0[1, 2] = 0, 0.0
    fixed[3, :], g0[3, :] = 0, 0.0
    ref = moe_linear_reference(x, fixed, g0, arts)
    v = judge(out, ref, moe_linear_tolerance("float32", x, fixed, g0, arts, ref))
    assert v.ok, v


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
@pytest.mark.parametrize("d_out", [100, 256])
def test_dispatch_top8_every_width(bits, d_out):
    rng = np.random.default_rng(bits + d_out)
    n, d, e, k = 6, 512, 32, 8
    x = rng.standard_normal((n, d)).astype(np.float16)
    experts = (rng.standard_normal((e, d_out, d)) * 0.02).astype(np.float16)
    packed, scales, biases, arts = quantize_experts(experts, bits)
    logits = rng.standard_normal((n, e)).astype(np.float32)
    idx, gate = route_topk(logits, k)
    for out_dtype in ("float16", "float32"):
        out = moe.dispatch_host(x, idx, gate, packed, scales, biases, bits=bits,
                                out_dtype=out_dtype)
        ref = moe_linear_reference(x, idx, gate, arts)
        v = judge(out, ref, moe_linear_tolerance(out_dtype, x, idx, gate, arts, ref))
        assert v.ok, (bits, d_out, out_dtype, v)


# ---------------------------------------------------------------------------
# SwiGLU experts
# ---------------------------------------------------------------------------
def swiglu_case(n, e, d_model, d_ffn, bits, seed, logits=None):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, d_model)).astype(np.float16)
    mats = {}
    for name, shape in (("gate", (e, d_ffn, d_model)), ("up", (e, d_ffn, d_model)),
                        ("down", (e, d_model, d_ffn))):
        w = (rng.standard_normal(shape) * 0.02).astype(np.float16)
        mats[name] = quantize_experts(w, bits)
    if logits is None:
        logits = rng.standard_normal((n, e)).astype(np.float32)
    return x, mats, logits


def judge_swiglu(x, mats, idx, gate, out, tokens, dtype="float16"):
    sl = slice(None) if tokens is None else tokens
    xs, ids, gs = x[sl], idx[sl], gate[sl]
    arts = [mats[m][3] for m in ("gate", "up", "down")]
    ref = swiglu_reference(xs, ids, gs, *arts)
    tol = swiglu_tolerance(dtype, xs, ids, gs, *arts, ref)
    return judge(out[sl], ref, tol)


def run_swiglu(x, mats, idx, gate, bits, out_dtype="float16"):
    return moe.swiglu_host(x, idx, gate, mats["gate"][:3], mats["up"][:3], mats["down"][:3],
                           bits=bits, out_dtype=out_dtype)


def test_config5_one_token():
    """128 experts, top-8 from fp32 N(0, 1) logits, d 2048, ffn 768, 4-bit."""
    x, mats, logits = swiglu_case(1, 128, 2048, 768, 4, seed=5)
    idx, gate = moe.route(logits, 8)
    out = run_swiglu(x, mats, idx, gate, 4)
    v = judge_swiglu(x, mats, idx.astype(np.int64), gate, out, None)
    print("cfg5 n1", v)
    assert v.ok, v


@pytest.mark.parametrize("n", [8, 32])
def test_config5_many_tokens(n):
    """n = 8 and 32: every token's output depends only on its own routing,
    so three tokens are judged in full (the oracle dequantizes per expert)."""
    x, mats, logits = swiglu_case(n, 128, 2048, 768, 4, seed=50 + n)
    idx, gate = moe.route(logits, 8)
    out = run_swiglu(x, mats, idx, gate, 4)
    assert np.isfinite(out.astype(np.float32)).all()
    v = judge_swiglu(x, mats, idx.astype(np.int64), gate, out, [0, n // 2, n - 1])
    print("cfg5 n", n, v)
    assert v.ok, v


@pytest.mark.parametrize("n,e,d_model,d_ffn,constant", [
    (10, 16, 1024, 768, True),    # gate/up G = 16 (one scale batch), 3 passes; down tile kept over 5
    (32, 64, 2048, 256, False),   # gate/up G = 32 (two batches a pass), experts past four pairs
])
def test_scale_tiles_over_several_passes(n, e, d_model, d_ffn, constant):
    """The per-wave scale tiles (one tile per wave: gate/up with whole
    four-step batches, the fp32-input down projection kept over its passes)
    on experts that take several passes: every pass re-requests the first
    batch of scales (gate/up) or reuses the tile written in the first (down).
    Three tokens judged in full against the oracle."""
    logits = np.zeros((n, e), dtype=np.float32) if constant else None
    x, mats, logits = swiglu_case(n, e, d_model, d_ffn, 4, seed=120 + n, logits=logits)
    idx, gate = moe.route(logits, 8)
    per_expert = np.bincount(idx.ravel().astype(np.int64), minlength=e)
    assert per_expert.max() > 4  # some expert takes a second gate/up pass
    out = run_swiglu(x, mats, idx, gate, 4, "float32")
    v = judge_swiglu(x, mats, idx.astype(np.int64), gate, out, [0, n // 2, n - 1], "float32")
    assert v.ok, v


def test_experts_shared_by_many_tokens():
    """Constant logits send all ten tokens to experts 0..7: each expert runs
    three token groups (four, four, two) over one weight stream."""
    logits = np.zeros((10, 16), dtype=np.float32)
    x, mats, _ = swiglu_case(10, 16, 512, 256, 4, seed=7, logits=logits)
    idx, gate = moe.route(logits, 8)
    assert np.array_equal(idx, np.tile(np.arange(8, dtype=np.uint32), (10, 1)))
    out = run_swiglu(x, mats, idx, gate, 4, "float32")
    v = judge_swiglu(x, mats, idx.astype(np.int64), gate, out, None, "float32")
    assert v.ok, v


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
def test_swiglu_every_width(bits):
    x, mats, logits = swiglu_case(3, 16, 512, 256, bits, seed=bits)
    idx, gate = route_topk(logits, 4)
    out = run_swiglu(x, mats, idx, gate, bits)
    v = judge_swiglu(x, mats, idx, gate, out, None)
    assert v.ok, (bits, v)


@pytest.mark.parametrize("bits", [4, 8])
def test_swiglu_hidden_state_beyond_fp16_range(bits):
    """x ~ N(0, 600^2): the fp32 hidden state exceeds 65504, so the down
    projection's hi/lo fp16 operands must be range-shifted by an exact power
    of two (the matrix-core path) and still match the fp64 reference."""
    x, mats, logits = swiglu_case(4, 16, 512, 256, bits, seed=40 + bits)
    x = (x.astype(np.float32) * 600.0).astype(np.float16)
    idx, gate = route_topk(logits, 4)
    g_art, u_art = mats["gate"][3][idx[0, 0]], mats["up"][3][idx[0, 0]]
    x0 = x[0].astype(np.float64)
    g, u = x0 @ dequantize(g_art, np.float64).T, x0 @ dequantize(u_art, np.float64).T
    assert np.abs(g / (1 + np.exp(-np.clip(g, -80, 80))) * u).max() > 65504  # as the name says
    out = run_swiglu(x, mats, idx, gate, bits, "float32")
    v = judge_swiglu(x, mats, idx, gate, out, None, "float32")
    assert v.ok, (bits, v)


def test_swiglu_group_count_off_the_matrix_core_tiling():
    """d_ffn = 320 (five groups, not a multiple of four): the down projection
    takes the VALU kernel; the result is the same operator."""
    x, mats, logits = swiglu_case(3, 16, 512, 320, 4, seed=9)
    idx, gate = route_topk(logits, 4)
    out = run_swiglu(x, mats, idx, gate, 4)
    v = judge_swiglu(x, mats, idx, gate, out, None)
    assert v.ok, v


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
def test_one_token_at_every_width(bits):
    """n = 1 (the decode step of one sequence) at every width, fp32 out."""
    x, mats, logits = swiglu_case(1, 16, 512, 256, bits, seed=60 + bits)
    idx, gate = route_topk(logits, 4)
    out = run_swiglu(x, mats, idx, gate, bits, "float32")
    v = judge_swiglu(x, mats, idx, gate, out, None, "float32")
    assert v.ok, (bits, v)


@pytest.mark.parametrize("bits", [4, 8])
def test_in_block_routing_equals_the_permute_launch(bits):
    """A few pairs on the matrix cores: the gate/up launch builds the
    permutation in-block. Its output is bit-identical to the separate
    permute launch (tuning key moe_permute = 1), also when one pair names no expert
    (that pair adds nothing: the reference with its gate zeroed) and when
    none does (zeros)."""
    x, mats, logits = swiglu_case(6, 16, 512, 256, bits, seed=70 + bits)
    idx, gate = route_topk(logits, 4)
    idx = idx.astype(np.uint32)
    bad = idx.copy()
    bad[2, 1] = 16
    none = np.full_like(idx, 99)
    outs = {}
    try:
        for name, ids in (("routed", idx), ("one-invalid", bad), ("none-valid", none)):
            lib.set_tuning("moe_permute", -1)
            fused = run_swiglu(x, mats, ids, gate, bits, "float32")
            lib.set_tuning("moe_permute", 1)
            separate = run_swiglu(x, mats, ids, gate, bits, "float32")
            assert np.array_equal(fused, separate), name
            outs[name] = fused
    finally:
        lib.set_tuning("moe_permute", -1)
    assert not np.any(outs["none-valid"])
    v = judge_swiglu(x, mats, idx, gate, outs["routed"], None, "float32")
    assert v.ok, v
    fixed, g0 = idx.copy(), gate.copy()
    fixed[2, 1], g0[2, 1] = 0, 0.0
    v = judge_swiglu(x, mats, fixed, g0, outs["one-invalid"], None, "float32")
    assert v.ok, v


@pytest.mark.parametrize("n,e,k,d_model,d_ffn,bits,scale", [
    (1, 128, 8, 2048, 768, 4, 1.0),    # config 5, the fused path's own case
    (3, 16, 4, 512, 256, 8, 1.0),
    (2, 32, 12, 512, 1024, 4, 1.0),    # k > 8: two slots on some waves
    (2, 16, 4, 512, 1280, 4, 1.0),     # 5 steps: two rounds of weight loads
    (4, 16, 4, 512, 256, 4, 600.0),    # hidden states beyond fp16 range
])
def test_down_combine_equals_the_two_launches(n, e, k, d_model, d_ffn, bits, scale):
    """The down projection fused with the gated sum (tuning key
    moe_down_combine = 1) is bit-identical to the down launch followed by
    the scatter (= 0) when that launch walks each tile's steps in one wave
    (moe_kq = 1, as the fused kernel does): the same fp32 y_s, summed in
    slot order. Also with a slot naming no expert and with none valid; fp16
    and fp32 outputs; the fused output against the oracle."""
    x, mats, logits = swiglu_case(n, e, d_model, d_ffn, bits, seed=90 + n + k)
    x = (x.astype(np.float32) * scale).astype(np.float16)
    idx, gate = route_topk(logits, k)
    idx = idx.astype(np.uint32)
    bad = idx.copy()
    bad[n - 1, 1] = e
    none = np.full_like(idx, e + 5)
    try:
        lib.set_tuning("moe_kq", 1)
        for name, ids in (("routed", idx), ("one-invalid", bad), ("none-valid", none)):
            for dtype in ("float16", "float32"):
                lib.set_tuning("moe_down_combine", 1)
                fused = run_swiglu(x, mats, ids, gate, bits, dtype)
                lib.set_tuning("moe_down_combine", 0)
                separate = run_swiglu(x, mats, ids, gate, bits, dtype)
                assert np.array_equal(fused, separate), (name, dtype)
                if name == "none-valid":
                    assert not np.any(fused)
                elif name == "routed" and dtype == "float32":
                    v = judge_swiglu(x, mats, idx, gate, fused, [0, n - 1], "float32")
                    assert v.ok, v
    finally:
        lib.set_tuning("moe_down_combine", -1)
        lib.set_tuning("moe_kq", -1)


@pytest.mark.parametrize("n", [64, 65])
def test_in_block_routing_limit(n):
    """n * k = 512 pairs is the largest in-block routing (bit-identical to
    the permute launch); 520 takes the permute launch. Both against the
    oracle on three tokens."""
    x, mats, logits = swiglu_case(n, 128, 512, 256, 4, seed=80 + n)
    idx, gate = route_topk(logits, 8)
    idx = idx.astype(np.uint32)
    out = run_swiglu(x, mats, idx, gate, 4, "float32")
    if n * 8 <= 512:
        lib.set_tuning("moe_permute", 1)
        try:
            assert np.array_equal(out, run_swiglu(x, mats, idx, gate, 4, "float32"))
        finally:
            lib.set_tuning("moe_permute", -1)
    v = judge_swiglu(x, mats, idx, gate, out, [0, n // 2, n - 1], "float32")
    assert v.ok, v


@pytest.mark.parametrize("n,e,k,bits", [(1, 128, 8, 4), (3, 64, 4, 8), (8, 128, 8, 4),
                                        (12, 128, 8, 4), (2, 200, 6, 4), (4, 32, 4, 2)])
def test_route_swiglu_equals_route_then_swiglu(n, e, k, bits):
    """kvp_moe_route_swiglu (routing inside the gate/up launch for up to 4
    tokens on the matrix cores, the routing kernel first otherwise) writes
    the same indices and gates as kvp_moe_route_logits and the same output,
    bit for bit, as kvp_moe_swiglu on that routing; the output also passes
    the oracle on the contract's routing."""
    d_model, d_ffn = 512, 256
    x, mats, logits = swiglu_case(n, e, d_model, d_ffn, bits, seed=300 + n * e + bits)
    assert not near_tie_rows(logits, k, ulps=64).any()
    idx, gate = moe.route(logits, k)
    want = run_swiglu(x, mats, idx, gate, bits, "float32")
    got, idx2, gate2 = moe.route_swiglu_host(x, logits, k, mats["gate"][:3], mats["up"][:3],
                                             mats["down"][:3], bits=bits, out_dtype="float32")
    assert np.array_equal(idx2, idx) and np.array_equal(gate2, gate)
    assert np.array_equal(got, want)
    want_idx, want_gate = route_topk(logits, k)
    assert np.array_equal(idx2.astype(np.int64), want_idx)
    v = judge_swiglu(x, mats, want_idx, gate2, got, None, "float32")
    assert v.ok, v


def test_route_swiglu_config5_one_token_and_constant_logits():
    """BASELINE config 5 at n = 1 through the fused call, and constant logits
    (every expert ties: experts 0..k-1, gates 1/k)."""
    x, mats, logits = swiglu_case(1, 128, 2048, 768, 4, seed=5)
    out, idx, gate = moe.route_swiglu_host(x, logits, 8, mats["gate"][:3], mats["up"][:3],
                                           mats["down"][:3], bits=4)
    want_idx, _ = route_topk(logits, 8)
    assert np.array_equal(idx.astype(np.int64), want_idx)
    v = judge_swiglu(x, mats, want_idx, gate, out, None)
    assert v.ok, v
    flat = np.full((2, 128), 0.5, dtype=np.float32)
    out, idx, gate = moe.route_swiglu_host(x[:1].repeat(2, 0), flat, 8, mats["gate"][:3],
                                           mats["up"][:3], mats["down"][:3], bits=4)
    assert np.array_equal(idx, np.tile(np.arange(8, dtype=np.uint32), (2, 1)))
    assert np.allclose(gate, 1 / 8, atol=1e-7)
