"""CPU control paths of the three pack operators, with their fault seams.

Follows vladmt06/kernelverify ``kernelverify/reference/native_kernels.py``:
``quantized_matmul`` :41-83, ``_topk_by_prob`` :92-101, ``moe_dispatch``
:104-147, ``_cache_dequant`` :153-165, ``kv_attention`` :168-221.

These are the "reference CPU path" the bench times beside the GPU (the
reference's own CPU implementation of each operator), and the correct
default of each is also an ensemble member of the moe tolerance.

Differences from the reference, all additive: ``TOP_K`` is a parameter
(``k``) rather than a module constant fixed at 2, because the MI355X
workload routes top-8; ``k=2`` reproduces the reference exactly.

Parity (tests/test_oracle_contract.py): each control agrees with its fp64
reference at the reference's own bounds (``tests/test_native_ops.py:37-42,
57-75, 115-122``: qmm < 5e-2 at bits 2/3/4/8, moe < 1e-4, kv < 5e-3 at bits
4/8), passes its own ensemble tolerance on a sampled case set, and every
non-equivalent seam is rejected by that tolerance on at least one sampled
case; the two equivalent moe seams stay equivalent. ``quantized_matmul_artefact``
is bit-identical to ``quantized_matmul`` on the canonical artefact and inside
the contract on drawn codes. ``_topk_by_prob`` is pinned by brute force and
the constant-row known answer (tests/test_oracle_routing.py).
"""

from __future__ import annotations

import numpy as np

from oracle.quant_contract import (
    QuantContract,
    canonical_quantize,
    dequantize,
    fault_bias_dropped,
    fault_group_size_halved,
    fault_nibble_swapped,
    fault_scales_rotated,
)

TOP_K = 2


def quantized_matmul(inputs, *, scales_rotated=False, nibble_swapped=False,
                     bias_dropped=False, group_size_halved=False,
                     dequant_dtype="float32", accum_dtype="float32"):
    """x @ dequant(quantize(w)).T: canonical quantize, fp32 dequant, BLAS MAC."""
    x, w = inputs["x"], inputs["w"]
    bits = int(inputs["bits"][0])
    art = canonical_quantize(w, QuantContract(bits=bits, group_size=64))
    for on, fault in ((scales_rotated, fault_scales_rotated),
                      (nibble_swapped, fault_nibble_swapped),
                      (bias_dropped, fault_bias_dropped),
                      (group_size_halved, fault_group_size_halved)):
        if on:
            art = fault(art)
    wd = dequantize(art, np.float32)
    if dequant_dtype != "float32":
        wd = wd.astype(dequant_dtype).astype(np.float32)
    if accum_dtype in ("float16", "float16-seq"):
        prods = x.astype(np.float16)[:, None, :] * wd.astype(np.float16)[None, :, :]
        if accum_dtype == "float16-seq":
            out = np.add.accumulate(prods, axis=-1, dtype=np.float16)[..., -1]
        else:
            out = np.add.reduce(prods, axis=-1, dtype=np.float16)
        return out.astype(x.dtype)
    return (x.astype(np.float32) @ wd.T).astype(x.dtype)


def quantized_matmul_artefact(x, art):
    """The same control path on a given artefact (no quantize step): fp32
    dequant then BLAS. The bench's CPU baseline for directly drawn artefacts."""
    return (x.astype(np.float32) @ dequantize(art, np.float32).T).astype(x.dtype)


def _topk_by_prob(probs, k, tie_high=False):
    """k largest per row; ties to the LOWER index (stable sort of -p), or to
    the higher index with ``tie_high``."""
    order = np.argsort(-probs, axis=-1, kind="stable")
    if tie_high:
        rev = np.argsort(-probs[:, ::-1], axis=-1, kind="stable")
        order = probs.shape[-1] - 1 - rev
    return order[:, :k]


def moe_dispatch(inputs, *, renormalize=True, expert_offset=0,
                 gate_dtype="float32", k_offset=0, tie_high=False,
                 softmax_topk_order=False, k=TOP_K):
    """Routing (fp32 logits, softmax over all experts, top-k by probability,
    ties low, renormalise) then sum_k gate_k * (x @ expert_k^T)."""
    x, router, experts = inputs["x"], inputs["router"], inputs["experts"]
    xf = x.astype(np.float32)
    logits = xf @ router.astype(np.float32).T
    if gate_dtype != "float32":
        logits = logits.astype(gate_dtype).astype(np.float32)
    probs = np.exp(logits - logits.max(axis=-1, keepdims=True))
    probs /= probs.sum(axis=-1, keepdims=True)

    kk = k + k_offset
    top = _topk_by_prob(probs, kk, tie_high)
    if softmax_topk_order:
        chosen = np.take_along_axis(logits, top, axis=-1)
        weights = np.exp(chosen - chosen.max(axis=-1, keepdims=True))
        weights /= weights.sum(axis=-1, keepdims=True)
    else:
        weights = np.take_along_axis(probs, top, axis=-1)
        if renormalize:
            weights = weights / weights.sum(axis=-1, keepdims=True)

    n_exp = experts.shape[0]
    out = np.zeros((x.shape[0], experts.shape[1]), dtype=np.float32)
    for row in range(x.shape[0]):
        for slot in range(kk):
            e = (int(top[row, slot]) + expert_offset) % n_exp
            out[row] += weights[row, slot] * (xf[row] @ experts[e].astype(np.float32).T)
    return out.astype(x.dtype)


def _cache_dequant(cache, bits, fault=None):
    """Canonically quantize an (H, T, DH) cache as its (H*T, DH) reshape and
    dequantize at fp32."""
    h, t, dh = cache.shape
    art = canonical_quantize(cache.reshape(h * t, dh), QuantContract(bits=bits, group_size=64))
    if fault is not None:
        art = fault(art)
    return dequantize(art, np.float32).reshape(h, t, dh)


def kv_attention(inputs, *, scores_dtype="float32", accum_dtype="float32",
                 k_scales_rotated=False, v_bias_dropped=False,
                 new_entry_skipped=False, dhead_scale_dropped=False):
    """One decode step over a quantized cache shared by the batch: scores for
    T cached positions plus the new entry, fp32 softmax over T+1, combine."""
    q, new_k, new_v = inputs["q"], inputs["new_k"], inputs["new_v"]
    bits = int(inputs["bits"][0])
    dh = q.shape[-1]
    kd = _cache_dequant(inputs["k_cache"], bits, fault_scales_rotated if k_scales_rotated else None)
    vd = _cache_dequant(inputs["v_cache"], bits, fault_bias_dropped if v_bias_dropped else None)

    qf = q.astype(np.float32)
    scale = 1.0 if dhead_scale_dropped else 1.0 / np.sqrt(np.float32(dh))
    scores = np.einsum("bhd,htd->bht", qf, kd) * scale
    s_new = np.sum(qf * new_k.astype(np.float32), axis=-1) * scale
    if not new_entry_skipped:
        scores = np.concatenate([scores, s_new[..., None]], axis=-1)
    if scores_dtype != "float32":
        scores = scores.astype(scores_dtype).astype(np.float32)
    probs = np.exp(scores - scores.max(axis=-1, keepdims=True))
    probs /= probs.sum(axis=-1, keepdims=True)

    pc = probs[..., :kd.shape[1]]
    if accum_dtype in ("float16", "float16-seq"):
        contrib = pc.astype(np.float16)[..., None] * vd.astype(np.float16)[None, ...]
        if accum_dtype == "float16-seq":
            out = np.add.accumulate(contrib, axis=2, dtype=np.float16)[:, :, -1]
        else:
            out = np.add.reduce(contrib, axis=2, dtype=np.float16)
        out = out.astype(np.float32)
    else:
        out = np.einsum("bht,htd->bhd", pc, vd)
    if not new_entry_skipped:
        out = out + probs[..., -1][..., None] * new_v.astype(np.float32)
    return out.astype(q.dtype)


NATIVE_KERNELS = {
    "quantized_matmul": quantized_matmul,
    "moe_dispatch": moe_dispatch,
    "kv_attention": kv_attention,
}
