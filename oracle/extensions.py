"""Generalisations the MI355X configs need beyond the reference's contracts.

Nothing here changes a reference formula; each function composes the
reference's own contracts in the way the reference's tests already do:

- ``kv_gqa_inputs``: GQA (H query heads over HKV cache heads) as the tiled
  cache, exactly ``tests/test_pack_kv_attention.py:176-205``: quantization is
  per cache row, so tiling the raw cache then quantizing equals quantizing
  then tiling.
- ``kv_per_sequence``: one B=1 oracle case per sequence with its own cache
  and length, the batch-row independence of
  ``tests/test_pack_kv_attention.py:120-130``.
- ``kv_reference_gqa`` / ``kv_tolerance_gqa``: the same reference and the same
  four members with query head h indexing cache head h // r instead of a
  tiled copy (identical per-head arithmetic; long contexts no longer
  quantize r copies of the cache). Pinned to the tiled form by
  tests/test_oracle_kv_gqa.py.
- ``route_topk``: the routing contract of ``schemas/native_ops.py:193-206`` at
  any k, from logits given directly (config 5 draws logits, not x @ router).
- ``permute_by_expert``: the stable counting sort of (token, slot) pairs by
  expert the dispatch kernels consume (closed form).
- ``swiglu_*``: the gate/up/down expert MLP of config 5. The reference has one
  linear per expert and no such composition; each projection follows the
  quantized_matmul contract.

Parity: kv wrappers inherit ``kv_reference``'s pins; ``route_topk`` is pinned by
brute force (sorting by (-p, index)) and torch ``sort(stable=True)``;
``permute_by_expert`` by brute force; ``swiglu_reference`` by a closed form
(experts that dequantize to scaled permutation matrices, silu per element)
and invariants (slot order, gate linearity, a repeated expert, zero gates),
``swiglu_tolerance`` by admitting its fp32 members and rejecting planted
mistakes (tests/test_oracle_swiglu.py); ``moe_linear_reference`` by a
closed form on permutation experts and equality with ``moe_reference`` on
the same routing, ``moe_linear_tolerance`` by admitting an fp32 evaluation
in another order and rejecting five planted mistakes
(tests/test_oracle_contract.py).
"""

from __future__ import annotations

import numpy as np

from oracle.floor import floored_tolerance
from oracle.native_kernels import _cache_dequant
from oracle.native_ops import K_QUANT, _base_tol, kv_reference, kv_tolerance, route_probs
from oracle.quant_contract import ENSEMBLE, QuantArtefact, dequantize
from oracle.verify import _Case, kv_inputs


# ---------------------------------------------------------------------------
# KV decode: GQA and per-sequence caches
# ---------------------------------------------------------------------------
def kv_gqa_inputs(q, k_cache, v_cache, new_k, new_v, bits):
    """q (B, H, DH); caches (HKV, T, DH); new_k/new_v (B, HKV, DH)."""
    r = q.shape[1] // k_cache.shape[0]
    tile = lambda a, axis: np.repeat(a, r, axis=axis)
    return kv_inputs(q, tile(k_cache, 0), tile(v_cache, 0), tile(new_k, 1), tile(new_v, 1), bits)


def _gqa_dequant(cache, bits):
    """The fp64 view of a canonically quantized (HKV, T, DH) cache, exactly as
    ``native_ops._kv_dequant64`` forms it (fp32 dequant, then widened)."""
    return _cache_dequant(cache, bits).astype(np.float64)


def kv_reference_gqa(q, k_cache, v_cache, new_k, new_v, bits, kd=None, vd=None):
    """``kv_reference`` with query head h reading cache head h // r, without
    tiling the cache: q (B, H, DH); caches (HKV, T, DH); new_k/new_v
    (B, HKV, DH). Same fp64 formula (native_ops.kv_reference); the tiled form
    pins it (tests/test_oracle_kv_gqa.py)."""
    b, h, dh = q.shape
    hkv = k_cache.shape[0]
    r = h // hkv
    kd = _gqa_dequant(k_cache, bits) if kd is None else kd
    vd = _gqa_dequant(v_cache, bits) if vd is None else vd
    q64 = q.astype(np.float64).reshape(b, hkv, r, dh)
    scale = 1.0 / np.sqrt(float(dh))
    scores = np.einsum("bgrd,gtd->bgrt", q64, kd) * scale
    s_new = np.sum(q64 * new_k.astype(np.float64)[:, :, None, :], axis=-1) * scale
    scores = np.concatenate([scores, s_new[..., None]], axis=-1)
    probs = np.exp(scores - scores.max(axis=-1, keepdims=True))
    probs /= probs.sum(axis=-1, keepdims=True)
    out = np.einsum("bgrt,gtd->bgrd", probs[..., :-1], vd)
    out = out + probs[..., -1][..., None] * new_v.astype(np.float64)[:, :, None, :]
    return out.reshape(b, h, dh)


def _kv_member_gqa(q, kd64, vd64, new_k, new_v, *, scores_order, combine_order):
    """``native_ops._kv_member`` with the head mapping h -> h // r: per query
    head, the same fp32 operations in the same order as on the tiled cache."""
    b, h, dh = q.shape
    hkv = kd64.shape[0]
    r = h // hkv
    q32 = q.astype(np.float32)
    kd = kd64.astype(np.float32)
    vd = vd64.astype(np.float32)
    nk = np.repeat(new_k.astype(np.float32), r, axis=1)
    nv = np.repeat(new_v.astype(np.float32), r, axis=1)
    scale = np.float32(1.0 / np.sqrt(float(dh)))
    t = kd.shape[1]
    scores = np.empty((b, h, t), dtype=np.float32)
    for hh in range(h):
        g = hh // r
        if scores_order == "serial":
            prods = q32[:, hh, None, :] * kd[None, g]
            scores[:, hh] = np.add.accumulate(prods, axis=-1, dtype=np.float32)[..., -1]
        else:
            scores[:, hh] = np.einsum("bd,td->bt", q32[:, hh], kd[g])
    scores = scores * scale
    s_new = np.sum(q32 * nk, axis=-1) * scale
    scores = np.concatenate([scores, s_new[..., None]], axis=-1)
    probs = np.exp(scores - scores.max(axis=-1, keepdims=True))
    probs /= probs.sum(axis=-1, keepdims=True)
    pc = probs[..., :-1]
    out = np.empty(q.shape, dtype=np.float32)
    for hh in range(h):
        g = hh // r
        if combine_order in ("serial", "reversed"):
            contrib = pc[:, hh, :, None] * vd[None, g]
            if combine_order == "reversed":
                contrib = contrib[:, ::-1, :]
            out[:, hh] = np.add.accumulate(contrib, axis=1, dtype=np.float32)[:, -1]
        else:
            out[:, hh] = np.einsum("bt,td->bd", pc[:, hh], vd[g])
    out = out + probs[..., -1][..., None] * nv
    return out.astype(q.dtype)


def kv_tolerance_gqa(dtype, q, k_cache, v_cache, new_k, new_v, bits, ref, kd=None, vd=None):
    """``kv_tolerance`` over the four KV members in their GQA-indexed form."""
    from oracle.native_ops import KV_MEMBERS, K_QUANT

    kd = _gqa_dequant(k_cache, bits) if kd is None else kd
    vd = _gqa_dequant(v_cache, bits) if vd is None else vd
    return floored_tolerance(_base_tol(dtype, ref), K_QUANT,
                             (_kv_member_gqa(q, kd, vd, new_k, new_v, **kw)
                              for kw in KV_MEMBERS.values()), ref)


def kv_per_sequence(q, k_caches, v_caches, new_k, new_v, lengths, bits, dtype="float16",
                    with_tolerance=True):
    """Reference (B, H, DH) and the per-sequence tolerances.

    k_caches/v_caches: per-sequence raw caches (HKV, T_b, DH) of length
    ``lengths[b]`` (extra rows past the length are ignored). Each sequence
    is an independent B = 1 case in the GQA-indexed form."""
    refs, tols = [], []
    for b, t in enumerate(lengths):
        kc, vc = k_caches[b][:, :t], v_caches[b][:, :t]
        kd, vd = _gqa_dequant(kc, bits), _gqa_dequant(vc, bits)
        args = (q[b:b + 1], kc, vc, new_k[b:b + 1], new_v[b:b + 1], bits)
        ref = kv_reference_gqa(*args, kd=kd, vd=vd)
        refs.append(ref)
        if with_tolerance:
            tols.append(kv_tolerance_gqa(dtype, *args, ref, kd=kd, vd=vd))
    return np.concatenate(refs, axis=0), (tols if with_tolerance else None)


# ---------------------------------------------------------------------------
# MoE routing from logits, token permutation
# ---------------------------------------------------------------------------
def route_topk(logits: np.ndarray, k: int):
    """fp32 contract routing: (idx (n, k) int64, gate (n, k) fp32)."""
    top, weights = route_probs(logits.astype(np.float32), k, np.float32)
    return top, weights.astype(np.float32)


def near_tie_rows(logits: np.ndarray, k: int, ulps: int = 2):
    """Rows whose k-th and (k+1)-th probabilities lie within ``ulps`` fp32
    ulps: a GPU exp that differs from numpy's in the last bit may order them
    differently, so bit-exact index checks report these rows separately."""
    logits = logits.astype(np.float32)
    probs = np.exp(logits - logits.max(axis=-1, keepdims=True))
    probs /= probs.sum(axis=-1, keepdims=True)
    srt = -np.sort(-probs, axis=-1)
    if k >= probs.shape[1]:
        return np.zeros(probs.shape[0], dtype=bool)
    gap = srt[:, k - 1] - srt[:, k]
    return gap <= ulps * np.spacing(srt[:, k - 1])


def permute_by_expert(idx: np.ndarray, n_experts: int):
    """Stable counting sort of the flattened (token, slot) pairs by expert.

    Returns (offsets (E+1,) int32, perm (n*k,) int32) with perm listing the
    flat index token*k + slot in expert order, ties in flat-index order."""
    flat = idx.reshape(-1).astype(np.int64)
    counts = np.bincount(flat, minlength=n_experts)
    offsets = np.zeros(n_experts + 1, dtype=np.int32)
    offsets[1:] = np.cumsum(counts)
    perm = np.argsort(flat, kind="stable").astype(np.int32)
    return offsets, perm


# ---------------------------------------------------------------------------
# SwiGLU experts (config 5): gate/up (I, D), down (D, I), all quantized
# ---------------------------------------------------------------------------
def _silu(a):
    return a / (1.0 + np.exp(-a))


def _dense(arts, dtype):
    return [dequantize(a, dtype) for a in arts]


def swiglu_reference(x, idx, gate, gate_arts, up_arts, down_arts):
    """fp64: out[t] = sum_s gate[t,s] * Wd_e (silu(Wg_e x_t) * (Wu_e x_t))."""
    out = np.zeros((x.shape[0], down_arts[int(idx[0, 0])].q.shape[0]), dtype=np.float64)
    x64 = x.astype(np.float64)
    cache = {}
    for t in range(x.shape[0]):
        for s in range(idx.shape[1]):
            e = int(idx[t, s])
            if e not in cache:
                cache[e] = (dequantize(gate_arts[e], np.float64), dequantize(up_arts[e], np.float64),
                            dequantize(down_arts[e], np.float64))
            wg, wu, wd = cache[e]
            h = _silu(wg @ x64[t]) * (wu @ x64[t])
            out[t] += float(gate[t, s]) * (wd @ h)
    return out


def _swiglu_member(x, idx, gate, gate_arts, up_arts, down_arts, *, order="forward",
                   projection="pairwise"):
    """fp32 evaluation: projections pairwise (BLAS) or int-domain factored
    (``factored-groups``), h at fp32, slots accumulated in ``order``."""
    out = np.zeros((x.shape[0], down_arts[int(idx[0, 0])].q.shape[0]), dtype=np.float32)
    x32 = x.astype(np.float32)
    slots = range(idx.shape[1]) if order == "forward" else range(idx.shape[1] - 1, -1, -1)

    def proj(v, art):
        if projection == "factored":
            return ENSEMBLE["factored-groups"](v[None, :].astype(np.float32), art)[0]
        return dequantize(art, np.float32) @ v

    for t in range(x.shape[0]):
        for s in slots:
            e = int(idx[t, s])
            g = proj(x32[t], gate_arts[e])
            u = proj(x32[t], up_arts[e])
            h = (g / (np.float32(1.0) + np.exp(-g))) * u
            out[t] += np.float32(gate[t, s]) * proj(h.astype(np.float32), down_arts[e])
    return out.astype(x.dtype)


SWIGLU_MEMBERS = {
    "swiglu:pairwise-forward": dict(order="forward", projection="pairwise"),
    "swiglu:pairwise-reversed": dict(order="reversed", projection="pairwise"),
    "swiglu:factored-forward": dict(order="forward", projection="factored"),
}


def swiglu_tolerance(dtype, x, idx, gate, gate_arts, up_arts, down_arts, ref):
    """max(base_tol, K_QUANT * worst fp32 member) over the three members."""
    return floored_tolerance(
        _base_tol(dtype, ref), K_QUANT,
        (_swiglu_member(x, idx, gate, gate_arts, up_arts, down_arts, **kw)
         for kw in SWIGLU_MEMBERS.values()), ref)


def moe_linear_reference(x, idx, gate, arts):
    """The reference's single-linear dispatch at any k, given routing:
    out[t] = sum_s gate[t,s] * (x_t @ W_e^T) in fp64 (``_moe_combine``)."""
    out = np.zeros((x.shape[0], arts[int(idx[0, 0])].q.shape[0]), dtype=np.float64)
    dense = {}
    for t in range(x.shape[0]):
        for s in range(idx.shape[1]):
            e = int(idx[t, s])
            if e not in dense:
                dense[e] = dequantize(arts[e], np.float64)
            out[t] += float(gate[t, s]) * (x[t].astype(np.float64) @ dense[e].T)
    return out


def moe_linear_tolerance(dtype, x, idx, gate, arts, ref):
    """K_NATIVE-style two-member floor of the reference (forward and reversed
    slot order at fp32) over the dense fp32 experts."""
    from oracle.native_ops import K_NATIVE

    def member(order):
        out = np.zeros((x.shape[0], arts[int(idx[0, 0])].q.shape[0]), dtype=np.float32)
        slots = range(idx.shape[1]) if order == "f" else range(idx.shape[1] - 1, -1, -1)
        for t in range(x.shape[0]):
            for s in slots:
                e = int(idx[t, s])
                out[t] += np.float32(gate[t, s]) * (x[t].astype(np.float32)
                                                    @ dequantize(arts[e], np.float32).T)
        return out.astype(x.dtype)

    return floored_tolerance(_base_tol(dtype, ref), K_NATIVE, (member("f"), member("r")), ref)


def artefact_from_arrays(q: np.ndarray, scales: np.ndarray, biases: np.ndarray, bits: int):
    """Wrap directly drawn arrays as an artefact (config 1: q ~ U{0..2^b-1})."""
    from oracle.quant_contract import QuantContract

    return QuantArtefact(q=q.astype(np.int32), scales=scales, biases=biases,
                         contract=QuantContract(bits=bits, group_size=64))
