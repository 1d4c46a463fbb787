"""Seeded input generators of the reference's calibration and gate harnesses.

Follows vladmt06/kernelverify ``bench/phase0_contract_k.py:64-82`` (``make_x``,
``make_w``), ``bench/pack_wide_qmv.py:124-131`` (``weights_for``),
``bench/pack_kv_attention.py:75-88`` (``make_case``) and
``bench/pack_moe_dispatch.py:76-100`` (``make_case``). The rng call order is
part of each definition: the committed golden records were produced from
these exact streams, so a reordered draw shows up as a golden mismatch.
"""

from __future__ import annotations

import numpy as np

MODES = ("unit", "corpus-scale", "near-zero", "constant-rows")
WEIGHT_DRAWS = ("normal-0.02", "heavy-tailed")


def make_x(batch, d_in, dtype, mode, rng):
    x = rng.standard_normal((batch, d_in)).astype(np.float32)
    if mode == "corpus-scale":
        x = x * np.float32(10.0)
    elif mode == "near-zero":
        x = x * np.float32(1e-3)
    elif mode == "constant-rows":
        x = np.broadcast_to(x[:, :1], x.shape).copy()
    return x.astype(dtype)


def make_w(d_out, d_in, draw, rng):
    w = rng.standard_normal((d_out, d_in)).astype(np.float32)
    if draw == "normal-0.02":
        w = w * np.float32(0.02)
    else:
        w = (w ** 3) * np.float32(0.02)
    return w.astype(np.float16)


def weights_for(d_out, d_in, seed):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((d_out, d_in)).astype(np.float32) * 0.02).astype(np.float16)


def kv_case(b, h, t, dh, seed, dtype="float16"):
    """q and new_k at peak 0.6, caches and new_v at unit scale."""
    rng = np.random.default_rng(seed)

    def peaked(shape):
        a = rng.standard_normal(shape).astype(np.float32)
        return (a * (0.6 / float(np.max(np.abs(a))))).astype(dtype)

    q, new_k = peaked((b, h, dh)), peaked((b, h, dh))
    k_cache = rng.standard_normal((h, t, dh)).astype(dtype)
    v_cache = rng.standard_normal((h, t, dh)).astype(dtype)
    new_v = rng.standard_normal((b, h, dh)).astype(dtype)
    return q, k_cache, v_cache, new_k, new_v


def moe_case(n_tokens, d_model, n_experts, d_ffn, seed, mode="normal"):
    rng = np.random.default_rng(seed)
    if mode == "constant_rows":
        x = np.repeat(rng.standard_normal((n_tokens, 1)).astype(np.float32),
                      d_model, axis=1).astype(np.float16)
        router = np.repeat(rng.standard_normal((1, d_model)).astype(np.float32) * 0.05,
                           n_experts, axis=0).astype(np.float16)
    else:
        x = (rng.standard_normal((n_tokens, d_model)).astype(np.float32) * 0.5).astype(np.float16)
        router = (rng.standard_normal((n_experts, d_model)).astype(np.float32)
                  * 0.05).astype(np.float16)
    experts = (rng.standard_normal((n_experts, d_ffn, d_model)).astype(np.float32)
               * 0.02).astype(np.float16)
    return x, router, experts
