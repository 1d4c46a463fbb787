"""Pins of the quantized-KV decode oracle (oracle.native_ops.kv_reference and
kv_tolerance, and the GQA-indexed oracle.extensions.kv_reference_gqa) against
torch's own attention routine, scaled_dot_product_attention in fp64 with its
default 1/sqrt(DH) scale:

- caches whose rows lie on the quantization grid (every group spans
  [-1, 1 - 2^(1-bits)] in steps of 2^(1-bits)) quantize exactly, so the oracle
  must equal plain attention over [K; new_k] and [V; new_v];
- drawn caches: plain attention over the dequantized caches (the quant
  contract's own dequantize, pinned by the golden records);
- grouped-query heads through SDPA's enable_gqa (query head h reads KV head
  h // G);
- the tolerance admits the fp32 members and rejects planted mistakes in the
  oracle: scores scaled by 1/DH, V bias dropped, the new entry dropped,
  values read one position late.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle.extensions import kv_reference_gqa
from oracle.native_ops import _kv_member, KV_MEMBERS, kv_reference
from oracle.quant_contract import QuantContract, canonical_quantize, dequantize
from oracle.verify import kv_inputs, reference_and_tolerance


def _sdpa(q, k, v, new_k, new_v, gqa=False):
    """q (B, H, DH); k, v (HK, T, DH) shared by the batch; new_k/new_v
    (B, HK, DH): one decode step of attention over T + 1 positions."""
    b = q.shape[0]
    qt = torch.from_numpy(q.astype(np.float64))[:, :, None, :]
    kt = torch.cat([torch.from_numpy(k.astype(np.float64))[None].expand(b, -1, -1, -1),
                    torch.from_numpy(new_k.astype(np.float64))[:, :, None, :]], dim=2)
    vt = torch.cat([torch.from_numpy(v.astype(np.float64))[None].expand(b, -1, -1, -1),
                    torch.from_numpy(new_v.astype(np.float64))[:, :, None, :]], dim=2)
    return F.scaled_dot_product_attention(qt, kt, vt, enable_gqa=gqa)[:, :, 0].numpy()


def _grid_cache(rng, h, t, dh, bits):
    """Rows on the grid -1 + j 2^(1-bits), j = 0 .. 2^bits - 1, each group
    holding both ends (so its min and max fix the step exactly)."""
    top = (1 << bits) - 1
    codes = rng.integers(0, top + 1, size=(h, t, dh))
    codes[..., 0::64] = 0
    codes[..., 1::64] = top
    return (-1.0 + codes * 2.0 ** (1 - bits)).astype(np.float16)


def _dequant(cache, bits):
    h, t, dh = cache.shape
    art = canonical_quantize(cache.reshape(h * t, dh), QuantContract(bits=bits, group_size=64))
    return dequantize(art, np.float64).reshape(h, t, dh)


def _case(seed, b, h, t, dh, hk=None):
    rng = np.random.default_rng(seed)
    hk = hk or h
    q = (rng.standard_normal((b, h, dh)) * 0.5).astype(np.float16)
    k = rng.standard_normal((hk, t, dh)).astype(np.float16)
    v = rng.standard_normal((hk, t, dh)).astype(np.float16)
    nk = rng.standard_normal((b, hk, dh)).astype(np.float16)
    nv = rng.standard_normal((b, hk, dh)).astype(np.float16)
    return rng, q, k, v, nk, nv


@pytest.mark.parametrize("bits,dh", [(4, 64), (4, 128), (8, 128), (2, 64)])
def test_grid_caches_are_plain_attention(bits, dh):
    rng, q, _, _, nk, nv = _case(bits + dh, 2, 4, 40, dh)
    k, v = _grid_cache(rng, 4, 40, dh, bits), _grid_cache(rng, 4, 40, dh, bits)
    assert np.array_equal(_dequant(k, bits), k.astype(np.float64))
    ref = kv_reference(kv_inputs(q, k, v, nk, nv, bits))
    want = _sdpa(q, k, v, nk, nv)
    assert np.max(np.abs(ref - want)) <= 1e-12 * np.max(np.abs(want))


@pytest.mark.parametrize("bits", [3, 4, 8])
def test_drawn_caches_are_attention_over_the_dequantized_cache(bits):
    _, q, k, v, nk, nv = _case(10 + bits, 3, 2, 70, 128)
    ref = kv_reference(kv_inputs(q, k, v, nk, nv, bits))
    want = _sdpa(q, _dequant(k, bits), _dequant(v, bits), nk, nv)
    assert np.max(np.abs(ref - want)) <= 1e-12 * np.max(np.abs(want))


def test_grouped_query_oracle_is_sdpa_with_gqa():
    _, q, k, v, nk, nv = _case(7, 2, 8, 33, 64, hk=2)
    ref = kv_reference_gqa(q, k, v, nk, nv, 4)
    want = _sdpa(q, _dequant(k, 4), _dequant(v, 4), nk, nv, gqa=True)
    assert np.max(np.abs(ref - want)) <= 1e-12 * np.max(np.abs(want))


def _mistake(q, k, v, nk, nv, bits, kind):
    """A planted mistake in the oracle's own formula (fp64, CPU)."""
    kd, vd = _dequant(k, bits), _dequant(v, bits)
    dh = q.shape[-1]
    if kind == "v-bias-dropped":
        h, t, _ = v.shape
        art = canonical_quantize(v.reshape(h * t, dh), QuantContract(bits=bits, group_size=64))
        vd = (art.q * art.scales.astype(np.float64).repeat(64, axis=1)).reshape(h, t, dh)
    if kind == "values-one-late":
        vd = np.roll(vd, -1, axis=1)
    qt = torch.from_numpy(q.astype(np.float64))[:, :, None, :]
    if kind == "new-entry-dropped":
        b = q.shape[0]
        kt = torch.from_numpy(kd)[None].expand(b, -1, -1, -1)
        vt = torch.from_numpy(vd)[None].expand(b, -1, -1, -1)
        return F.scaled_dot_product_attention(qt, kt, vt)[:, :, 0].numpy()
    scale = 1.0 / dh if kind == "scale-1-over-dh" else None
    b = q.shape[0]
    kt = torch.cat([torch.from_numpy(kd)[None].expand(b, -1, -1, -1),
                    torch.from_numpy(nk.astype(np.float64))[:, :, None, :]], dim=2)
    vt = torch.cat([torch.from_numpy(vd)[None].expand(b, -1, -1, -1),
                    torch.from_numpy(nv.astype(np.float64))[:, :, None, :]], dim=2)
    return F.scaled_dot_product_attention(qt, kt, vt, scale=scale)[:, :, 0].numpy()


@pytest.mark.parametrize("bits", [4, 8])
def test_tolerance_admits_fp32_and_rejects_planted_mistakes(bits):
    _, q, k, v, nk, nv = _case(20 + bits, 2, 4, 96, 128)
    inputs = kv_inputs(q, k, v, nk, nv, bits)
    ref, tol = reference_and_tolerance("kv_attention", inputs)
    for kw in KV_MEMBERS.values():
        assert np.max(np.abs(_kv_member(inputs, **kw).astype(np.float64) - ref)) <= tol
    for kind in ("scale-1-over-dh", "v-bias-dropped", "new-entry-dropped", "values-one-late"):
        err = np.max(np.abs(_mistake(q, k, v, nk, nv, bits, kind) - ref))
        assert err > tol, (kind, err, tol)
