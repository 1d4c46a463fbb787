"""bench.py's CPU paths (the numpy ports timed beside each KV and MoE row)
against the oracle on small cases: host dequantization of 4- and 8-bit
streams, the KV decode step on shared and per-sequence caches, and the MoE
SwiGLU step. No device is touched."""

from __future__ import annotations

import numpy as np
import pytest

import bench
from oracle.extensions import kv_reference_gqa, route_topk, swiglu_reference
from oracle.quant_contract import QuantContract, canonical_quantize, dequantize, pack_codes


def _stored(raw, bits):
    """A raw (..., DH) fp16 array as the stored artefact (codes, scales, biases)."""
    dh = raw.shape[-1]
    art = canonical_quantize(raw.reshape(-1, dh), QuantContract(bits=bits, group_size=64))
    lead = raw.shape[:-1]
    return art, [pack_codes(art.q, bits).reshape(lead + (-1,)), art.scales.reshape(lead + (-1,)),
                 art.biases.reshape(lead + (-1,))]


@pytest.mark.parametrize("bits", [4, 8])
def test_host_dequant_is_the_contract_dequantize(bits):
    raw = np.random.default_rng(bits).standard_normal((6, 256)).astype(np.float16)
    art, parts = _stored(raw, bits)
    assert np.array_equal(bench.host_dequant(*parts, bits), dequantize(art, np.float32))


@pytest.mark.parametrize("bits,per_seq", [(4, False), (8, True)])
def test_kv_cpu_path_is_the_oracle(bits, per_seq):
    rng = np.random.default_rng(10 + bits)
    b, h, hkv, ts, dh = 2, 8, 2, 160, 128
    c = b if per_seq else 1
    kr = rng.standard_normal((c, hkv, ts, dh)).astype(np.float16)
    vr = rng.standard_normal((c, hkv, ts, dh)).astype(np.float16)
    kp, vp = _stored(kr, bits)[1], _stored(vr, bits)[1]
    if not per_seq:
        kp, vp = [a[0] for a in kp], [a[0] for a in vp]
    q = rng.standard_normal((b, h, dh)).astype(np.float16)
    nk = rng.standard_normal((b, hkv, dh)).astype(np.float16)
    nv = rng.standard_normal((b, hkv, dh)).astype(np.float16)
    lengths = [97, 160]
    out = bench.kv_cpu_path(q, nk, nv, kp, vp, lengths, bits, per_seq)
    for i, t in enumerate(lengths):
        cc = i if per_seq else 0
        ref = kv_reference_gqa(q[i:i + 1], kr[cc][:, :t], vr[cc][:, :t], nk[i:i + 1],
                               nv[i:i + 1], bits)
        assert np.max(np.abs(out[i:i + 1] - ref)) <= 1e-5 * np.max(np.abs(ref))


def test_moe_cpu_path_is_the_oracle():
    rng = np.random.default_rng(3)
    e, dm, df, n, k = 12, 128, 64, 5, 4
    raw = [(rng.standard_normal(s) * 0.05).astype(np.float16)
           for s in ((e, df, dm), (e, df, dm), (e, dm, df))]
    arts, host = [], []
    for w in raw:
        per = [canonical_quantize(w[j], QuantContract(bits=4, group_size=64)) for j in range(e)]
        arts.append(per)
        host.append((np.stack([pack_codes(a.q, 4) for a in per]),
                     np.stack([a.scales for a in per]), np.stack([a.biases for a in per])))
    x = rng.standard_normal((n, dm)).astype(np.float16)
    logits = rng.standard_normal((n, e)).astype(np.float32)
    out = bench.moe_cpu_path(x, logits, k, *host, 4)
    idx, gate = route_topk(logits, k)
    ref = swiglu_reference(x, idx, gate, *arts)
    assert np.max(np.abs(out - ref)) <= 1e-4 * np.max(np.abs(ref))
