"""The serving door's host logic on CPU (reference: tests/test_serve_sub4bit.py,
the flattened-M rule of docs/adr/0018): code unpacking, the stock paths
against the oracle, every refusal reason, and the patch's install/uninstall.
No kernel runs here; routed calls are `tests/test_serving_gpu.py`."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
from torch import nn

from kernelverify_amd.pack import wide_qmv
from kernelverify_amd.serving import (
    KvDoor,
    Patch,
    QuantizedKVCache,
    QuantizedLinear,
    RoutedLinear,
    unpack_codes,
)
from oracle.extensions import kv_reference_gqa
from oracle.quant_contract import QuantContract, canonical_quantize, dequantize, pack_codes


def _layer(d_out, d_in, bits, seed=0, **kw):
    w = (np.random.default_rng(seed).standard_normal((d_out, d_in)) * 0.02).astype(np.float16)
    art = canonical_quantize(w, QuantContract(bits=bits, group_size=64))
    words = pack_codes(art.q, bits).view(np.int32)
    layer = QuantizedLinear(torch.from_numpy(words.copy()), torch.from_numpy(art.scales.copy()),
                            torch.from_numpy(art.biases.copy()), bits, **kw)
    return layer, art


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
def test_unpack_matches_the_packer(bits):
    q = np.random.default_rng(bits).integers(0, 1 << bits, (5, 192))
    words = torch.from_numpy(pack_codes(q, bits).view(np.int32).copy())
    assert np.array_equal(unpack_codes(words, bits, 192).numpy(), q)


@pytest.mark.parametrize("bits", [3, 4])
def test_stock_linear_is_the_dequantized_product(bits):
    layer, art = _layer(96, 256, bits)
    x = np.random.default_rng(1).standard_normal((3, 256)).astype(np.float32)
    ref = x.astype(np.float64) @ dequantize(art).astype(np.float64).T
    got = layer(torch.from_numpy(x)).numpy()
    assert np.max(np.abs(got - ref)) <= 1e-5 * np.max(np.abs(ref))


def _routed_m(bits, d_out, d_in):
    """An M the committed routing table routes at this cell, and one it does not."""
    window = sorted(m for m in range(2, 17) if wide_qmv.should_dispatch(m, bits, d_out, d_in))
    outside = next(m for m in range(17, 40))
    return window[0] if window else None, outside


def test_flattened_m_is_the_only_judge_at_every_rank():
    layer, _ = _layer(4096, 4096, 4)
    routed = RoutedLinear(layer, Patch(nn.Module()))
    m_in, m_out = _routed_m(4, 4096, 4096)
    assert m_in is not None
    for m, expect in ((m_in, "device-cpu"), (m_out, f"m-{m_out}-outside-dispatch-4096x4096")):
        spellings = [torch.zeros((1, m, 4096), dtype=torch.float16),
                     torch.zeros((m, 1, 4096), dtype=torch.float16),
                     torch.zeros((m, 4096), dtype=torch.float16)]
        assert {routed.ineligible(x) for x in spellings} == {expect}


def test_every_refusal_names_its_reason():
    layer, _ = _layer(128, 256, 4)
    routed = RoutedLinear(layer, Patch(nn.Module()))
    x = torch.zeros((1, 256), dtype=torch.float16)
    assert routed.ineligible(x.float()) == "dtype-torch.float32-torch.float16"
    assert routed.ineligible(torch.zeros((1, 320), dtype=torch.float16)) == "din-320"
    # an unpriced shape routes nowhere
    assert routed.ineligible(x) == "m-1-outside-dispatch-128x256"
    for kw, why in ((dict(mode="mxfp4"), "mode-mxfp4"), (dict(group_size=32), "quant-4b-gs32"),
                    (dict(bias=torch.zeros(128)), "bias-term")):
        other, _ = _layer(128, 256, 4, **kw)
        assert RoutedLinear(other, Patch(nn.Module())).ineligible(x) == why


def test_buffers_the_kernel_would_misread_are_named_refusals():
    """The kernel reads weight, scales and biases raw: a biases dtype other
    than fp16, a code array of the wrong shape (a short one would be read
    past its end) or a strided buffer is refused by name, before M."""
    layer, art = _layer(128, 256, 4)
    x = torch.zeros((1, 256), dtype=torch.float16)
    w, s, b = layer.weight, layer.scales, layer.biases

    def why(weight, scales, biases):
        return RoutedLinear(QuantizedLinear(weight, scales, biases, 4),
                            Patch(nn.Module())).ineligible(x)

    assert why(w, s, b.float()) == "biases-dtype-torch.float32"
    assert why(w, s, b.to(torch.bfloat16)) == "biases-dtype-torch.bfloat16"
    assert why(w[:, :16].contiguous(), s, b) == "weight-shape-(128, 16)"
    assert why(w[:64], s, b) == "weight-shape-(64, 32)"
    assert why(w, s, b[:, :2].contiguous()) == "biases-shape-(128, 2)"
    strided = torch.zeros((128, 64), dtype=torch.int32)[:, ::2]
    strided.copy_(w)
    assert why(strided, s, b) == "noncontiguous"
    assert why(w, s.t().contiguous().t(), b) == "noncontiguous"
    assert why(w, s, b) == "m-1-outside-dispatch-128x256"


def test_patch_wraps_every_site_counts_and_restores():
    a, _ = _layer(4096, 4096, 4, seed=1)
    b, _ = _layer(128, 256, 4, seed=2)
    model = nn.Sequential(a, nn.ReLU(), nn.Sequential(b))
    with pytest.raises(ValueError):
        Patch(nn.Module(), mode="fast")
    patch = Patch(model)
    assert patch.n_wrapped == 2 and patch.site_cells == [(4, 4096, 4096), (4, 128, 256)]
    assert isinstance(model[0], RoutedLinear) and isinstance(model[2][0], RoutedLinear)
    with pytest.raises(RuntimeError):
        Patch(model)
    y = model[0](torch.zeros((1, 4096), dtype=torch.float16))  # routable but on the CPU
    assert y.shape == (1, 4096) and patch.fallbacks == {"device-cpu": 1} and patch.calls == 0
    patch.uninstall()
    assert model[0] is a and model[2][0] is b
    Patch(model, mode="stock").uninstall()


def _cache_from(k_raw, v_raw, bits, max_len):
    """A CPU cache filled by the oracle's canonical quantizer."""
    hkv, t, dh = k_raw.shape
    cache = QuantizedKVCache(hkv, dh, bits, max_len, device="cpu")
    for dst, raw in ((cache.keys, k_raw), (cache.values, v_raw)):
        art = canonical_quantize(raw.reshape(-1, dh), QuantContract(bits=bits, group_size=64))
        dst[0][0, :, :t] = torch.from_numpy(pack_codes(art.q, bits).view(np.int32)
                                            .reshape(hkv, t, -1).copy())
        dst[1][0, :, :t] = torch.from_numpy(art.scales.reshape(hkv, t, -1).copy())
        dst[2][0, :, :t] = torch.from_numpy(art.biases.reshape(hkv, t, -1).copy())
    cache.offset = t
    return cache


def test_kv_refusals_and_the_stock_step_against_the_oracle():
    rng = np.random.default_rng(3)
    h, hkv, t, dh, bits = 8, 2, 40, 64, 4
    k_raw = rng.standard_normal((hkv, t, dh)).astype(np.float16)
    v_raw = rng.standard_normal((hkv, t, dh)).astype(np.float16)
    q = (rng.standard_normal((1, h, dh)) * 0.3).astype(np.float16)
    nk = (rng.standard_normal((1, hkv, dh)) * 0.3).astype(np.float16)
    nv = rng.standard_normal((1, hkv, dh)).astype(np.float16)
    cache = _cache_from(k_raw, v_raw, bits, max_len=64)
    scale = 1 / math.sqrt(dh)
    qt = torch.from_numpy(q).reshape(1, h, 1, dh)
    door = KvDoor()
    assert door.ineligible(qt, cache, scale) == "device-cpu"
    assert door.ineligible(qt.float(), cache, scale) == "dtype-torch.float32"
    assert door.ineligible(qt.expand(1, h, 3, dh), cache, scale) == "prefill-L3"
    assert door.ineligible(qt, object(), scale) == "cache-not-quantized"
    assert door.ineligible(qt.expand(2, h, 1, dh), cache, scale) == "batch-B2"
    assert door.ineligible(qt, cache, 0.5) == "nonstandard-scale"
    assert door.ineligible(qt, cache, scale, mask=torch.ones(1)) == "mask-array"
    assert door.ineligible(qt[:, :6], cache, scale) == "gqa-6/2"
    out = door(qt, cache, torch.from_numpy(nk).reshape(1, hkv, 1, dh),
               torch.from_numpy(nv).reshape(1, hkv, 1, dh), scale)
    assert door.fallbacks == {"device-cpu": 1} and door.calls == 0
    ref = kv_reference_gqa(q, k_raw, v_raw, nk, nv, bits)
    err = np.max(np.abs(out.reshape(1, h, dh).numpy().astype(np.float64) - ref))
    assert err <= 4 * 9.77e-4 * np.max(np.abs(ref))


def test_cpu_cache_refuses_append_and_shapes_are_checked():
    """append quantizes with the GPU library: a CPU cache refuses it before
    any call, and mis-shaped entries are named."""
    cache = QuantizedKVCache(2, 64, 4, 16, device="cpu")
    k = torch.zeros((1, 2, 3, 64))
    with pytest.raises(ValueError, match="on the GPU"):
        cache.append(k, k)
    assert cache.offset == 0
