"""The serving door on the GPU: routed linear calls run kvp_qmv (bit-identical
to the pack API, every rank spelling of the same rows identical, ADR 0018),
refused calls run the stock path and are counted, and the KV door's decode
step over a cache whose logical length is below its padded stride matches
the oracle."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
from torch import nn

from kernelverify_amd.pack import wide_qmv
from kernelverify_amd.serving import KvDoor, Patch, QuantizedKVCache, QuantizedLinear
from oracle.extensions import kv_reference_gqa
from oracle.quant_contract import QuantContract, canonical_quantize, pack_codes

pytestmark = pytest.mark.gpu


def _layer(d_out, d_in, bits, seed=0):
    w = (np.random.default_rng(seed).standard_normal((d_out, d_in)) * 0.02).astype(np.float16)
    art = canonical_quantize(w, QuantContract(bits=bits, group_size=64))
    words = pack_codes(art.q, bits)
    layer = QuantizedLinear(torch.from_numpy(words.view(np.int32).copy()).cuda(),
                            torch.from_numpy(art.scales.copy()).cuda(),
                            torch.from_numpy(art.biases.copy()).cuda(), bits)
    return layer, words, art


def test_routed_calls_are_the_kernel_at_every_rank():
    layer, words, art = _layer(4096, 4096, 4)
    model = nn.Sequential(layer)
    patch = Patch(model)
    ms = [m for m in range(1, 17) if wide_qmv.should_dispatch(m, 4, 4096, 4096)]
    m = max(ms)
    x = (np.random.default_rng(1).standard_normal((m, 4096))).astype(np.float16)
    want = wide_qmv.qmv(x, words, art.scales, art.biases, bits=4)
    xt = torch.from_numpy(x).cuda()
    outs = [model(xt), model(xt.reshape(1, m, 4096)), model(xt.reshape(m, 1, 4096))]
    torch.cuda.synchronize()
    for out in outs:
        assert np.array_equal(out.reshape(m, 4096).cpu().numpy(), want)
    assert patch.calls == 3 and not patch.fallbacks
    # a width the table does not route runs the stock path, named
    x_out = torch.zeros((17, 4096), dtype=torch.float16, device="cuda")
    stock = layer(x_out)
    assert torch.equal(model(x_out), stock)
    assert patch.fallbacks == {"m-17-outside-dispatch-4096x4096": 1}
    patch.uninstall()
    forced = Patch(model, mode="stock")
    model(xt)
    assert forced.calls == 0 and forced.fallbacks == {"forced-stock": 1}


@pytest.mark.parametrize("bits, dh, gqa", [(4, 128, 4), (8, 64, 2)])
def test_kv_door_reads_the_logical_length_not_the_stride(bits, dh, gqa):
    rng = np.random.default_rng(bits)
    hkv, t, stride = 2, 100, 256
    h = hkv * gqa
    k_raw = rng.standard_normal((hkv, t, dh)).astype(np.float16)
    v_raw = rng.standard_normal((hkv, t, dh)).astype(np.float16)
    q = (rng.standard_normal((1, h, dh)) * 0.3).astype(np.float16)
    nk = (rng.standard_normal((1, hkv, dh)) * 0.3).astype(np.float16)
    nv = rng.standard_normal((1, hkv, dh)).astype(np.float16)
    cache = QuantizedKVCache(hkv, dh, bits, stride)
    # the padding past the logical length holds garbage the kernel must not read
    for part in (*cache.keys, *cache.values):
        part[0, :, t:] = 7 if part.dtype == torch.int32 else 1000.0
    cache.append(torch.from_numpy(k_raw[None, :, :60]).cuda(),
                 torch.from_numpy(v_raw[None, :, :60]).cuda())
    # entries given on the host move to the cache's device; an empty append is a no-op
    cache.append(torch.from_numpy(k_raw[None, :, 60:]), torch.from_numpy(v_raw[None, :, 60:]))
    cache.append(torch.zeros((1, hkv, 0, dh)), torch.zeros((1, hkv, 0, dh)))
    assert cache.offset == t
    art = canonical_quantize(k_raw.reshape(-1, dh), QuantContract(bits=bits, group_size=64))
    assert np.array_equal(cache.keys[0][0, :, :t].cpu().numpy().view(np.uint32).reshape(-1, dh * bits // 32),
                          pack_codes(art.q, bits))
    door = KvDoor()
    scale = 1 / math.sqrt(dh)
    qd = torch.from_numpy(q).cuda().reshape(1, h, 1, dh)
    host_cache = QuantizedKVCache(hkv, dh, bits, stride, device="cpu")
    assert door.ineligible(qd, host_cache, scale) == "cache-device-cpu"
    # the step's own entry may come from the host: it moves to the queries' device
    out = door(qd, cache, torch.from_numpy(nk).reshape(1, hkv, 1, dh),
               torch.from_numpy(nv).reshape(1, hkv, 1, dh), scale)
    torch.cuda.synchronize()
    assert door.calls == 1 and not door.fallbacks
    ref = kv_reference_gqa(q, k_raw, v_raw, nk, nv, bits)
    err = np.max(np.abs(out.reshape(1, h, dh).cpu().numpy().astype(np.float64) - ref))
    assert err <= 4 * 9.77e-4 * np.max(np.abs(ref)), err


def test_a_loaded_checkpoint_serves_through_the_patch(tmp_path):
    """MLX-affine safetensors straight to the device and through the routed
    linear: the same output as the pack API on the file's own bytes."""
    from kernelverify_amd.checkpoint import load_quantized_linears, save_quantized_linears

    _, words, art = _layer(4096, 4096, 4, seed=5)
    save_quantized_linears(tmp_path / "model.safetensors",
                           {"mlp.up_proj": (words, art.scales, art.biases)}, bits=4)
    layers = load_quantized_linears(tmp_path)
    model = nn.Sequential(layers["mlp.up_proj"])
    patch = Patch(model)
    x = np.random.default_rng(6).standard_normal((1, 4096)).astype(np.float16)
    got = model(torch.from_numpy(x).cuda())
    torch.cuda.synchronize()
    assert patch.calls == 1
    assert np.array_equal(got.cpu().numpy(), wide_qmv.qmv(x, words, art.scales, art.biases, bits=4))
