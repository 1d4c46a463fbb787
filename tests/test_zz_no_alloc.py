"""kvp_kv_decode_static, the allocation-free entry point, against kvp_kv_decode.

Both run the same kernels with the same chunk, so the outputs must be
bit-identical. Two calls in a row, the second on a smaller input, show that
what the first call left in the shared static scratch does not leak into the
second. The smaller case is also judged against the CPU oracle.
"""

import ctypes

import numpy as np
import pytest

from kernelverify_amd import hip, lib
from kernelverify_amd.hip import DeviceArray
from kernelverify_amd.pack import kv_attention
from oracle.extensions import kv_per_sequence
from oracle.quant_contract import QuantContract, canonical_quantize
from oracle.verify import judge

pytestmark = pytest.mark.gpu


def _packed(cache, bits):
    dh = cache.shape[-1]
    art = canonical_quantize(cache.reshape(-1, dh), QuantContract(bits=bits, group_size=64))
    return kv_attention.pack_cache(art.q.reshape(cache.shape), art.scales, art.biases, bits)


def _case(seed, b, h, hkv, dh, lengths, t_stride, bits):
    rng = np.random.default_rng(seed)
    q = (rng.standard_normal((b, h, dh)) * 0.3).astype(np.float16)
    kc = rng.standard_normal((b, hkv, t_stride, dh)).astype(np.float16)
    vc = rng.standard_normal((b, hkv, t_stride, dh)).astype(np.float16)
    nk = (rng.standard_normal((b, hkv, dh)) * 0.3).astype(np.float16)
    nv = rng.standard_normal((b, hkv, dh)).astype(np.float16)
    return q, kc, vc, nk, nv, np.asarray(lengths, dtype=np.int32)


def _both(case, bits, chunk=0):
    """Outputs of kvp_kv_decode (caller workspace) and kvp_kv_decode_static
    on the same device inputs, per-sequence caches, fp32 out."""
    q, kc, vc, nk, nv, lengths = case
    b, h, dh = q.shape
    hkv, t_stride = kc.shape[1], kc.shape[2]
    dev = [DeviceArray.from_host(np.ascontiguousarray(a)) for a in
           (q, *_packed(kc, bits), *_packed(vc, bits), nk, nv, lengths)]
    cdll = lib.load()
    if chunk == 0:
        _, _, chunk = kv_attention.launch_config(b, hkv, t_stride, bits, None, gqa=h // hkv)
    need = int(cdll.kvp_kv_decode_workspace_bytes(b, h, dh, t_stride, chunk))
    ws = DeviceArray((need,), np.uint8)
    ws.fill_byte(0x7F)  # garbage in the caller's workspace must not matter either
    outs = []
    for static in (False, True):
        out = DeviceArray((b, h, dh), np.float32)
        out.fill_byte(0xFF)
        args = [d.ptr for d in dev] + [out.ptr, lib.KVP_F32, b, h, hkv, dh, t_stride, bits, 1,
                                       chunk]
        if static:
            rc = cdll.kvp_kv_decode_static(*args, None)
        else:
            rc = cdll.kvp_kv_decode(*args, ws.ptr, need, None)
        lib.check(rc)
        hip.synchronize()
        outs.append(out.to_host())
    return outs


def test_static_entry_matches_the_workspace_entry_twice_in_a_row():
    print("no-alloc: call 1, B2 H32/8 DH128 T<=6000 4-bit", flush=True)
    big = _case(1, 2, 32, 8, 128, [6000, 4100], 6000, 4)
    a, b = _both(big, 4)
    assert np.array_equal(a, b)
    assert np.all(np.isfinite(b))

    print("no-alloc: call 2 (smaller), B1 H8/2 DH128 T=700 8-bit", flush=True)
    small = _case(2, 1, 8, 2, 128, [700], 768, 8)
    a2, b2 = _both(small, 8)
    assert np.array_equal(a2, b2)
    q, kc, vc, nk, nv, lengths = small
    ref, tols = kv_per_sequence(q, kc[:, :, :700], vc[:, :, :700], nk, nv, [700], 8,
                                dtype="float32")
    v = judge(b2, ref, tols[0])
    assert v.ok, v


def test_static_entry_refuses_a_call_beyond_its_scratch():
    cdll = lib.load()
    cap = int(cdll.kvp_kv_decode_static_scratch_bytes())
    assert cap == 4 << 20
    # 8 sequences x 32 heads x (32768 / 64 + 1) chunks of 130 floats: 68 MB
    null = ctypes.c_void_p(0)
    rc = cdll.kvp_kv_decode_static(*([null] * 11), lib.KVP_F16, 8, 32, 8, 128, 32768, 4, 1, 64,
                                   None)
    assert rc == lib.KVP_INVALID
    assert "static scratch" in lib.last_error()
