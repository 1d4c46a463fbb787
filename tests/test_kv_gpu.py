"""kvp_kv_decode on the GPU against the CPU oracle's ``kv_reference`` + ensemble floor.

Mirrors the reference's kernel tests (tests/test_pack_kv_attention.py:70-239)
case for case, with the capacity tests turned around (T > 1024 now runs), and
adds BASELINE configs 3 and 4: GQA 32/8 at T = 8192 (8-bit) and a batch of
eight per-sequence caches with lengths drawn from U[1024, 32768] (4-bit).

Cache artefacts come from the oracle's canonical quantizer (test side) and
the product's packer. GQA and per-sequence cases are judged through the
oracle's tiled-cache and one-sequence-at-a-time forms
(oracle/extensions.py), which the reference's own tests establish as exact
(tests/test_pack_kv_attention.py:120-130, :176-205).
"""

import numpy as np
import pytest

from kernelverify_amd.pack import kv_attention
from oracle.extensions import kv_gqa_inputs, kv_per_sequence
from oracle.inputs import kv_case
from oracle.native_ops import kv_reference, kv_tolerance
from oracle.quant_contract import QuantContract, canonical_quantize
from oracle.verify import _Case, judge, kv_inputs, verify_output

pytestmark = pytest.mark.gpu


def quantize_cache(cache: np.ndarray, bits: int):
    """(..., T, DH) raw cache -> kernel-layout (codes, scales, biases)."""
    dh = cache.shape[-1]
    art = canonical_quantize(cache.reshape(-1, dh), QuantContract(bits=bits, group_size=64))
    return kv_attention.pack_cache(art.q.reshape(cache.shape), art.scales, art.biases, bits)


def run(q, kc, vc, nk, nv, bits, dtype="float16", t=None, pad_to=None, chunk=0):
    """Reference layout: one (HKV, T, DH) cache shared by every batch row."""
    t = kc.shape[1] if t is None else t
    k = quantize_cache(kc, bits)
    v = quantize_cache(vc, bits)
    if pad_to is not None and pad_to > kc.shape[1]:
        rng = np.random.default_rng(99)

        def padded(parts):
            junk = rng.standard_normal((kc.shape[0], pad_to - kc.shape[1], kc.shape[2]))
            jparts = quantize_cache(junk.astype(np.float16), bits)
            return [np.concatenate([a, j], axis=1) for a, j in zip(parts, jparts)]

        k, v = padded(k), padded(v)
    lengths = np.full(q.shape[0], t, dtype=np.int32)
    return kv_attention.kv_decode(q, *k, *v, nk, nv, lengths, bits=bits, out_dtype=dtype,
                                  chunk=chunk)


@pytest.mark.parametrize("shape", [(1, 8, 512, 128), (4, 2, 64, 64), (1, 4, 300, 128)])
@pytest.mark.parametrize("bits", [4, 8])
def test_agrees_with_the_shipped_reference(shape, bits):
    b, h, t, dh = shape
    q, kc, vc, nk, nv = kv_case(b, h, t, dh, seed=t + bits)
    out = run(q, kc, vc, nk, nv, bits)
    v = verify_output("kv_attention", kv_inputs(q, kc, vc, nk, nv, bits), out)
    assert v.ok, v


@pytest.mark.parametrize("bits", [4, 8])
def test_float32_dtype(bits):
    """fp32 output: base tolerance ~4e-7 * scale, the strict test of fp32
    arithmetic everywhere (split partials and combine included)."""
    q, kc, vc, nk, nv = kv_case(2, 4, 256, 128, seed=17 + bits, dtype="float32")
    q, nk, nv = (a.astype(np.float16) for a in (q, nk, nv))
    kc, vc = kc.astype(np.float16), vc.astype(np.float16)
    out = run(q, kc, vc, nk, nv, bits, "float32")
    v = verify_output("kv_attention", kv_inputs(q, kc, vc, nk, nv, bits), out, dtype="float32")
    assert v.ok, v


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
@pytest.mark.parametrize("dh", [64, 128])
def test_every_supported_width(bits, dh):
    q, kc, vc, nk, nv = kv_case(1, 4, 128, dh, seed=40 + bits)
    out = run(q, kc, vc, nk, nv, bits)
    v = verify_output("kv_attention", kv_inputs(q, kc, vc, nk, nv, bits), out)
    assert v.ok, v


def test_new_entry_dominates_when_it_should():
    b, h, t, dh = 2, 4, 128, 64
    q, kc, vc, _, nv = kv_case(b, h, t, dh, seed=5)
    new_k = (q.astype(np.float32) * 60.0).astype(np.float16)
    out = run(q, kc, vc, new_k, nv, 8)
    v = verify_output("kv_attention", kv_inputs(q, kc, vc, new_k, nv, 8), out)
    assert v.ok, v
    assert float(np.max(np.abs(out - nv.astype(np.float64)))) < 0.05


def test_batch_rows_are_independent():
    """Each batch row reproduces its own B=1 answer bit for bit."""
    b, h, t, dh = 4, 2, 96, 64
    q, kc, vc, nk, nv = kv_case(b, h, t, dh, seed=11)
    full = run(q, kc, vc, nk, nv, 4)
    for row in range(b):
        one = run(q[row:row + 1], kc, vc, nk[row:row + 1], nv[row:row + 1], 4)
        assert np.array_equal(full[row:row + 1], one)


@pytest.mark.parametrize("t", [1, 63, 64, 65])
def test_short_caches(t):
    q, kc, vc, nk, nv = kv_case(1, 2, t, 64, seed=3 + t)
    out = run(q, kc, vc, nk, nv, 4)
    v = verify_output("kv_attention", kv_inputs(q, kc, vc, nk, nv, 4), out)
    assert v.ok, v


def test_empty_cache_returns_new_v():
    """T = 0: the softmax has one term, the new entry, so out == new_v."""
    q, kc, vc, nk, nv = kv_case(2, 2, 8, 64, seed=4)
    out = run(q, kc, vc, nk, nv, 4, "float32", t=0)
    assert np.array_equal(out, nv.astype(np.float32))


def test_padded_cache_reads_only_the_logical_prefix():
    b, h, t, t_pad, dh, bits = 1, 4, 300, 512, 128, 8
    q, kc, vc, nk, nv = kv_case(b, h, t, dh, seed=23)
    out = run(q, kc, vc, nk, nv, bits, pad_to=t_pad)
    v = verify_output("kv_attention", kv_inputs(q, kc, vc, nk, nv, bits), out)
    assert v.ok, v


def test_gqa_matches_the_tiled_cache_reference():
    b, h, hkv, t, dh, bits = 1, 8, 2, 128, 64, 8
    q, kc_full, vc_full, nk_full, nv_full = kv_case(b, h, t, dh, seed=31)
    kc, vc = kc_full[:hkv], vc_full[:hkv]
    nk, nv = nk_full[:, :hkv], nv_full[:, :hkv]
    out = run(q, kc, vc, nk, nv, bits)
    v = verify_output("kv_attention", kv_gqa_inputs(q, kc, vc, nk, nv, bits), out)
    assert v.ok, v


@pytest.mark.parametrize("t,chunk", [(1025, 0), (4096, 0), (3000, 64), (3000, 128)])
def test_past_the_reference_capacity(t, chunk):
    """The reference refuses T > 1024 (kv_attention.py:77); the split kernel
    runs it, at the library's chunk and at forced small and large chunks."""
    q, kc, vc, nk, nv = kv_case(1, 4, t, 128, seed=t)
    out = run(q, kc, vc, nk, nv, 4, chunk=chunk)
    v = verify_output("kv_attention", kv_inputs(q, kc, vc, nk, nv, 4), out)
    assert v.ok, v


def test_chunking_is_exact_to_rounding():
    """Different chunk sizes are different association orders of the same
    online softmax (contract clause C3): fp32 outputs agree to rounding."""
    q, kc, vc, nk, nv = kv_case(1, 8, 2048, 128, seed=77)
    a = run(q, kc, vc, nk, nv, 4, "float32", chunk=64)
    b = run(q, kc, vc, nk, nv, 4, "float32", chunk=128)
    assert np.max(np.abs(a - b)) <= 1e-5 * np.max(np.abs(a))


def baseline_cache(rng, b, hkv, t, dh):
    k = rng.standard_normal((b, hkv, t, dh)).astype(np.float16)
    v = rng.standard_normal((b, hkv, t, dh)).astype(np.float16)
    return k, v


def test_config3_gqa_32_8_context_8192_8bit():
    """B1, 32 query heads over 8 KV heads, DH 128, T 8192,
    8-bit K/V fitted per 64-group to K, V ~ N(0, 1); fp16 Q ~ N(0, 1)."""
    rng = np.random.default_rng(3)
    b, h, hkv, t, dh, bits = 1, 32, 8, 8192, 128, 8
    kc, vc = baseline_cache(rng, b, hkv, t, dh)
    q = rng.standard_normal((b, h, dh)).astype(np.float16)
    nk = rng.standard_normal((b, hkv, dh)).astype(np.float16)
    nv = rng.standard_normal((b, hkv, dh)).astype(np.float16)
    out = run(q, kc[0], vc[0], nk, nv, bits)
    ref, tols = kv_per_sequence(q, kc, vc, nk, nv, [t], bits)
    v = judge(out, ref, max(tols))
    print("cfg3", v)
    assert v.ok, v


def test_config4_stress_per_sequence_lengths_4bit():
    """eight sequences, lengths ~ U[1024, 32768] (seed 0:
    28027, 21244, 17250, 9588, 10796, 2324, 3412, 1548), 4-bit per-sequence
    caches padded to 32768, GQA 32/8, DH 128. Judged per sequence."""
    lengths = np.random.default_rng(0).integers(1024, 32769, 8)
    assert list(lengths) == [28027, 21244, 17250, 9588, 10796, 2324, 3412, 1548]
    rng = np.random.default_rng(4)
    b, h, hkv, t_stride, dh, bits = 8, 32, 8, 32768, 128, 4
    kc, vc = baseline_cache(rng, b, hkv, t_stride, dh)
    q = rng.standard_normal((b, h, dh)).astype(np.float16)
    nk = rng.standard_normal((b, hkv, dh)).astype(np.float16)
    nv = rng.standard_normal((b, hkv, dh)).astype(np.float16)
    k = quantize_cache(kc, bits)
    v = quantize_cache(vc, bits)
    out = kv_attention.kv_decode(q, *k, *v, nk, nv, lengths.astype(np.int32), bits=bits,
                                 cache_per_sequence=True)
    # Judge three sequences in full (longest, a middle one, shortest); every
    # sequence is independent (batch-row independence above).
    for i in (0, 4, 7):
        ref, tols = kv_per_sequence(q[i:i + 1], [kc[i]], [vc[i]], nk[i:i + 1], nv[i:i + 1],
                                    [int(lengths[i])], bits)
        v = judge(out[i:i + 1], ref, tols[0])
        print("cfg4 seq", i, int(lengths[i]), v)
        assert v.ok, (i, v)
    assert np.isfinite(out.astype(np.float32)).all()


def test_lengths_past_t_stride_are_clamped_not_read():
    """A length beyond the allocation is clamped to t_stride in the kernel:
    the answer equals the full-cache answer, and nothing past it is read."""
    q, kc, vc, nk, nv = kv_case(1, 2, 256, 64, seed=8)
    full = run(q, kc, vc, nk, nv, 4, "float32")
    over = run(q, kc, vc, nk, nv, 4, "float32", t=10_000)
    assert np.array_equal(full, over)


def test_repeated_steps_reuse_the_workspace():
    """Ten steps through one KvDecodeCall (one workspace) give ten identical
    answers: nothing carries over from one step to the next."""
    from kernelverify_amd import hip
    from kernelverify_amd.hip import DeviceArray

    q, kc, vc, nk, nv = kv_case(2, 8, 700, 128, seed=12)
    k, v = quantize_cache(kc, 4), quantize_cache(vc, 4)
    dev = [DeviceArray.from_host(np.ascontiguousarray(a)) for a in (q, *k, *v, nk, nv)]
    lengths = DeviceArray.from_host(np.array([700, 333], dtype=np.int32))
    out = DeviceArray(q.shape, "float32")
    call = kv_attention.KvDecodeCall(*dev, lengths, out, bits=4)
    first = None
    for _ in range(10):
        call()
        hip.synchronize()
        got = out.to_host()
        if first is None:
            first = got
        assert np.array_equal(got, first)
    assert np.isfinite(first).all()


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("dh", [64, 128])
@pytest.mark.parametrize("g", [1, 2, 4, 8])
def test_every_query_group_size(bits, dh, g):
    """G = H / HKV query heads per KV head, 1 .. 8, on a ragged length (777,
    not a multiple of the 32-position step), fp32 output."""
    hkv = 2
    rng = np.random.default_rng(100 * g + dh + bits)
    q = rng.standard_normal((1, g * hkv, dh)).astype(np.float16)
    kc = rng.standard_normal((hkv, 777, dh)).astype(np.float16)
    vc = rng.standard_normal((hkv, 777, dh)).astype(np.float16)
    nk = rng.standard_normal((1, hkv, dh)).astype(np.float16)
    nv = rng.standard_normal((1, hkv, dh)).astype(np.float16)
    out = run(q, kc, vc, nk, nv, bits, "float32")
    v = verify_output("kv_attention", kv_gqa_inputs(q, kc, vc, nk, nv, bits), out,
                      dtype="float32")
    assert v.ok, (bits, dh, g, v)


def ranged_case(rng, g, hkv, t, dh, growth):
    """V rows scaled by ``growth`` (per position) and K rows that lean on the
    mean query by -ln(growth), so that p_t * |v_t| stays level along t and
    every magnitude band matters to the output."""
    q = rng.standard_normal((1, g * hkv, dh)).astype(np.float16)
    qbar = q[0].astype(np.float64).reshape(hkv, g, dh).mean(axis=1)
    beta = -np.log(growth)[None, :] * np.sqrt(dh) / (qbar ** 2).sum(-1, keepdims=True)
    kc = (beta[..., None] * qbar[:, None, :]
          + 0.3 * rng.standard_normal((hkv, t, dh))).astype(np.float16)
    vc = (rng.standard_normal((hkv, t, dh)) * growth[None, :, None]).astype(np.float16)
    nk = (0.1 * rng.standard_normal((1, hkv, dh))).astype(np.float16)
    nv = rng.standard_normal((1, hkv, dh)).astype(np.float16)
    return q, kc, vc, nk, nv


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("profile", ["rising", "falling", "zero_band"])
@pytest.mark.parametrize("dh,g", [(128, 4), (64, 8)])
def test_value_scales_across_many_octaves(bits, profile, dh, g):
    """V scales spanning 2^16 along the cache: the matrix-core value path
    carries p * s under a per-group power-of-two range shift that must drop
    when a larger scale arrives (rising), hold precision for small scales
    after large ones (falling), and survive all-zero groups (zero_band)."""
    t = 1500
    rng = np.random.default_rng({"rising": 1, "falling": 2, "zero_band": 3}[profile] + bits)
    growth = 2.0 ** (np.arange(t) * 16.0 / t - 8.0)
    if profile == "falling":
        growth = growth[::-1].copy()
    q, kc, vc, nk, nv = ranged_case(rng, g, 1, t, dh, growth)
    if profile == "zero_band":
        vc[:, t // 3:t // 2] = 0
    for chunk in (0, 64):
        out = run(q, kc, vc, nk, nv, bits, "float32", chunk=chunk)
        v = verify_output("kv_attention", kv_gqa_inputs(q, kc, vc, nk, nv, bits), out,
                          dtype="float32")
        assert v.ok, (bits, profile, dh, g, chunk, v)


def test_all_zero_values():
    """V = 0 everywhere in the cache: the output is p_new * new_v / L."""
    rng = np.random.default_rng(9)
    q = rng.standard_normal((1, 8, 128)).astype(np.float16)
    kc = rng.standard_normal((2, 600, 128)).astype(np.float16)
    vc = np.zeros((2, 600, 128), dtype=np.float16)
    nk = rng.standard_normal((1, 2, 128)).astype(np.float16)
    nv = rng.standard_normal((1, 2, 128)).astype(np.float16)
    out = run(q, kc, vc, nk, nv, 4, "float32")
    v = verify_output("kv_attention", kv_gqa_inputs(q, kc, vc, nk, nv, 4), out, dtype="float32")
    assert v.ok, v


def test_one_workspace_serves_calls_of_every_shape():
    """One workspace serves calls of different shapes in turn (an empty
    sequence among them): nothing one call leaves in it changes the next,
    and each output passes the oracle."""
    from kernelverify_amd import hip
    from kernelverify_amd.hip import DeviceArray

    ws = DeviceArray((8 << 20,), np.uint8)
    ws.fill_byte(0x7F)
    cases = [(1, 32, 8, 5000, 4, [5000]), (3, 8, 2, 2600, 8, [100, 0, 2600]),
             (2, 16, 2, 3000, 4, [3000, 1])]
    for b, h, hkv, t_stride, bits, lengths in cases:
        rng = np.random.default_rng(b * 100 + h)
        q = (rng.standard_normal((b, h, 128)) * 0.3).astype(np.float16)
        kc = rng.standard_normal((b, hkv, t_stride, 128)).astype(np.float16)
        vc = rng.standard_normal((b, hkv, t_stride, 128)).astype(np.float16)
        nk = (rng.standard_normal((b, hkv, 128)) * 0.3).astype(np.float16)
        nv = rng.standard_normal((b, hkv, 128)).astype(np.float16)
        dev = [DeviceArray.from_host(np.ascontiguousarray(a)) for a in
               (q, *quantize_cache(kc, bits), *quantize_cache(vc, bits), nk, nv)]
        t_dev = DeviceArray.from_host(np.array(lengths, dtype=np.int32))
        out = DeviceArray((b, h, 128), "float32")
        kv_attention.KvDecodeCall(*dev, t_dev, out, bits=bits, cache_per_sequence=True,
                                  workspace=ws)()
        hip.synchronize()
        got = out.to_host()
        for i, t in enumerate(lengths):
            if t == 0:  # the softmax has one term: out = new_v of the head's KV head
                want = np.repeat(nv[i].astype(np.float32), h // hkv, axis=0)
                assert np.max(np.abs(got[i] - want)) <= 1e-6 * np.max(np.abs(want))
                continue
            ref, tols = kv_per_sequence(q[i:i + 1], kc[i:i + 1], vc[i:i + 1], nk[i:i + 1],
                                        nv[i:i + 1], [t], bits, dtype="float32")
            v = judge(got[i:i + 1], ref, tols[0])
            assert v.ok, (b, h, bits, i, v)


def test_32k_target_shape_4bit():
    """The 32k target: B1, 32 query heads over 8 KV heads, DH 128, 4-bit K/V
    over T = 32768 cached positions, judged in full against the oracle."""
    rng = np.random.default_rng(32)
    b, h, hkv, t, dh, bits = 1, 32, 8, 32768, 128, 4
    kc, vc = baseline_cache(rng, b, hkv, t, dh)
    q = rng.standard_normal((b, h, dh)).astype(np.float16)
    nk = rng.standard_normal((b, hkv, dh)).astype(np.float16)
    nv = rng.standard_normal((b, hkv, dh)).astype(np.float16)
    out = run(q, kc[0], vc[0], nk, nv, bits)
    ref, tols = kv_per_sequence(q, kc, vc, nk, nv, [t], bits)
    v = judge(out, ref, max(tols))
    print("32k", v)
    assert v.ok, v
