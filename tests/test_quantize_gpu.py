"""kvp_quantize_affine against the oracle's canonical quantizer + packer, bit for bit.

The oracle quantizer is pinned to the reference's committed calibration
records (tests/test_oracle_golden.py); this pins the GPU one to it: every
code word, every fp16 scale and bias, at every width, on the calibration
draws plus the groups that exercise each branch of the algorithm (all
negative, all zero, constant, the q0 = 0 snap, exact half-way codes).
"""

import numpy as np
import pytest

from kernelverify_amd.pack.quant import quantize
from oracle.inputs import make_w
from oracle.quant_contract import QuantContract, canonical_quantize, pack_codes

pytestmark = pytest.mark.gpu


def oracle(w, bits):
    art = canonical_quantize(w, QuantContract(bits=bits, group_size=64))
    return pack_codes(art.q, bits), art.scales, art.biases


def assert_same(w, bits):
    got = quantize(w, bits)
    want = oracle(w, bits)
    for name, g, e in zip(("codes", "scales", "biases"), got, want):
        assert g.shape == e.shape, name
        assert np.array_equal(g.view(np.uint16 if g.dtype == np.float16 else g.dtype),
                              e.view(np.uint16 if e.dtype == np.float16 else e.dtype)), name


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
@pytest.mark.parametrize("draw", ["normal-0.02", "heavy-tailed"])
def test_calibration_draws(bits, draw):
    w = make_w(512, 1024, draw, np.random.default_rng(10_000 + bits))
    assert_same(w, bits)


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
def test_branch_cases(bits):
    rng = np.random.default_rng(bits)
    rows = [
        -np.abs(rng.standard_normal(64)),              # all negative: max clamps to 0
        np.zeros(64),                                  # all zero: step floor 1e-7
        np.full(64, 0.37),                             # constant positive
        np.full(64, -2.5),                             # constant negative
        np.r_[np.full(63, 0.0), [-1e-6]],              # q0 rounds to 0: bias 0
        np.linspace(-1.0, 1.0, 64),                    # ties at exact half steps
        rng.standard_normal(64) * 1e-3,                # tiny
        rng.standard_normal(64) * 300.0,               # large
    ]
    w = np.stack(rows).astype(np.float16)
    assert_same(w, bits)


def test_kv_cache_shape():
    """quantize_cache of an (HKV, T, DH) cache: rows per position, layout (HKV, T, .)."""
    rng = np.random.default_rng(0)
    cache = rng.standard_normal((4, 100, 128)).astype(np.float16)
    codes, s, b = quantize(cache, 4)
    assert codes.shape == (4, 100, 16) and s.shape == (4, 100, 2)
    want = oracle(cache.reshape(-1, 128), 4)
    assert np.array_equal(codes.reshape(-1, 16), want[0])
