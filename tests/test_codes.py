"""The product's code-stream packer against the oracle's independent one.

``oracle.quant_contract.pack_codes`` is an explicit bit scatter (bit planes
through ``np.packbits``); the product's packer ORs codes by in-word offset.
Both must produce the MLX layout: code i at bits [i*bits, (i+1)*bits) of a
little-endian row stream (kernelverify/pack/wide_qmv.py:185-201).
"""

import numpy as np
import pytest

from kernelverify_amd.pack.codes import pack_codes, unpack_codes
from oracle.quant_contract import pack_codes as oracle_pack, unpack_codes as oracle_unpack


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
def test_packer_matches_oracle(bits):
    rng = np.random.default_rng(bits)
    q = rng.integers(0, 1 << bits, size=(7, 256), dtype=np.int32)
    got = pack_codes(q, bits)
    assert got.dtype == np.uint32 and got.shape == (7, 256 * bits // 32)
    assert np.array_equal(got, oracle_pack(q, bits))
    assert np.array_equal(unpack_codes(got, 256, bits), q)
    assert np.array_equal(oracle_unpack(got, 256, bits), q)


def test_four_bit_known_answer():
    """Word j, nibble k holds code 8j + k."""
    q = (np.arange(16) % 16).reshape(1, 16)
    words = pack_codes(q, 4)
    assert [hex(w) for w in words[0]] == ["0x76543210", "0xfedcba98"]


def test_eight_bit_byte_order():
    q = np.array([[1, 2, 3, 4]])
    assert pack_codes(q, 8)[0, 0] == 0x04030201


def test_three_bit_straddles_words():
    q = np.zeros((1, 32), dtype=np.int32)
    q[0, 10] = 7  # bits 30..32: two bits in word 0, one in word 1
    words = pack_codes(q, 3)
    assert words[0, 0] == 0xC0000000 and words[0, 1] == 0x1 and words[0, 2] == 0


def test_rejects_out_of_range_codes():
    with pytest.raises(ValueError):
        pack_codes(np.array([[16] * 8]), 4)
