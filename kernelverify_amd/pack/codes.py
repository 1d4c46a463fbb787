"""The MLX affine code-stream layout every pack kernel reads.

Per row, a contiguous little-endian bit stream of ``bits``-wide codes viewed
as uint32 words: code i occupies bits [i*bits, (i+1)*bits) of the row's
stream (kernelverify/pack/wide_qmv.py:185-201, whose own docstring records it
bit-identical to ``mx.quantize`` at 2/3/4/5/6/8 bits).

This packer is vectorised by bit offset: all codes that start at the same
offset inside their word are OR-ed in one numpy step, and the bits that spill
past a word boundary are carried into the next word.
"""

from __future__ import annotations

import numpy as np


def pack_codes(q: np.ndarray, bits: int) -> np.ndarray:
    """(rows, cols) integer codes in [0, 2^bits) -> (rows, cols*bits/32) uint32."""
    q = np.asarray(q)
    if q.ndim != 2:
        raise ValueError(f"pack_codes expects a 2-D code matrix, got shape {q.shape}")
    rows, cols = q.shape
    if not 1 <= bits <= 16:
        raise ValueError(f"bits={bits} outside 1..16")
    if (cols * bits) % 32:
        raise ValueError(f"{cols} codes of {bits} bits do not fill whole 32-bit words")
    if q.size and (q.min() < 0 or q.max() >= (1 << bits)):
        raise ValueError(f"codes outside [0, {1 << bits})")
    n_words = cols * bits // 32
    acc = np.zeros((rows, n_words + 1), dtype=np.uint64)
    start = np.arange(cols, dtype=np.int64) * bits
    word, offset = start // 32, start % 32
    codes = q.astype(np.uint64)
    for off in np.unique(offset):
        cols_at = np.nonzero(offset == off)[0]
        acc[:, word[cols_at]] |= codes[:, cols_at] << np.uint64(off)
    low = acc[:, :n_words] & np.uint64(0xFFFFFFFF)
    carry = np.zeros_like(low)
    carry[:, 1:] = acc[:, :n_words - 1] >> np.uint64(32)
    return np.ascontiguousarray((low | carry).astype(np.uint32))


def pack_nibbles(q: np.ndarray) -> np.ndarray:
    """The 4-bit case (kernelverify/pack/wide_qmv.py:204-206)."""
    return pack_codes(q, 4)


def unpack_codes(words: np.ndarray, cols: int, bits: int) -> np.ndarray:
    """Inverse of ``pack_codes``: (rows, cols*bits/32) uint32 -> (rows, cols) int32."""
    words = np.ascontiguousarray(words, dtype=np.uint32)
    rows = words.shape[0]
    wide = np.zeros((rows, words.shape[1] + 1), dtype=np.uint64)
    wide[:, :-1] = words
    start = np.arange(cols, dtype=np.int64) * bits
    word, offset = start // 32, start % 32
    both = wide[:, word] | (wide[:, word + 1] << np.uint64(32))
    return ((both >> offset.astype(np.uint64)) & np.uint64((1 << bits) - 1)).astype(np.int32)
