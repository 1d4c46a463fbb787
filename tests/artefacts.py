"""Seeded synthetic artefacts of the BASELINE configurations.

Config 1/2 (qmv): codes q ~ U{0 .. 2^bits - 1}, fp16 scales ~ |N(0, 0.02)|,
fp16 biases ~ N(0, 0.01) per 64-code group, fp16 x ~ N(0, 1). The artefact is
drawn directly (it is not the quantization of some W), so the oracle judges it
through ``r_contract`` on the artefact (``oracle.extensions.artefact_from_arrays``).
"""

from __future__ import annotations

import numpy as np


def draw_qmv(d_out: int, d_in: int, bits: int, m: int, seed: int):
    """(x fp16 (m, d_in), q int32 (d_out, d_in), scales fp16, biases fp16)."""
    rng = np.random.default_rng(seed)
    q = rng.integers(0, 1 << bits, size=(d_out, d_in), dtype=np.int32)
    g = d_in // 64
    scales = np.abs(rng.standard_normal((d_out, g)) * 0.02).astype(np.float16)
    biases = (rng.standard_normal((d_out, g)) * 0.01).astype(np.float16)
    x = rng.standard_normal((m, d_in)).astype(np.float16)
    return x, q, scales, biases
