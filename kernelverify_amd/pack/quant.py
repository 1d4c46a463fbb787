"""MLX-affine quantization on the GPU (``kvp_quantize_affine``).

The pack's artefact builder: fp16 rows -> packed code stream + fp16 scale and
bias per 64-value group, in the layout every pack kernel reads. Replaces the
reference's host path ``canonical_quantize`` + ``pack_codes``
(kernelverify/schemas/quant_contract.py:60-104, pack/wide_qmv.py:185-201),
with the same fp32 arithmetic, so artefacts are bit-identical.
"""

from __future__ import annotations

import numpy as np

from kernelverify_amd import lib
from kernelverify_amd.hip import DeviceArray

SUPPORTED_BITS = (2, 3, 4, 8)
GROUP = 64


def quantize_affine(w: DeviceArray, bits: int, stream=None):
    """Device fp16 (..., cols) -> (w_q uint32 (..., cols*bits/32), scales, biases)."""
    if w.dtype != np.float16 or len(w.shape) < 1:
        raise lib.InvalidArgument(f"quantize: w must be fp16, got {w.dtype}")
    if bits not in SUPPORTED_BITS:
        raise lib.Unsupported(f"quantize: bits={bits} not in {SUPPORTED_BITS}")
    cols = w.shape[-1]
    if cols % GROUP:
        raise lib.InvalidArgument(f"quantize: {cols} columns is not a multiple of {GROUP}")
    lead = w.shape[:-1]
    rows = int(np.prod(lead, dtype=np.int64)) if lead else 1
    wq = DeviceArray(lead + (cols * bits // 32,), np.uint32)
    sc = DeviceArray(lead + (cols // GROUP,), np.float16)
    bi = DeviceArray(lead + (cols // GROUP,), np.float16)
    lib.check(lib.load().kvp_quantize_affine(w.ptr, rows, cols, bits, wq.ptr, sc.ptr, bi.ptr,
                                             getattr(stream, "handle", stream)))
    return wq, sc, bi


def quantize(w: np.ndarray, bits: int):
    """Host convenience: (codes, scales, biases) as numpy arrays."""
    from kernelverify_amd import hip

    out = quantize_affine(DeviceArray.from_host(np.ascontiguousarray(w, dtype=np.float16)), bits)
    hip.synchronize()
    return tuple(a.to_host() for a in out)


def quantize_cache(cache: np.ndarray, bits: int):
    """(..., T, DH) fp16 cache -> kernel-layout (codes, scales, biases): each
    (position, head) row quantized on its own (kv_attention.py:270-283)."""
    return quantize(cache, bits)
