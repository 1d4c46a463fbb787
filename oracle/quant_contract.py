"""MLX-affine quantization contract, restated for the CPU oracle.

Follows vladmt06/kernelverify ``kernelverify/schemas/quant_contract.py``:

- ``canonical_quantize``   :60-104  (the MLX affine_quantize replica)
- ``dequantize``           :107-113
- ``r_contract``           :116-118 (fp64 truth of the quantized layer)
- ensemble members         :131-245 (six fp32 evaluations whose worst error
                                     against ``r_contract`` is the floor)
- artefact faults          :253-313
- ``pack_codes``/``unpack_codes``: the contiguous little-endian code stream of
  ``kernelverify/pack/wide_qmv.py:185-201`` and its inverse
  (``bench/phase0_contract_k.py:84-100``).

Every member's arithmetic is the member's definition: the sequence of fp32
roundings is what sets the floor, so each one uses the same numpy primitive
(pairwise ``@``, ``np.add.accumulate``, ``einsum(optimize=True)``) in the same
order as the reference describes.

Parity pins (tests/test_oracle_golden.py, tests/test_oracle_contract.py):
- quantizer, dequantizer and ``r_contract``: ``ref_scale`` of all 768
  committed records of ``bench/results/quant_device_adequacy.json`` at bits
  2/3/4/8, plus the closed-form checks (codes in range, edge exactly
  representable, round-half-away on exact halves);
- BLAS-free members (dequant-serial, dequant-reversed, factored-groups chains):
  the committed per-member errors, plus a scalar-chain rewrite of
  factored-groups (``tests/test_quant_contract_members.py:56-108``);
- BLAS members (dequant-pairwise, lut-gather, factored-serial): the committed
  per-member errors within the BLAS-difference band (the reference ran
  Accelerate, this container OpenBLAS);
- faults: every committed fault error, and "every fault fails the gate";
- packing: brute-force bit stream on tiny rows, pack/unpack round trip at
  bits 2/3/4/5/6/8.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

QUANT_ENSEMBLE_VERSION = "quant-ensemble-v2"


@dataclass(frozen=True)
class QuantContract:
    scheme: str = "mlx-affine"
    bits: int = 4
    group_size: int = 64


@dataclass(frozen=True)
class QuantArtefact:
    """Unpacked artefact: integer levels plus per-group scale and bias."""

    q: np.ndarray        # (rows, cols) int32 in [0, 2^bits - 1]
    scales: np.ndarray   # (rows, cols // group) in W's dtype
    biases: np.ndarray   # (rows, cols // group) in W's dtype
    contract: QuantContract


def round_half_away(v: np.ndarray) -> np.ndarray:
    """sign(v) * floor(|v| + 0.5), evaluated in v's own precision (fp32 here).

    This is the contract's rounding, including its fp32 quirk: |v| + 0.5 is
    itself rounded, so 0.49999997 rounds up. The GPU quantizer evaluates the
    same expression to stay bit-exact.
    """
    return np.sign(v) * np.floor(np.abs(v) + np.float32(0.5))


def canonical_quantize(w: np.ndarray, contract: QuantContract) -> QuantArtefact:
    """MLX-affine quantization of a 2-D weight matrix, all arithmetic in fp32.

    Per 64-wide group along the columns:
      lo = min(group), hi = max(max(group), 0)
      step = max((hi - lo) / (2^bits - 1), 1e-7), negated unless |lo| > |hi|
      edge = lo if |lo| > |hi| else hi
      q0 = round_half_away(edge / step)
      if q0 != 0: step = edge / q0 and bias = edge, else bias = 0
      q = min(round_half_away((w - bias) / step), 2^bits - 1)
    Scales and biases are cast to W's dtype only when stored.
    """
    g = contract.group_size
    top = np.float32((1 << contract.bits) - 1)
    rows, cols = w.shape
    if cols % g:
        raise ValueError(f"d_in {cols} must be a multiple of group_size {g}")
    blocks = w.astype(np.float32).reshape(rows, cols // g, g)
    lo = blocks.min(axis=2)
    hi = np.maximum(blocks.max(axis=2), np.float32(0.0))

    low_side = np.abs(lo) > np.abs(hi)
    step = np.maximum((hi - lo) / top, np.float32(1e-7))
    step = np.where(low_side, step, -step).astype(np.float32)
    edge = np.where(low_side, lo, hi).astype(np.float32)
    q0 = round_half_away((edge / step).astype(np.float32))
    snapped = q0 != 0.0
    safe_q0 = np.where(snapped, q0, np.float32(1.0))
    step = np.where(snapped, (edge / safe_q0).astype(np.float32), step)
    bias = np.where(snapped, edge, np.float32(0.0)).astype(np.float32)

    levels = round_half_away(((blocks - bias[..., None]) / step[..., None])
                             .astype(np.float32))
    levels = np.minimum(levels, top).astype(np.int32).reshape(rows, cols)
    return QuantArtefact(q=levels, scales=step.astype(w.dtype),
                         biases=bias.astype(w.dtype), contract=contract)


def dequantize(a: QuantArtefact, dtype=np.float64) -> np.ndarray:
    """W~ = scale * q + bias per group, at ``dtype`` (fp64 is the truth)."""
    g = a.contract.group_size
    rows, cols = a.q.shape
    levels = a.q.reshape(rows, cols // g, g).astype(dtype)
    wt = a.scales.astype(dtype)[..., None] * levels + a.biases.astype(dtype)[..., None]
    return wt.reshape(rows, cols)


def r_contract(x: np.ndarray, a: QuantArtefact) -> np.ndarray:
    """fp64 evaluation of the intended quantized layer: x @ W~^T."""
    return x.astype(np.float64) @ dequantize(a, np.float64).T


# ---------------------------------------------------------------------------
# Code stream packing (the artefact layout the kernels read)
# ---------------------------------------------------------------------------
def pack_codes(q: np.ndarray, bits: int) -> np.ndarray:
    """Contiguous little-endian bit stream per row, viewed as uint32.

    Code i of a row occupies bits [i*bits, (i+1)*bits) of the row's stream.
    Written as an explicit bit scatter so it shares nothing with the
    product's packer it is used to check.
    """
    rows, cols = q.shape
    if (cols * bits) % 32:
        raise ValueError("a row's code stream must fill whole 32-bit words")
    q = q.astype(np.uint64)
    bitplanes = ((q[:, :, None] >> np.arange(bits, dtype=np.uint64)) & 1).astype(np.uint8)
    stream = bitplanes.reshape(rows, cols * bits)
    packed = np.packbits(stream, axis=1, bitorder="little")
    return np.ascontiguousarray(packed).view(np.uint32)


def unpack_codes(words: np.ndarray, cols: int, bits: int) -> np.ndarray:
    """Inverse of ``pack_codes``: (rows, cols*bits/32) uint32 -> (rows, cols) int32."""
    words = np.ascontiguousarray(words, dtype=np.uint32)
    stream = np.unpackbits(words.view(np.uint8).reshape(words.shape[0], -1),
                           axis=1, bitorder="little")
    pos = np.arange(cols)[:, None] * bits + np.arange(bits)[None, :]
    weight = (1 << np.arange(bits)).astype(np.int64)
    return (stream[:, pos].astype(np.int64) * weight).sum(axis=2).astype(np.int32)


# ---------------------------------------------------------------------------
# The legitimate fp32 ensemble (reference :131-245)
# ---------------------------------------------------------------------------
def _as_f32(v):
    return v.astype(np.float32)


def member_dequant_pairwise(x, a):
    """fp32 dequant, then a pairwise (BLAS) product."""
    return (_as_f32(x) @ dequantize(a, np.float32).T).astype(x.dtype)


# Row-chunk budget for the serial members' (m, rows, d_in) product. Chunking
# by output row is exact: each accumulation runs along d_in inside one row.
SERIAL_CHUNK_BYTES = 1 << 27


def _serial_accumulate(x32, w32, reverse: bool):
    m, d_in = x32.shape
    rows = w32.shape[0]
    per_row = m * d_in * 4
    step = max(1, SERIAL_CHUNK_BYTES // per_row)
    out = np.empty((m, rows), dtype=np.float32)
    for r0 in range(0, rows, step):
        prod = x32[:, None, :] * w32[r0:r0 + step][None, :, :]
        if reverse:
            prod = prod[:, :, ::-1]
        out[:, r0:r0 + step] = np.add.accumulate(prod, axis=2)[:, :, -1]
    return out


def member_dequant_serial(x, a):
    """fp32 dequant, strictly left-to-right accumulation over d_in."""
    return _serial_accumulate(_as_f32(x), dequantize(a, np.float32), False).astype(x.dtype)


def member_dequant_reversed(x, a):
    """fp32 dequant, strictly right-to-left accumulation over d_in."""
    return _serial_accumulate(_as_f32(x), dequantize(a, np.float32), True).astype(x.dtype)


def member_lut_gather(x, a):
    """Per-group table of the 2^bits dequantized levels, gathered, then BLAS."""
    g = a.contract.group_size
    rows, cols = a.q.shape
    table = (a.scales.astype(np.float32)[..., None]
             * np.arange(1 << a.contract.bits, dtype=np.float32)
             + a.biases.astype(np.float32)[..., None])
    wt = np.take_along_axis(table, a.q.reshape(rows, cols // g, g), axis=2)
    return (_as_f32(x) @ wt.reshape(rows, cols).T).astype(x.dtype)


def member_factored_groups(x, a):
    """Integer-domain form s*sum(x*q) + b*sum(x) with both per-group sums as
    explicit fp32 chains over the 64 group positions; groups then combine
    pairwise (scale term) and through BLAS (bias term)."""
    g = a.contract.group_size
    rows, cols = a.q.shape
    ng = cols // g
    xg = _as_f32(x).reshape(x.shape[0], ng, g)
    qg = a.q.reshape(rows, ng, g).astype(np.float32)
    dot = np.zeros((x.shape[0], rows, ng), dtype=np.float32)
    xsum = np.zeros((x.shape[0], ng), dtype=np.float32)
    for k in range(g):
        dot += xg[:, None, :, k] * qg[None, :, :, k]
        xsum += xg[:, :, k]
    out = (dot * a.scales.astype(np.float32)[None]).sum(axis=2)
    out += xsum @ a.biases.astype(np.float32).T
    return out.astype(x.dtype)


def member_factored_serial(x, a):
    """Integer-domain form with a strictly serial sum across groups."""
    g = a.contract.group_size
    rows, cols = a.q.shape
    xg = _as_f32(x).reshape(x.shape[0], cols // g, g)
    qg = a.q.reshape(rows, cols // g, g).astype(np.float32)
    dot = np.einsum("bgk,rgk->brg", xg, qg, optimize=True)
    per_group = (dot * a.scales.astype(np.float32)[None]
                 + xg.sum(axis=2)[:, None, :] * a.biases.astype(np.float32)[None])
    return np.add.accumulate(per_group, axis=2)[:, :, -1].astype(x.dtype)


ENSEMBLE = {
    "dequant-pairwise": member_dequant_pairwise,
    "dequant-serial": member_dequant_serial,
    "lut-gather": member_lut_gather,
    "factored-groups": member_factored_groups,
    "factored-serial": member_factored_serial,
    "dequant-reversed": member_dequant_reversed,
}


# ---------------------------------------------------------------------------
# Artefact faults (reference :253-313): each must FAIL the gate
# ---------------------------------------------------------------------------
def _art(a, q=None, scales=None, biases=None):
    return QuantArtefact(a.q if q is None else q,
                         a.scales if scales is None else scales,
                         a.biases if biases is None else biases, a.contract)


def fault_scales_rotated(a):
    """Each group reads its neighbour's scale and bias."""
    return _art(a, scales=np.roll(a.scales, 1, axis=1), biases=np.roll(a.biases, 1, axis=1))


def fault_nibble_swapped(a):
    """Adjacent codes transposed pairwise."""
    q = a.q.reshape(a.q.shape[0], -1, 2)[:, :, ::-1].reshape(a.q.shape)
    return _art(a, q=np.ascontiguousarray(q))


def fault_bias_dropped(a):
    """Affine bias discarded."""
    return _art(a, biases=np.zeros_like(a.biases))


def fault_group_size_halved(a):
    """Each scale/bias applied to half its span."""
    n = a.scales.shape[1]
    return _art(a, scales=np.repeat(a.scales, 2, axis=1)[:, :n],
                biases=np.repeat(a.biases, 2, axis=1)[:, :n])


def fault_unpack_mask_too_wide(a):
    """Mask one bit too wide: each code picks up its right neighbour's low bit
    as its own top bit, clipped to the top level."""
    top = (1 << a.contract.bits) - 1
    carry = np.roll(a.q, -1, axis=1) & 1
    q = np.minimum(a.q + (carry << a.contract.bits) // 2, top)
    return _art(a, q=np.ascontiguousarray(q.astype(a.q.dtype)))


def fault_all_groups_read_group_zero(a):
    """Every group reads group 0's scale and bias."""
    return _art(a,
                scales=np.ascontiguousarray(np.broadcast_to(a.scales[:, :1], a.scales.shape)),
                biases=np.ascontiguousarray(np.broadcast_to(a.biases[:, :1], a.biases.shape)))


FAULTS = {
    "scales-rotated-one-group": fault_scales_rotated,
    "nibble-order-swapped": fault_nibble_swapped,
    "bias-dropped": fault_bias_dropped,
    "group-size-halved": fault_group_size_halved,
    "unpack-mask-too-wide": fault_unpack_mask_too_wide,
    "all-groups-read-group-0": fault_all_groups_read_group_zero,
}


def boundary_fp16_dequant(x, a):
    """fp16 intermediate dequant then fp32 MAC: the precision-boundary case
    the reference's calibration records (``bench/calibrate_quant_bits.py``
    ``boundary_fp16_dequant``); a contract violation, kept as a negative
    control."""
    w16 = dequantize(a, np.float32).astype(np.float16).astype(np.float32)
    return (x.astype(np.float32) @ w16.T).astype(x.dtype)
