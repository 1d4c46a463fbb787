"""Affine group-quantized matvec on MI355X: one weight pass for any M.

Host side of ``kvp_qmv`` (kernelverify_amd/csrc/qmv.hip), mirroring the
reference's pack module ``kernelverify/pack/wide_qmv.py``: the same artefact
layout (code stream + fp16 scale/bias per 64-code group), the same output
(``out[m, row]``, M x d_out, fp16 or fp32) and the same single-pass promise:
the weights stream from HBM once whatever M is.

What differs is the tiling, chosen for CDNA4 rather than inherited from the
Metal register wall (wide_qmv.py:17-26): 64-lane waves own RW rows (2 for
M <= 8, 1 above), lanes stream 16-byte units, and codes multiply as exact
fp16 denormals through V_DOT2_F32_F16. Three kernel paths share that core:
streaming (M = 1: each wave loads its own activation fragments, no LDS, no
barrier), resident (x staged once per persistent block) and chunked (x too
large for LDS, staged in chunks). From M = 2, 4- and 8-bit rows run on the
matrix cores instead (csrc/qmv_mfma.hip): codes as exact fp16 denormals
times a block-diagonal activation operand, so the cost no longer grows with
M. Widths 2, 3, 4 and 8 bits are all served (the reference kernel stops at
4, :140).
"""

from __future__ import annotations

import hashlib
from pathlib import Path

import numpy as np

from kernelverify_amd import build, lib
from kernelverify_amd.hip import DeviceArray
from kernelverify_amd.pack.codes import pack_codes, pack_nibbles, unpack_codes  # noqa: F401

KERNEL_NAME = "kvp_qmv"
SUPPORTED_BITS = (2, 3, 4, 8)
MAX_M = 16
GROUP = 64
WAVE = 64
WAVES_PER_BLOCK = 4
OUT_DTYPES = {"float16": lib.KVP_F16, "float32": lib.KVP_F32}


def rows_per_wave(m: int, bits: int = 4, d_out: int = 0, d_in: int = 1 << 30) -> int:
    """RW: rows a wave of the VALU paths walks together (the VGPR budget of
    M * RW accumulators; csrc/qmv.hip, launch_qmv_rw). The same at every
    shape; the shape arguments stay for callers that pin a priced cell."""
    return 2 if m <= 8 else 1


KERNEL_SOURCES = ("csrc/qmv.hip", "csrc/qmv_core.h", "csrc/qmv_mfma.hip", "csrc/mfma_core.h",
                  "csrc/common.h")


def kernel_source_sha256() -> str:
    """sha256 over the qmv kernel sources and the device flags they are
    compiled with (the body a routing recording priced; the reference pins
    the MSL string, routed_windows.py:61-64)."""
    h = hashlib.sha256()
    for rel in KERNEL_SOURCES:
        h.update((Path(__file__).resolve().parents[1] / rel).read_bytes())
    h.update(build.flags_fingerprint())
    return h.hexdigest()


def should_dispatch(m: int, bits: int, d_out: int, d_in: int) -> bool:
    """Whether this cell should run on the pack or stay on the vendor GEMM
    (reference: pack/wide_qmv.py:143-177).

    Every argument is required: routing is a property of the whole (tile
    width, bit width, shape) cell, read from the measured windows in
    routed_windows. A shape or width the recording did not price routes
    nowhere, whatever the kernel supports.
    """
    from kernelverify_amd.pack import routed_windows

    return m in routed_windows.window_for(bits, d_out, d_in)


def launch_config(d_out: int, m: int, bits: int = 4, d_in: int = 1 << 30) -> tuple:
    """(grid, block, RW): blocks of four waves over ceil(d_out / (4 * RW))."""
    r = rows_per_wave(m, bits, d_out, d_in)
    rows_per_block = WAVES_PER_BLOCK * r
    return (((d_out + rows_per_block - 1) // rows_per_block, 1, 1),
            (WAVE * WAVES_PER_BLOCK, 1, 1), r)


def artefact_bytes(d_out: int, d_in: int, bits: int) -> int:
    """Packed codes plus fp16 scales and biases (bench/pack_wide_qmv.py:134-137)."""
    return d_out * d_in * bits // 8 + 2 * (d_out * d_in // GROUP) * 2


def algorithmic_bytes(m: int, d_out: int, d_in: int, bits: int, out_itemsize: int = 2) -> int:
    """HBM bytes one call must move at minimum: the artefact once, x, out."""
    return artefact_bytes(d_out, d_in, bits) + m * d_in * 2 + m * d_out * out_itemsize


def check_shapes(x: DeviceArray, w_q: DeviceArray, scales: DeviceArray, biases: DeviceArray,
                 out: DeviceArray, bits: int) -> tuple[int, int, int]:
    """(m, d_out, d_in) after checking every operand against the layout."""
    if bits not in SUPPORTED_BITS:
        raise lib.Unsupported(f"qmv: bits={bits} not in {SUPPORTED_BITS}")
    if len(x.shape) != 2 or x.dtype != np.float16:
        raise lib.InvalidArgument(f"qmv: x must be fp16 (M, d_in), got {x.dtype} {x.shape}")
    m, d_in = x.shape
    if d_in % GROUP:
        raise lib.InvalidArgument(f"qmv: d_in={d_in} is not a multiple of {GROUP}")
    if not 1 <= m <= MAX_M:
        raise lib.InvalidArgument(f"qmv: M={m} outside 1..{MAX_M}")
    if len(w_q.shape) != 2 or w_q.dtype != np.uint32:
        raise lib.InvalidArgument(f"qmv: w_q must be uint32 (d_out, words), got {w_q.dtype}")
    d_out = w_q.shape[0]
    if w_q.shape[1] * 32 != d_in * bits:
        raise lib.InvalidArgument(
            f"qmv: w_q has {w_q.shape[1]} words per row, {bits}-bit d_in={d_in} needs "
            f"{d_in * bits // 32}")
    for name, t in (("scales", scales), ("biases", biases)):
        if t.shape != (d_out, d_in // GROUP) or t.dtype != np.float16:
            raise lib.InvalidArgument(
                f"qmv: {name} must be fp16 {(d_out, d_in // GROUP)}, got {t.dtype} {t.shape}")
    if out.shape != (m, d_out) or out.dtype.name not in OUT_DTYPES:
        raise lib.InvalidArgument(f"qmv: out must be fp16/fp32 {(m, d_out)}, got {out.dtype} "
                                  f"{out.shape}")
    return m, d_out, d_in


def run_qmv(x: DeviceArray, w_q: DeviceArray, scales: DeviceArray, biases: DeviceArray,
            out: DeviceArray, *, bits: int, stream=None) -> None:
    """Enqueue out = x @ dequant(w)^T on ``stream`` (device buffers, no sync)."""
    m, d_out, d_in = check_shapes(x, w_q, scales, biases, out, bits)
    lib.check(lib.load().kvp_qmv(x.ptr, w_q.ptr, scales.ptr, biases.ptr, out.ptr,
                                 OUT_DTYPES[out.dtype.name], m, d_out, d_in, bits,
                                 getattr(stream, "handle", stream)))


class QmvCall:
    """One validated qmv launch with its ctypes arguments bound once.

    For serving loops and graph capture: ``call(stream)`` is a bare C call,
    no per-launch Python shape checks.
    """

    def __init__(self, x: DeviceArray, w_q: DeviceArray, scales: DeviceArray,
                 biases: DeviceArray, out: DeviceArray, *, bits: int):
        m, d_out, d_in = check_shapes(x, w_q, scales, biases, out, bits)
        self._fn = lib.load().kvp_qmv
        self._args = (x.ptr, w_q.ptr, scales.ptr, biases.ptr, out.ptr,
                      OUT_DTYPES[out.dtype.name], m, d_out, d_in, bits)
        self._keep = (x, w_q, scales, biases, out)

    def __call__(self, stream=None) -> None:
        status = self._fn(*self._args, getattr(stream, "handle", stream))
        if status:
            lib.check(status)


def qmv(x: np.ndarray, w_q: np.ndarray, scales: np.ndarray, biases: np.ndarray, *, bits: int,
        out_dtype: str = "float16") -> np.ndarray:
    """Host convenience: upload, run, synchronise, download."""
    from kernelverify_amd import hip

    dx, dw = DeviceArray.from_host(x.astype(np.float16)), DeviceArray.from_host(w_q)
    ds, db = DeviceArray.from_host(scales), DeviceArray.from_host(biases)
    out = DeviceArray((x.shape[0], w_q.shape[0]), out_dtype)
    run_qmv(dx, dw, ds, db, out, bits=bits)
    hip.synchronize()
    return out.to_host()


def kernel_spec():
    """The runner-door template (reference: kernelverify/pack/wide_qmv.py:218-260).

    A pack-library descriptor with the reference template's compile-time
    constants: `specialize()` fills `T` (half | float), `BITS`, `M` and `R`;
    the bindings keep the reference's names and order (x, w_q, scales,
    biases, out, d_in_arg, d_out_arg). `R` is accepted and recorded; the
    library tiles by its own rule (`rows_per_wave`). The grid's `row_blocks`
    extent is informational for the library, which launches its own grid.
    """
    from kernelverify_amd.runners import Binding, BindingKind, KernelSpec, LaunchMode, LaunchSpec

    return KernelSpec(
        source="kvpack:wide_qmv T=$T BITS=$BITS M=$M R=$R",
        entry_point=KERNEL_NAME,
        name=f"{KERNEL_NAME}-$BITS bit-M$M-R$R-$T",
        bindings=(Binding(BindingKind.INPUT, "x"),
                  Binding(BindingKind.INPUT, "w_q"),
                  Binding(BindingKind.INPUT, "scales"),
                  Binding(BindingKind.INPUT, "biases"),
                  Binding(BindingKind.OUTPUT),
                  Binding(BindingKind.SCALAR, "d_in_arg", "uint32"),
                  Binding(BindingKind.SCALAR, "d_out_arg", "uint32")),
        launch=LaunchSpec(grid=("row_blocks", 1, 1), threadgroup=(WAVE * WAVES_PER_BLOCK, 1, 1),
                          mode=LaunchMode.THREADGROUPS),
    )
