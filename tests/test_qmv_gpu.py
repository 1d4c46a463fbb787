"""kvp_qmv on the GPU against the CPU oracle (fp64 ``r_contract`` + ensemble floor).

Mirrors the reference's kernel tests (tests/test_pack_wide_qmv.py:60-153):
contract agreement across M, d_out not divisible by the row tile, every bit
width x M, plus the MI355X additions: BASELINE configs 1 and 2 at full size,
fp32 output, activations large enough to be staged in chunks, the
calibration input modes, and negative controls (a faulted artefact must fail
the same gate).

Tolerance: ``max(4 * eps(out dtype) * max|ref|, 4.0 * worst ensemble member)``
(kernelverify/schemas/native_ops.py:42-50, :128-132).
"""

import numpy as np
import pytest

from kernelverify_amd.pack import wide_qmv
from kernelverify_amd.pack.codes import pack_codes
from oracle.extensions import artefact_from_arrays
from oracle.inputs import make_w, make_x
from oracle.native_ops import qmm_reference_artefact, qmm_tolerance_artefact
from oracle.quant_contract import FAULTS, QuantContract, canonical_quantize
from oracle.verify import judge, qmv_inputs, verify_output
from tests.artefacts import draw_qmv

pytestmark = pytest.mark.gpu


def run_gpu(x, art, bits, out_dtype="float16"):
    return wide_qmv.qmv(x, pack_codes(art.q, bits), art.scales, art.biases, bits=bits,
                        out_dtype=out_dtype)


def gate(x, art, got, out_dtype, rows=None):
    """Verdict on all rows, or on a row subset (rows are independent)."""
    if rows is not None:
        art = artefact_from_arrays(art.q[rows], art.scales[rows], art.biases[rows],
                                   art.contract.bits)
        got = got[:, rows]
    ref = qmm_reference_artefact(x, art)
    tol = qmm_tolerance_artefact(out_dtype, x, art, ref)
    return judge(got, ref, tol)


def test_config1_4096_square_4bit_m1():
    x, q, s, b = draw_qmv(4096, 4096, 4, 1, seed=1)
    art = artefact_from_arrays(q, s, b, 4)
    got = run_gpu(x, art, 4)
    v = gate(x, art, got, "float16")
    print("cfg1", v)
    assert v.ok, v


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8, 11, 16])
def test_every_width_and_m(bits, m):
    x, q, s, b = draw_qmv(300, 1024, bits, m, seed=100 + 7 * bits + m)
    art = artefact_from_arrays(q, s, b, bits)
    for out_dtype in ("float16", "float32"):
        got = run_gpu(x, art, bits, out_dtype)
        assert got.dtype == np.dtype(out_dtype)
        v = gate(x, art, got, out_dtype)
        assert v.ok, (bits, m, out_dtype, v)


@pytest.mark.parametrize("bits", [2, 3])
@pytest.mark.parametrize("m", [1, 2, 4, 5, 8, 9, 16])
@pytest.mark.parametrize("d_out,d_in", [(300, 1024), (77, 384), (40, 320)])
def test_matrix_cores_at_two_and_three_bits(bits, m, d_out, d_in):
    """The matrix-core kernel forced (tuning key qmv_path = 4) at 2 and 3
    bits: four, two or one group per step (M <= 4, <= 8 with an even group
    count, otherwise; a 3-bit lane then holds 48 bits of a group, loaded as
    three halfwords), judged against the oracle on all rows."""
    from kernelverify_amd import lib

    x, q, s, b = draw_qmv(d_out, d_in, bits, m, seed=500 + 13 * bits + m + d_in)
    art = artefact_from_arrays(q, s, b, bits)
    lib.set_tuning("qmv_path", 4)
    try:
        got = run_gpu(x, art, bits, "float32")
    finally:
        lib.set_tuning("qmv_path", -1)
    v = gate(x, art, got, "float32")
    assert v.ok, (bits, m, d_out, d_in, v)


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
@pytest.mark.parametrize("m", [9, 16])
def test_valu_kernels_above_eight_rows(bits, m):
    """The VALU kernels forced (tuning key qmv_path = 3, chunked x) at M = 9
    and 16: the library runs them as two calls of at most eight rows of x
    (rows 8.. offset into x and out), judged against the oracle."""
    from kernelverify_amd import lib

    x, q, s, b = draw_qmv(200, 1024, bits, m, seed=700 + 11 * bits + m)
    art = artefact_from_arrays(q, s, b, bits)
    lib.set_tuning("qmv_path", 3)
    try:
        got = run_gpu(x, art, bits, "float32")
    finally:
        lib.set_tuning("qmv_path", -1)
    v = gate(x, art, got, "float32")
    assert v.ok, (bits, m, v)


@pytest.mark.parametrize("d_out", [1, 3, 15, 17, 1000])
def test_d_out_not_divisible_by_the_row_tile(d_out):
    x, q, s, b = draw_qmv(d_out, 512, 4, 2, seed=d_out)
    art = artefact_from_arrays(q, s, b, 4)
    v = gate(x, art, run_gpu(x, art, 4), "float16")
    assert v.ok, v


@pytest.mark.parametrize("bits,m", [(4, 16), (2, 16), (8, 12), (3, 9)])
def test_activations_staged_in_chunks(bits, m):
    """M * d_in large enough that x is staged into LDS in several chunks."""
    x, q, s, b = draw_qmv(64, 14336, bits, m, seed=bits * 31 + m)
    art = artefact_from_arrays(q, s, b, bits)
    v = gate(x, art, run_gpu(x, art, bits, "float32"), "float32")
    assert v.ok, v


@pytest.mark.parametrize("mode", ["unit", "corpus-scale", "near-zero", "constant-rows"])
@pytest.mark.parametrize("bits", [2, 3, 4, 8])
def test_raw_weight_gate_every_calibration_mode(mode, bits):
    """The reference gate's own path: raw W, the oracle quantizes it
    (pack/verify.py:61-69), in the calibration harness's input modes."""
    rng = np.random.default_rng(10_000 + bits)
    w = make_w(256, 1024, "normal-0.02", rng)
    art = canonical_quantize(w, QuantContract(bits=bits, group_size=64))
    for dtype, name in ((np.float16, "float16"), (np.float32, "float32")):
        x = make_x(2, 1024, dtype, mode, rng)
        got = run_gpu(x.astype(np.float16), art, bits, name)
        if dtype == np.float16:
            v = verify_output("quantized_matmul", qmv_inputs(x, w, bits), got, name)
        else:
            # fp32 activations are narrowed to the kernel's fp16 x: judge the
            # kernel on the x it was given.
            v = gate(x.astype(np.float16), art, got, name)
        assert v.ok, (mode, bits, name, v)


@pytest.mark.parametrize("fault", sorted(FAULTS))
def test_faulted_artefact_fails_the_gate(fault):
    """Negative control: the kernel run on a faulted artefact must fail the
    gate of the true artefact (kernelverify/schemas/quant_contract.py:253-313)."""
    x, q, s, b = draw_qmv(256, 1024, 4, 2, seed=5)
    art = artefact_from_arrays(q, s, b, 4)
    bad = FAULTS[fault](art)
    got = run_gpu(x, bad, 4)
    assert not gate(x, art, got, "float16").ok


@pytest.mark.parametrize("d_out,d_in", [(14336, 4096), (4096, 14336)])
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("m", [1, 4, 8])
def test_config2_llama_mlp_shapes(d_out, d_in, bits, m):
    """Full-size BASELINE config 2; the oracle judges a spread row subset
    (every output row is an independent dot product)."""
    x, q, s, b = draw_qmv(d_out, d_in, bits, m, seed=2000 + bits + m)
    art = artefact_from_arrays(q, s, b, bits)
    got = run_gpu(x, art, bits)
    assert np.isfinite(got.astype(np.float32)).all()
    rows = np.unique(np.concatenate([np.arange(256), np.arange(d_out - 64, d_out),
                                     np.random.default_rng(0).choice(d_out, 256, replace=False)]))
    v = gate(x, art, got, "float16", rows=rows)
    assert v.ok, v


def test_single_pass_is_linear_in_x():
    """Size-independent property at full size: out(x1 + x2) = out(x1) + out(x2)
    to fp32 rounding (fp32 output, sums of fp16 inputs kept exact)."""
    x, q, s, b = draw_qmv(14336, 4096, 4, 2, seed=9)
    art = artefact_from_arrays(q, s, b, 4)
    x1 = (x.astype(np.float32) * 0.5).astype(np.float16)
    x2 = (x.astype(np.float32) - x1.astype(np.float32)).astype(np.float16)
    both = np.concatenate([x1, x2], axis=0)
    xsum = (x1.astype(np.float32) + x2.astype(np.float32)).astype(np.float16)
    parts = run_gpu(both, art, 4, "float32")
    whole = run_gpu(xsum, art, 4, "float32")
    lhs = parts[:2] + parts[2:]
    scale = np.abs(whole).max()
    assert np.max(np.abs(lhs - whole)) <= 1e-5 * scale


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("d_out,d_in", [(4099, 2560), (1001, 4096), (70001, 256)])
def test_persistent_m1_kernel_every_width(bits, d_out, d_in):
    """The persistent M = 1 kernel (waves walking row sets through a ring),
    forced with tuning key qmv_path = 5 on shapes whose d_out is not a
    multiple of its two-row set and, for 70001 rows, of the grid's waves;
    judged on all rows against the oracle."""
    from kernelverify_amd import lib

    x, q, s, b = draw_qmv(d_out, d_in, bits, 1, seed=bits * 7 + d_out)
    art = artefact_from_arrays(q, s, b, bits)
    lib.set_tuning("qmv_path", 5)
    try:
        got = run_gpu(x, art, bits, "float32")
    finally:
        lib.set_tuning("qmv_path", -1)
    v = gate(x, art, got, "float32")
    assert v.ok, (bits, d_out, d_in, v)
