"""The CPU oracle against the reference's committed calibration evidence.

``tests/golden/quant_device_adequacy.records.json`` is a field subset of the
reference's ``bench/results/quant_device_adequacy.json``: 768 records, 192 at
each of bits 2/3/4/8, over shapes 512x512, 1024x4096 and 4096x4096 (config 1's
shape), produced on the reference machine by the reference's own quantizer
(checked bit-exact against mx.quantize there) and numpy/Accelerate.

Each record's inputs regenerate from ``default_rng(10000 + seed)``: ``make_w``
first, then ``make_x(2, d_in, dtype, mode)`` for every mode then dtype. What
each check pins:

- ``ref_scale`` = max |r_contract| must match to fp64 round-off: a wrong code,
  scale, bias, dequant formula or transposed product moves it far above that.
- the BLAS-free members (serial / reversed chains) must reproduce the
  recorded error to 1e-9 relative: their fp32 outputs are platform-independent
  and only the fp64 dgemm inside ``r_contract`` rounds differently.
- BLAS members and faults run through sgemm, whose rounding differs between
  Accelerate and OpenBLAS: they must match within that band.
"""

import json
from functools import lru_cache
from pathlib import Path

import numpy as np
import pytest

from oracle.inputs import MODES, make_w, make_x
from oracle.native_ops import _base_tol
from oracle.quant_contract import (
    ENSEMBLE,
    FAULTS,
    QuantContract,
    boundary_fp16_dequant,
    canonical_quantize,
    r_contract,
)

GOLDEN = Path(__file__).resolve().parent / "golden" / "quant_device_adequacy.records.json"
BLAS_FREE = ("dequant-serial", "dequant-reversed")
BLAS_MEMBERS = ("dequant-pairwise", "lut-gather", "factored-serial", "factored-groups")


@lru_cache(maxsize=1)
def _records():
    return json.loads(GOLDEN.read_text())["records"]


def _blocks(shapes, bits_list=(2, 3, 4, 8), seeds=(0, 1, 100, 101)):
    out = {}
    for r in _records():
        if r["shape"] in shapes and r["bits"] in bits_list and r["seed"] in seeds:
            out.setdefault((r["bits"], r["shape"], r["draw"], r["seed"]), []).append(r)
    return out


def _regenerate(bits, shape, draw, seed):
    d_out, d_in = (int(v) for v in shape.split("x"))
    rng = np.random.default_rng(10_000 + seed)
    w = make_w(d_out, d_in, draw, rng)
    art = canonical_quantize(w, QuantContract(bits=bits, group_size=64))
    xs = {}
    for mode in MODES:
        for name in ("float32", "float16"):
            xs[(mode, name)] = make_x(2, d_in, np.float32 if name == "float32" else np.float16,
                                      mode, rng)
    return art, xs


def _err(c, ref):
    return float(np.max(np.abs(c.astype(np.float64) - ref)))


def test_fixture_has_every_record():
    recs = _records()
    assert len(recs) == 768
    assert sorted({r["bits"] for r in recs}) == [2, 3, 4, 8]
    assert {r["shape"] for r in recs} == {"512x512", "1024x4096", "4096x4096"}


SMALL = sorted(_blocks(("512x512",)).keys())


@pytest.mark.parametrize("key", SMALL, ids=[f"b{k[0]}-{k[2]}-s{k[3]}" for k in SMALL])
def test_512_blocks_reproduce_every_field(key):
    """Full check on the cheapest shape: ref_scale, base_tol, all six members,
    all six faults and the fp16-dequant boundary."""
    art, xs = _regenerate(*key)
    for rec in _blocks(("512x512",))[key]:
        x = xs[(rec["mode"], rec["dtype"])]
        ref = r_contract(x, art)
        scale = float(np.abs(ref).max())
        assert scale == pytest.approx(rec["ref_scale"], rel=1e-12, abs=0.0)
        assert _base_tol(rec["dtype"], ref) == pytest.approx(rec["base_tol"], rel=1e-12)
        for name in BLAS_FREE:
            # exact up to the fp64 dgemm rounding inside r_contract itself
            assert _err(ENSEMBLE[name](x, art), ref) == pytest.approx(
                rec["members"][name], rel=1e-9), name
        for name in BLAS_MEMBERS:
            got = _err(ENSEMBLE[name](x, art), ref)
            want = rec["members"][name]
            # Accelerate vs OpenBLAS rounding band (measured up to ~17x apart
            # at these sizes); a restatement mistake is O(scale), 1e4x above.
            assert got <= max(64.0 * want, 1e-5 * scale), (name, got, want)
            assert want <= max(64.0 * got, 1e-5 * scale), (name, got, want)
        for name, fault in FAULTS.items():
            got = _err(ENSEMBLE["dequant-pairwise"](x, fault(art)), ref)
            want = rec["faults"][name]
            if want > 1e-3 * scale:
                assert got == pytest.approx(want, rel=1e-3), name
            else:  # the fault is invisible on this input (e.g. constant rows)
                assert got <= 1e-3 * scale, name
        got = _err(boundary_fp16_dequant(x, art), ref)
        assert got == pytest.approx(rec["boundary_fp16_dequant"], rel=0.5, abs=1e-5 * scale)


MID = sorted(_blocks(("1024x4096",), seeds=(0, 101)).keys())


@pytest.mark.parametrize("key", MID, ids=[f"b{k[0]}-{k[2]}-s{k[3]}" for k in MID])
def test_1024x4096_ref_scale_and_serial_members(key):
    art, xs = _regenerate(*key)
    for rec in _blocks(("1024x4096",), seeds=(0, 101))[key]:
        x = xs[(rec["mode"], rec["dtype"])]
        ref = r_contract(x, art)
        assert float(np.abs(ref).max()) == pytest.approx(rec["ref_scale"], rel=1e-12, abs=0.0)
        if rec["mode"] in ("unit", "constant-rows"):
            assert _err(ENSEMBLE["dequant-serial"](x, art), ref) == pytest.approx(
                rec["members"]["dequant-serial"], rel=1e-9)


BIG = [(b, "4096x4096", "normal-0.02", 0) for b in (2, 3, 4, 8)] + [(4, "4096x4096", "heavy-tailed", 101)]


@pytest.mark.parametrize("key", BIG, ids=[f"b{k[0]}-{k[2]}-s{k[3]}" for k in BIG])
def test_config1_shape_ref_scale(key):
    """Config 1's 4096x4096 shape: the quantizer is exact at full size."""
    art, xs = _regenerate(*key)
    recs = [r for r in _records() if (r["bits"], r["shape"], r["draw"], r["seed"]) == key]
    assert len(recs) == 8
    for rec in recs:
        x = xs[(rec["mode"], rec["dtype"])]
        ref = r_contract(x, art)
        assert float(np.abs(ref).max()) == pytest.approx(rec["ref_scale"], rel=1e-12, abs=0.0)
        for name, fault in FAULTS.items():
            want = rec["faults"][name]
            if want > 1e-3 * rec["ref_scale"]:
                got = _err(ENSEMBLE["dequant-pairwise"](x, fault(art)), ref)
                assert got == pytest.approx(want, rel=1e-3), name
