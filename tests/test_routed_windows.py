"""The routed windows: derived from the committed MI355X recording, pinned as
data (reference: tests/test_pack_routed_windows.py).

The table is the whole routing decision, so what is pinned is what makes a
silent change impossible: the derived cells against hand-written literals,
and the three things the cells are a claim about (the recording, the kernel
sources it priced, the launch config it ran at). Any of them moving fails
here rather than shipping a table that describes a kernel nobody measured.
"""

import copy
import json

import pytest

from kernelverify_amd.pack import routed_windows as rw
from kernelverify_amd.pack import wide_qmv
from tests.gates.price_qmv_boundary import classify

# Written out by hand from kernelverify_amd/pack/recordings/
# qmv-boundary-pricing-mi355x.json: the tile widths at which kvp_qmv beat the
# vendor fp16 GEMM with the whole ratio interval above 1 (every width runs on
# the matrix cores from M = 2 or 3), less any excluded islands (none in this recording).
EXPECTED_TABLE = {
    (2, 1024, 2560): range(1, 5), (2, 2560, 4096): range(1, 5), (2, 2560, 9728): range(1, 12),
    (2, 4096, 2560): range(1, 6), (2, 4096, 4096): range(1, 9), (2, 4096, 14336): range(1, 17),
    (2, 9728, 2560): range(1, 9), (2, 14336, 4096): range(1, 9), (2, 151936, 2560): range(1, 9),
    (3, 1024, 2560): range(1, 8), (3, 2560, 4096): range(1, 5), (3, 2560, 9728): range(1, 12),
    (3, 4096, 2560): range(1, 9), (3, 4096, 4096): range(1, 9), (3, 4096, 14336): range(1, 17),
    (3, 9728, 2560): range(1, 9), (3, 14336, 4096): range(1, 9), (3, 151936, 2560): range(1, 9),
    (4, 1024, 2560): range(1, 9), (4, 2560, 4096): range(1, 9), (4, 2560, 9728): range(1, 12),
    (4, 4096, 2560): range(1, 9), (4, 4096, 4096): range(1, 9), (4, 4096, 14336): range(1, 17),
    (4, 9728, 2560): range(1, 9), (4, 14336, 4096): range(1, 9), (4, 151936, 2560): range(1, 9),
    (8, 1024, 2560): range(1, 9), (8, 2560, 4096): range(1, 9), (8, 2560, 9728): range(1, 12),
    (8, 4096, 2560): range(1, 9), (8, 4096, 4096): range(1, 9), (8, 4096, 14336): range(1, 17),
    (8, 9728, 2560): range(1, 9), (8, 14336, 4096): range(1, 9), (8, 151936, 2560): range(1, 9),
}


def test_derived_table_matches_the_hand_written_cells():
    assert {k: set(v) for k, v in rw.ROUTED_WINDOWS.items()} == {
        k: set(v) for k, v in EXPECTED_TABLE.items()}


def test_windows_are_sets_and_contiguous_today():
    """Stored as sets (a hole is representable); this recording has none, so
    a hole in a later one is a finding to rule on, not something to ship."""
    for key, window in rw.ROUTED_WINDOWS.items():
        assert isinstance(window, frozenset)
        ms = sorted(window)
        assert ms == list(range(ms[0], ms[-1] + 1)), (key, ms)


def test_every_priced_shape_is_in_the_denominator():
    for bits in (2, 3, 4, 8):
        assert len(rw.PRICED_SHAPES[bits]) == 9
        assert (14336, 4096) in rw.PRICED_SHAPES[bits]


def test_pins_match_the_live_kernel_and_launch_config():
    """The recording priced these sources at this launch config; an edited
    kernel or a changed RW voids the windows until it is priced again."""
    assert rw.KERNEL_SOURCE_SHA256 == wide_qmv.kernel_source_sha256()
    for bits in (2, 3, 4, 8):
        for d_out, d_in in ((14336, 4096), (4096, 14336), (4096, 4096), (151936, 2560), (1024, 2560)):
            for m in range(1, 17):
                assert rw.rows_per_wave(m, bits, d_out, d_in) == wide_qmv.rows_per_wave(
                    m, bits, d_out, d_in), (bits, d_out, d_in, m)


def test_a_changed_device_flag_voids_the_pins(monkeypatch):
    """The digests cover how the kernels are compiled, not only their text:
    a flag that changes the machine code changes both pins, while include
    paths (which differ between machines) do not enter them."""
    from kernelverify_amd import build, counters
    kernel, library = wide_qmv.kernel_source_sha256(), counters.library_source_sha256()
    flags = list(build.DEVICE_FLAGS)
    monkeypatch.setattr(build, "DEVICE_FLAGS", [f for f in flags if not f.startswith("-I")]
                        + ["-I/elsewhere/include"])
    assert wide_qmv.kernel_source_sha256() == kernel
    assert counters.library_source_sha256() == library
    monkeypatch.setattr(build, "DEVICE_FLAGS", flags + ["-mllvm", "-amdgpu-kernarg-preload-count=0"])
    assert wide_qmv.kernel_source_sha256() != kernel
    assert counters.library_source_sha256() != library


def test_the_recording_is_read_only_as_its_pinned_bytes(tmp_path):
    changed = tmp_path / rw.RECORDING_PATH.name
    changed.write_bytes(rw.RECORDING_PATH.read_bytes() + b" ")
    with pytest.raises(ValueError, match="has changed"):
        rw._load(changed)
    assert rw._load()["probe"] == "price_qmv_boundary"


def _record():
    return copy.deepcopy(json.loads(rw.RECORDING_PATH.read_bytes()))


def test_derivation_refuses_a_foreign_kernel_or_launch_config():
    record = _record()
    record["kernel_source_sha256"] = "0" * 64
    with pytest.raises(ValueError, match="kernel sources"):
        rw._derive(record)
    record = _record()
    record["points"][0]["r"] = 4
    with pytest.raises(ValueError, match="RW="):
        rw._derive(record)


def test_only_win_with_an_interval_above_one_routes():
    record = _record()
    point = next(p for p in record["points"]
                 if (p["bits"], p["d_out"], p["d_in"], p["m"]) == (4, 14336, 4096, 1))
    for verdict, lo in (("LOSS", 0.9), ("REFUSED", 0.99), ("REJECTED", 1.2), ("WIN", 1.0)):
        point["verdict"], point["ratio_lo"] = verdict, lo
        _, windows = rw._derive(record)
        assert 1 not in windows[(4, 14336, 4096)]


def test_should_dispatch_reads_the_windows():
    assert wide_qmv.should_dispatch(1, 4, 14336, 4096)
    assert wide_qmv.should_dispatch(8, 4, 14336, 4096)
    assert not wide_qmv.should_dispatch(16, 4, 14336, 4096)   # measured LOSS
    assert wide_qmv.should_dispatch(8, 4, 151936, 2560)       # measured WIN, in the window
    assert wide_qmv.should_dispatch(8, 8, 151936, 2560)       # measured WIN, in the window
    assert wide_qmv.should_dispatch(5, 2, 9728, 2560)         # measured WIN, in the window
    assert not wide_qmv.should_dispatch(8, 3, 1024, 2560)     # measured LOSS
    assert not wide_qmv.should_dispatch(1, 4, 14336, 4097)    # never priced
    assert not wide_qmv.should_dispatch(1, 5, 14336, 4096)    # unpriced width
    with pytest.raises(TypeError):
        wide_qmv.should_dispatch(1, 4, 14336)                  # every argument required


def test_boundary_prose_names_the_routed_shapes():
    prose = rw.dispatch_boundary_prose(4, 1)
    assert "9 of the 9 priced shapes" in prose and rw.RECORDING_SHA256[:12] in prose
    assert "routes nowhere" in rw.dispatch_boundary_prose(5, 1)


def test_classify_is_the_interval_rule():
    assert classify([1e-6] * 7, [1.2e-6] * 7).verdict == "WIN"
    assert classify([1e-6] * 7, [0.8e-6] * 7).verdict == "LOSS"
    assert classify([1.0e-6, 1.1e-6], [1.05e-6, 1.06e-6]).verdict == "REFUSED"
    assert classify([1e-6] * 2, [1e-6, 1.6e-6]).verdict == "REJECTED"
