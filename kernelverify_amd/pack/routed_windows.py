"""Where the qmv kernel is routed: per shape, per bit width, from measurement
(reference: kernelverify/pack/routed_windows.py:1-180).

`wide_qmv.should_dispatch(m, bits, d_out, d_in)` asks one question: is M in
the set of tile widths a recording measured the pack winning at, for this
(bits, d_out, d_in)? The table is keyed by the whole cell and holds SETS of
winning widths (a set can represent a hole; a (lo, hi) pair cannot). It is
derived at import from a committed recording made on MI355X by
`tests/gates/price_qmv_boundary.py`, which times `kvp_qmv` against the
vendor fp16 GEMM on the same layer in interleaved rounds and classifies
each cell WIN / LOSS / REFUSED / REJECTED by its ratio interval.

A window is a claim about ONE kernel body at ONE launch config from ONE
recording, so all three are pinned below as literals:

- RECORDING_SHA256, checked at import: a re-run over the same file cannot
  silently re-derive the table;
- KERNEL_SOURCE_SHA256, the kernel sources the recording priced (the
  recording states it too, and the derivation refuses a mismatch; the tests
  re-hash the live sources against it);
- ROWS_PER_WAVE, the launch config at every priced width (every point is
  checked against it at import; the tests check wide_qmv against it).

A cell routes only when it was judged WIN with ratio_lo > 1 on a round whose
incumbent arm held steady. LOSS, REFUSED (undecided) and REJECTED (the clock
moved) route nowhere; neither does any shape or width the recording did not
price.

This module imports nothing from the package (wide_qmv consults it).
"""

from __future__ import annotations

import hashlib
import json
from pathlib import Path
from types import MappingProxyType

RECORDING_PATH = Path(__file__).resolve().parent / "recordings" / "qmv-boundary-pricing-mi355x.json"

RECORDING_SHA256 = "43d6d8319016d9c21c7c62e39814875b2c51e655dedb12956ad0a3245d198f47"

KERNEL_SOURCE_SHA256 = "c76bffa3f639c2decd6d9368ee004ca621424f6bbda8ad245185f1c1e9b54e50"

ROWS_PER_WAVE = MappingProxyType({m: (2 if m <= 8 else 1) for m in range(1, 17)})


def rows_per_wave(m: int, bits: int, d_out: int, d_in: int) -> int:
    """The pinned launch config of a priced cell."""
    return ROWS_PER_WAVE[m]

# Cells measured WIN but not routed, with the reason. A window only admits
# cells contiguous with its lower part: a WIN above a measured LOSS is an
# island, not a window edge, and is listed here as {(bits, d_out, d_in):
# frozenset of M}. This recording has none (every window is contiguous).
EXCLUDED_CELLS = MappingProxyType({})


def _load(path: Path = RECORDING_PATH, pinned: str | None = None) -> dict:
    """The recording, refusing to be read as anything but the pinned bytes."""
    raw = path.read_bytes()
    digest = hashlib.sha256(raw).hexdigest()
    pinned = RECORDING_SHA256 if pinned is None else pinned
    if digest != pinned:
        raise ValueError(
            f"{path.name} has changed (sha256 {digest}, pinned {pinned}): the routed "
            "windows describe the pinned recording, so re-derive and re-pin deliberately")
    return json.loads(raw)


def _derive(record: dict, kernel_sha: str | None = None) -> tuple[dict, dict]:
    """(priced shapes per bit width, routed cells) read out of the recording."""
    kernel_sha = KERNEL_SOURCE_SHA256 if kernel_sha is None else kernel_sha
    if record.get("kernel_source_sha256") != kernel_sha:
        raise ValueError("the recording priced kernel sources "
                         f"{record.get('kernel_source_sha256')}, the pin is {kernel_sha}: "
                         "its windows describe a kernel that is not this one")
    shapes: dict[int, list] = {}
    windows: dict[tuple[int, int, int], set] = {}
    for point in record["points"]:
        m, r, bits = point["m"], point["r"], point["bits"]
        pinned_rw = rows_per_wave(m, bits, point["d_out"], point["d_in"]) if m in ROWS_PER_WAVE else None
        if pinned_rw != r:
            raise ValueError(f"{point['site']} {bits}-bit M={m} was priced at RW={r}, but the "
                             f"pinned launch config is RW={pinned_rw}")
        shape = (point["d_out"], point["d_in"])
        if shape not in shapes.setdefault(bits, []):
            shapes[bits].append(shape)
        window = windows.setdefault((bits, *shape), set())
        if point["verdict"] == "WIN" and point["ratio_lo"] > 1.0:
            window.add(m)
    for key, excluded in EXCLUDED_CELLS.items():
        if key not in windows:
            raise ValueError(f"cell {key} is excluded, but the recording did not price it")
        windows[key] -= set(excluded)
    return ({bits: tuple(v) for bits, v in shapes.items()},
            {key: frozenset(ms) for key, ms in windows.items() if ms})


_RECORD = _load()
RECORDING_DATE = _RECORD["date"]
_PRICED_SHAPES, _WINDOWS = _derive(_RECORD)

# Every (d_out, d_in) priced, per bit width, won anywhere or not: the
# denominator of any "routed at N shapes" statement.
PRICED_SHAPES = MappingProxyType(_PRICED_SHAPES)
ROUTED_WINDOWS = MappingProxyType(_WINDOWS)

PROVENANCE = (f"kernelverify_amd/pack/recordings/{RECORDING_PATH.name} ({RECORDING_DATE}, "
              f"sha256 {RECORDING_SHA256[:12]}, {_RECORD['machine']['arch']})")


def window_for(bits: int, d_out: int, d_in: int) -> frozenset:
    """The tile widths measured profitable at this cell; empty for a shape or
    width never priced (no evidence is not a default)."""
    return ROUTED_WINDOWS.get((bits, d_out, d_in), frozenset())


def dispatch_boundary_prose(bits: int, m: int) -> str:
    """One sentence stating where this (bits, M) specialization is routed
    (reference: routed_windows.py:157-180), for a certificate emitter."""
    head = "should_dispatch(m, bits, d_out, d_in) is per-shape and per-width"
    tail = ("a routing boundary, not a correctness bound: the correctness claim holds "
            "wherever this specialization is launched")
    shapes = PRICED_SHAPES.get(bits, ())
    if not shapes:
        return (f"{head}: {bits}-bit is unpriced, so it routes nowhere and the vendor GEMM "
                f"serves every shape at this width; {tail}")
    routed = [f"{d_out}x{d_in}" for d_out, d_in in shapes if m in window_for(bits, d_out, d_in)]
    where = (f"{len(routed)} of the {len(shapes)} priced shapes ({', '.join(routed)})"
             if routed else f"none of the {len(shapes)} priced shapes")
    return (f"{head}: at BITS={bits}, M={m} it routes here at {where} and nowhere else, "
            f"per {PROVENANCE}; {tail}")
