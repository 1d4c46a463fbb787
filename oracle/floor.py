"""The verdict formula every tolerance in the oracle is built on.

Follows vladmt06/kernelverify ``kernelverify/tolerance/floor.py:76-89``:
the fp64 max-abs metric and ``tol = max(base_tol, k * floor)``, where the
floor is the worst max-abs error of any legitimate working-precision member
against the fp64 reference.

Parity: closed form; pinned by tests/test_oracle_contract.py (empty input is
0.0, known differences, broadcast of a flat candidate).
"""

from __future__ import annotations

import numpy as np


def max_abs_error(candidate, ref) -> float:
    """fp64 max |candidate - ref|; 0.0 for an empty array."""
    diff = np.abs(np.asarray(candidate).astype(np.float64) - np.asarray(ref).astype(np.float64))
    return float(diff.max()) if diff.size else 0.0


def floored_tolerance(base_tol: float, k: float, member_outputs, ref) -> float:
    """max(base_tol, k * worst member error against ``ref``)."""
    return max(base_tol, k * max(max_abs_error(out, ref) for out in member_outputs))
