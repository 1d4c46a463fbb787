"""Shared pytest configuration.

Three tiers, as in the reference suite (``tests/conftest.py:31-61``):
CPU oracle tests run anywhere; HIP tests carry the ``gpu`` marker and skip
when no device answers; runner fault tests force failures from the host.
"""

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")
    config.addinivalue_line("markers", "slow: long CPU oracle sweeps")


def _device_count() -> int:
    """HIP devices visible to this process, without initialising torch's CUDA
    state in the parent (a ctypes call into the HIP runtime)."""
    if os.environ.get("KV_FORCE_NO_GPU") == "1":
        return 0
    try:
        import ctypes

        hip = ctypes.CDLL("libamdhip64.so")
        n = ctypes.c_int(0)
        if hip.hipGetDeviceCount(ctypes.byref(n)) != 0:
            return 0
        return n.value
    except OSError:
        return 0


HIP_DEVICES = _device_count()

requires_gpu = pytest.mark.skipif(HIP_DEVICES == 0, reason="no HIP device")


def pytest_collection_modifyitems(config, items):
    for item in items:
        if "gpu" in item.keywords and HIP_DEVICES == 0:
            item.add_marker(pytest.mark.skip(reason="no HIP device visible"))
