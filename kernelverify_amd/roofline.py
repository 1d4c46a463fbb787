"""Measured MI355X ceilings: the denominators the pack is scored against.

Re-targets the reference's ``bench/roofline.py`` + ``bench/metal/roofline_probe.mm``
(streaming read and copy GB/s, best-of repeats over large buffers) to HIP:
the probe kernels are ``kvp_probe_stream_read`` / ``kvp_probe_stream_copy``
in libkvpack, timed with HIP events.

Two read ceilings are reported, because the pack's kernels are small:
- ``read_large``: one launch streaming a buffer far larger than the 256 MB
  Infinity Cache (the asymptotic HBM read rate);
- ``read_like(nbytes)``: back-to-back launches each reading ``nbytes`` from a
  rotation of distinct buffers totalling >= 1 GiB, the same shape of work as
  one qmv or KV-decode call (includes per-launch ramp-up and drain).

Published spec: 8 TB/s HBM3E (SPECS below). "Score every backend against its
own ceiling" (the reference's rule): the bench reports both fractions.
"""

from __future__ import annotations

import numpy as np

from kernelverify_amd import hip, lib

SPECS = {
    "MI355X": {"hbm_GBps": 8000.0, "cus": 256, "xcds": 8, "infinity_cache_MB": 256,
               "valu_lane_ops_per_s": 256 * 4 * 16 * 2.4e9},
}


def _time_launches(fn, launches: int, stream) -> float:
    start, stop = hip.Event(), hip.Event()
    start.record(stream)
    for i in range(launches):
        fn(i)
    stop.record(stream)
    stop.synchronize()
    return start.elapsed_ms(stop) / launches


def read_large(nbytes: int = 2 << 30, blocks: int = 256 * 16, reps: int = 5) -> float:
    """Best GB/s of one read sweep over ``nbytes``."""
    L = lib.load()
    buf = hip.DeviceArray((nbytes,), np.uint8)
    buf.fill_byte(1)
    sink = hip.DeviceArray((blocks,), np.float32)
    stream = hip.Stream()
    best = float("inf")
    for _ in range(reps):
        ms = _time_launches(lambda i: lib.check(L.kvp_probe_stream_read(
            buf.ptr, nbytes, sink.ptr, blocks, stream.handle)), 1, stream)
        best = min(best, ms)
    return nbytes / (best * 1e-3) / 1e9


def copy_large(nbytes: int = 1 << 30, blocks: int = 256 * 16, reps: int = 5) -> float:
    """Best GB/s of one copy (bytes read + bytes written) over ``nbytes``."""
    L = lib.load()
    src = hip.DeviceArray((nbytes,), np.uint8)
    dst = hip.DeviceArray((nbytes,), np.uint8)
    src.fill_byte(1)
    stream = hip.Stream()
    best = float("inf")
    for _ in range(reps):
        ms = _time_launches(lambda i: lib.check(L.kvp_probe_stream_copy(
            src.ptr, dst.ptr, nbytes, blocks, stream.handle)), 1, stream)
        best = min(best, ms)
    return 2 * nbytes / (best * 1e-3) / 1e9


def read_like(nbytes: int, launches: int = 2000, blocks: int | None = None,
              rotation_bytes: int = 1 << 30) -> tuple[float, float]:
    """(GB/s, us per launch) of back-to-back reads of ``nbytes`` each."""
    L = lib.load()
    nbytes = (nbytes + 15) // 16 * 16
    copies = max(2, -(-rotation_bytes // nbytes))
    bufs = [hip.DeviceArray((nbytes,), np.uint8) for _ in range(copies)]
    for b in bufs:
        b.fill_byte(1)
    if blocks is None:
        blocks = max(256, min(256 * 16, nbytes // (256 * 16 * 4)))
    sink = hip.DeviceArray((blocks,), np.float32)
    stream = hip.Stream()
    run = lambda i: lib.check(L.kvp_probe_stream_read(bufs[i % copies].ptr, nbytes, sink.ptr,
                                                      blocks, stream.handle))
    _time_launches(run, 100, stream)
    # Replayed as one captured graph, like the pack's own timing.
    graph = hip.Graph(stream, lambda: [run(i) for i in range(launches)])
    graph.launch()
    stream.synchronize()
    ms = _time_launches(lambda i: graph.launch(), 1, stream) / launches
    graph.destroy()
    return nbytes / (ms * 1e-3) / 1e9, ms * 1e3


def measure(shapes=(33_067_008, 37_769_216, 9_453_568)) -> dict:
    """Ceilings as a dict (the reference writes bench/results/roofline.json)."""
    out = {"spec": SPECS["MI355X"], "read_large_GBps": read_large(),
           "copy_large_GBps": copy_large(), "read_like": {}}
    for n in shapes:
        gbs, us = read_like(n)
        out["read_like"][str(n)] = {"GBps": gbs, "us": us}
    return out


if __name__ == "__main__":
    import json
    import sys

    if "--copy-only" in sys.argv:
        # One 256 MiB copy: the calibration kernel for FETCH_SIZE/WRITE_SIZE.
        L = lib.load()
        n = 256 << 20
        src, dst = hip.DeviceArray((n,), np.uint8), hip.DeviceArray((n,), np.uint8)
        src.fill_byte(1)
        for _ in range(5):
            lib.check(L.kvp_probe_stream_copy(src.ptr, dst.ptr, n, 4096, None))
        hip.synchronize()
        print(json.dumps({"copy_bytes": n, "launches": 5}))
    else:
        print(json.dumps(measure(), indent=1))
