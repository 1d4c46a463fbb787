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


LOADS = {0: "plain", 1: "non-temporal", 2: "buffer"}


class _Rotation:
    """Distinct device buffers of ``nbytes`` each, totalling >= ``total``
    bytes (more than the 256 MB Infinity Cache), filled once."""

    def __init__(self, nbytes: int, total: int = 1 << 30):
        self.nbytes = (nbytes + 15) // 16 * 16
        self.copies = max(2, -(-total // self.nbytes))
        self.bufs = [hip.DeviceArray((self.nbytes,), np.uint8) for _ in range(self.copies)]
        for b in self.bufs:
            b.fill_byte(1)

    def ptr(self, i: int) -> int:
        return self.bufs[i % self.copies].ptr


def _graph_us(stream, launch_one, launches: int, replays: int = 3) -> float:
    """Best of ``replays`` timings of one captured graph of ``launches``
    back-to-back launches, in us per launch."""
    graph = hip.Graph(stream, lambda: [launch_one(i) for i in range(launches)])
    graph.launch()
    stream.synchronize()
    best = min(_time_launches(lambda i: graph.launch(), 1, stream) for _ in range(replays))
    graph.destroy()
    return best * 1e3 / launches


def read_tiled_us(rot: _Rotation, blocks: int, threads: int, unroll: int, flags: int,
                  stream, sink, launches: int = 200) -> float:
    L = lib.load()
    run = lambda i: lib.check(L.kvp_probe_read_tiled(rot.ptr(i), rot.nbytes, sink.ptr, blocks,
                                                     threads, unroll, flags, stream.handle))
    run(0)
    return _graph_us(stream, run, launches)


def sweep_read(nbytes: int, cus: int = 256, launches: int = 200) -> list[dict]:
    """Every probe shape for back-to-back reads of ``nbytes``: threads per
    block, blocks per CU, loads in flight per lane, load kind and tile order.
    Returns rows sorted fastest first."""
    rot = _Rotation(nbytes)
    stream = hip.Stream()
    sink = hip.DeviceArray((cus * 64,), np.float32)
    rows = []
    for threads in (256, 512, 1024):
        for per_cu in (1, 2, 4, 8):
            blocks = cus * per_cu
            if blocks * threads > cus * 2048:
                continue  # beyond the 32 waves a CU holds
            for unroll in (1, 2, 4, 8, 16):
                for kind in LOADS:
                    for contiguous in (0, 1):
                        flags = kind | (contiguous << 2)
                        us = read_tiled_us(rot, blocks, threads, unroll, flags, stream, sink,
                                           launches)
                        rows.append({"bytes": rot.nbytes, "threads": threads, "blocks": blocks,
                                     "unroll": unroll, "load": LOADS[kind],
                                     "tiles": "contiguous" if contiguous else "strided",
                                     "us": us, "GBps": rot.nbytes / (us * 1e-6) / 1e9})
    rows.sort(key=lambda r: r["us"])
    return rows


def best_read_like(nbytes: int, shapes: list[dict] | None = None,
                   launches: int = 1000) -> tuple[float, float, dict]:
    """(GB/s, us per launch, shape) of the fastest probe shape among
    ``shapes`` (default: LEADING_READ_SHAPES) for back-to-back reads of
    ``nbytes`` each: the measured ceiling for a call moving ``nbytes``."""
    rot = _Rotation(nbytes)
    stream = hip.Stream()
    best = None
    for shape in shapes or LEADING_READ_SHAPES:
        sink = hip.DeviceArray((shape["blocks"],), np.float32)
        flags = ({v: k for k, v in LOADS.items()}[shape["load"]]
                 | (4 if shape["tiles"] == "contiguous" else 0))
        us = read_tiled_us(rot, shape["blocks"], shape["threads"], shape["unroll"], flags,
                           stream, sink, launches)
        if best is None or us < best[1]:
            best = (rot.nbytes / (us * 1e-6) / 1e9, us, dict(shape))
    return best


# The leading shapes of sweep_read at the pack's call sizes on MI355X (the
# fastest at 9.45, 33.1 and 37.8 MB and the runners-up within 1% of them;
# profiles/roofline_ceilings_mi355x.md): non-temporal loads, tiles strided
# over the grid.
LEADING_READ_SHAPES = [
    {"threads": 512, "blocks": 1024, "unroll": 4, "load": "non-temporal", "tiles": "strided"},
    {"threads": 512, "blocks": 512, "unroll": 2, "load": "non-temporal", "tiles": "strided"},
    {"threads": 512, "blocks": 1024, "unroll": 1, "load": "non-temporal", "tiles": "strided"},
    {"threads": 256, "blocks": 2048, "unroll": 2, "load": "non-temporal", "tiles": "strided"},
    {"threads": 512, "blocks": 256, "unroll": 16, "load": "non-temporal", "tiles": "strided"},
    {"threads": 512, "blocks": 1024, "unroll": 2, "load": "non-temporal", "tiles": "contiguous"},
    {"threads": 1024, "blocks": 256, "unroll": 2, "load": "non-temporal", "tiles": "contiguous"},
]

COMPUTE_KINDS = {0: "fp32 FMA (v_fma_f32)", 1: "fp16 dot2 (v_dot2_f32_f16)",
                 2: "fp16 MFMA (v_mfma_f32_16x16x32_f16)"}


def compute_ceilings(blocks: int = 256 * 8, iters: int = 4096) -> dict:
    """Measured TFLOP/s of each compute probe (best of 5 single launches)."""
    L = lib.load()
    stream = hip.Stream()
    sink = hip.DeviceArray((blocks,), np.float32)
    out = {}
    for kind, name in COMPUTE_KINDS.items():
        run = lambda i: lib.check(L.kvp_probe_compute(kind, blocks, iters, sink.ptr, stream.handle))
        run(0)
        stream.synchronize()
        ms = min(_time_launches(run, 1, stream) for _ in range(5))
        flops = float(L.kvp_probe_compute_flops(kind, blocks, iters))
        out[name] = {"TFLOPs": flops / (ms * 1e-3) / 1e12, "ms": ms, "flops": flops}
    return out


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

    if "--sweep" in sys.argv:
        # The probe-shape sweep at the pack's call sizes, then the compute
        # probes: one JSON object per line, fastest shapes first.
        for n in (9_453_568, 33_067_008, 37_769_216):
            rows = sweep_read(n)
            print(json.dumps({"sweep_bytes": n, "configs": len(rows), "rows": rows}), flush=True)
        print(json.dumps({"compute": compute_ceilings()}), flush=True)
        print(json.dumps({"read_large_GBps": read_large(), "copy_large_GBps": copy_large()}),
              flush=True)
    elif "--copy-only" in sys.argv:
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
