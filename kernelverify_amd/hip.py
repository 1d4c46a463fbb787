"""Minimal ctypes bindings to the HIP runtime (libamdhip64).

Device memory, copies, streams and events: what the host side of the pack
needs to hand device pointers to libkvpack and time it. No torch: the runner
worker and the bench both run on these calls alone.

Every call checks its hipError_t and raises ``HipError`` with the runtime's
own message.
"""

from __future__ import annotations

import ctypes
import os
from functools import lru_cache

import numpy as np

HIP_MEMCPY_H2D = 1
HIP_MEMCPY_D2H = 2
HIP_MEMCPY_D2D = 3


class HipError(RuntimeError):
    pass


@lru_cache(maxsize=1)
def runtime() -> ctypes.CDLL:
    names = ("libamdhip64.so", "libamdhip64.so.7", "/opt/rocm/lib/libamdhip64.so")
    last = None
    for name in names:
        try:
            lib = ctypes.CDLL(name)
            break
        except OSError as exc:  # pragma: no cover - depends on the image
            last = exc
    else:
        raise HipError(f"HIP runtime not loadable: {last}")
    vp, sz, i = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
    sigs = {
        "hipGetDeviceCount": [ctypes.POINTER(i)],
        "hipSetDevice": [i],
        "hipGetDevice": [ctypes.POINTER(i)],
        "hipMalloc": [ctypes.POINTER(vp), sz],
        "hipFree": [vp],
        "hipMemcpy": [vp, vp, sz, i],
        "hipMemcpyAsync": [vp, vp, sz, i, vp],
        "hipMemsetAsync": [vp, i, sz, vp],
        "hipMemset": [vp, i, sz],
        "hipDeviceSynchronize": [],
        "hipStreamCreate": [ctypes.POINTER(vp)],
        "hipStreamDestroy": [vp],
        "hipStreamSynchronize": [vp],
        "hipEventCreate": [ctypes.POINTER(vp)],
        "hipEventDestroy": [vp],
        "hipEventRecord": [vp, vp],
        "hipEventRecordWithFlags": [vp, vp, ctypes.c_uint],
        "hipEventSynchronize": [vp],
        "hipEventQuery": [vp],
        "hipEventElapsedTime": [ctypes.POINTER(ctypes.c_float), vp, vp],
        "hipGetLastError": [],
        "hipMemGetInfo": [ctypes.POINTER(sz), ctypes.POINTER(sz)],
        "hipStreamBeginCapture": [vp, i],
        "hipStreamEndCapture": [vp, ctypes.POINTER(vp)],
        "hipGraphInstantiate": [ctypes.POINTER(vp), vp, vp, ctypes.c_char_p, sz],
        "hipGraphLaunch": [vp, vp],
        "hipGraphExecDestroy": [vp],
        "hipGraphDestroy": [vp],
        # module API: run-time compiled kernels (kernelverify_amd/runners/rtc.py)
        "hipModuleLoadData": [ctypes.POINTER(vp), vp],
        "hipModuleGetFunction": [ctypes.POINTER(vp), vp, ctypes.c_char_p],
        "hipModuleLaunchKernel": [vp, ctypes.c_uint, ctypes.c_uint, ctypes.c_uint, ctypes.c_uint,
                                  ctypes.c_uint, ctypes.c_uint, ctypes.c_uint, vp,
                                  ctypes.POINTER(vp), ctypes.POINTER(vp)],
        "hipModuleUnload": [vp],
    }
    for name, args in sigs.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = ctypes.c_int
    lib.hipGetErrorString.argtypes = [ctypes.c_int]
    lib.hipGetErrorString.restype = ctypes.c_char_p
    return lib


def check(err: int, what: str) -> None:
    if err != 0:
        rt = runtime()
        rt.hipGetLastError()  # consumed here, so no later launch check reports it
        msg = rt.hipGetErrorString(err).decode(errors="replace")
        raise HipError(f"{what}: {msg} (hipError {err})")


def device_count() -> int:
    """Visible HIP devices; 0 when the runtime or driver is absent."""
    if os.environ.get("KV_FORCE_NO_GPU") == "1":
        return 0
    try:
        n = ctypes.c_int(0)
        if runtime().hipGetDeviceCount(ctypes.byref(n)) != 0:
            return 0
        return n.value
    except (HipError, OSError):
        return 0


def synchronize() -> None:
    check(runtime().hipDeviceSynchronize(), "hipDeviceSynchronize")


def malloc(nbytes: int) -> int:
    ptr = ctypes.c_void_p()
    check(runtime().hipMalloc(ctypes.byref(ptr), max(int(nbytes), 1)), f"hipMalloc({nbytes})")
    return ptr.value


def free(ptr: int) -> None:
    if ptr:
        check(runtime().hipFree(ctypes.c_void_p(ptr)), "hipFree")


def mem_info() -> tuple[int, int]:
    free_b, total = ctypes.c_size_t(), ctypes.c_size_t()
    check(runtime().hipMemGetInfo(ctypes.byref(free_b), ctypes.byref(total)), "hipMemGetInfo")
    return free_b.value, total.value


class DeviceArray:
    """A device allocation with a numpy shape and dtype; frees itself."""

    def __init__(self, shape, dtype, ptr: int | None = None):
        self.shape = tuple(int(d) for d in shape)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        self._owned = ptr is None
        self.ptr = malloc(self.nbytes) if ptr is None else ptr

    @classmethod
    def from_host(cls, array: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(array)
        dev = cls(a.shape, a.dtype)
        if a.nbytes:
            check(runtime().hipMemcpy(ctypes.c_void_p(dev.ptr), a.ctypes.data_as(ctypes.c_void_p),
                                      a.nbytes, HIP_MEMCPY_H2D), "hipMemcpy H2D")
        return dev

    @classmethod
    def zeros(cls, shape, dtype) -> "DeviceArray":
        dev = cls(shape, dtype)
        dev.fill_zero()
        return dev

    def fill_zero(self) -> None:
        if self.nbytes:
            check(runtime().hipMemset(ctypes.c_void_p(self.ptr), 0, self.nbytes), "hipMemset")

    def fill_byte(self, value: int) -> None:
        if self.nbytes:
            check(runtime().hipMemset(ctypes.c_void_p(self.ptr), int(value) & 0xFF, self.nbytes),
                  "hipMemset")

    def to_host(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        if out.nbytes:
            check(runtime().hipMemcpy(out.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(self.ptr),
                                      out.nbytes, HIP_MEMCPY_D2H), "hipMemcpy D2H")
        return out

    def copy_from(self, array: np.ndarray) -> None:
        a = np.ascontiguousarray(array, dtype=self.dtype)
        if a.nbytes != self.nbytes:
            raise ValueError(f"copy_from: {a.nbytes} bytes into a {self.nbytes}-byte buffer")
        check(runtime().hipMemcpy(ctypes.c_void_p(self.ptr), a.ctypes.data_as(ctypes.c_void_p),
                                  a.nbytes, HIP_MEMCPY_H2D), "hipMemcpy H2D")

    def free(self) -> None:
        if self._owned and self.ptr:
            free(self.ptr)
        self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:  # interpreter shutdown
            pass

    def __repr__(self) -> str:
        return f"DeviceArray(shape={self.shape}, dtype={self.dtype}, ptr=0x{self.ptr:x})"


class Stream:
    """A default-priority HIP stream."""

    def __init__(self):
        handle = ctypes.c_void_p()
        check(runtime().hipStreamCreate(ctypes.byref(handle)), "hipStreamCreate")
        self.handle = handle.value

    def synchronize(self) -> None:
        check(runtime().hipStreamSynchronize(ctypes.c_void_p(self.handle)), "hipStreamSynchronize")

    def destroy(self) -> None:
        if self.handle:
            runtime().hipStreamDestroy(ctypes.c_void_p(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class Event:
    def __init__(self):
        handle = ctypes.c_void_p()
        check(runtime().hipEventCreate(ctypes.byref(handle)), "hipEventCreate")
        self.handle = handle.value

    def record(self, stream: Stream | None = None) -> None:
        s = ctypes.c_void_p(stream.handle if stream else None)
        check(runtime().hipEventRecord(ctypes.c_void_p(self.handle), s), "hipEventRecord")

    def record_external(self, stream: Stream) -> None:
        """Record on ``stream``; under stream capture this becomes an event
        record node of the graph (hipEventRecordExternal), so a replay
        stamps the event on the device between the nodes around it."""
        check(runtime().hipEventRecordWithFlags(ctypes.c_void_p(self.handle),
                                                ctypes.c_void_p(stream.handle),
                                                HIP_EVENT_RECORD_EXTERNAL),
              "hipEventRecordWithFlags")

    def synchronize(self) -> None:
        check(runtime().hipEventSynchronize(ctypes.c_void_p(self.handle)), "hipEventSynchronize")

    def query(self) -> bool:
        """True once the work before the record has completed (no wait)."""
        err = runtime().hipEventQuery(ctypes.c_void_p(self.handle))
        if err == HIP_ERROR_NOT_READY:
            return False
        check(err, "hipEventQuery")
        return True

    def wait_until(self, deadline: float, poll_s: float = 2e-4) -> bool:
        """Poll until the event completes or the host clock
        (``time.perf_counter``) passes ``deadline``; True if it completed."""
        import time

        while not self.query():
            if time.perf_counter() > deadline:
                return False
            time.sleep(poll_s)
        return True

    def elapsed_ms(self, later: "Event") -> float:
        ms = ctypes.c_float()
        check(runtime().hipEventElapsedTime(ctypes.byref(ms), ctypes.c_void_p(self.handle),
                                            ctypes.c_void_p(later.handle)), "hipEventElapsedTime")
        return float(ms.value)

    def __del__(self):
        try:
            if self.handle:
                runtime().hipEventDestroy(ctypes.c_void_p(self.handle))
        except Exception:
            pass


HIP_STREAM_CAPTURE_RELAXED = 2
HIP_EVENT_RECORD_EXTERNAL = 1
HIP_ERROR_NOT_READY = 600


class Graph:
    """A captured sequence of launches on one stream, replayed as one graph.

    ``Graph(stream, fn)`` calls ``fn()`` while ``stream`` is in capture mode
    (every kernel ``fn`` enqueues on that stream becomes a node), then
    instantiates the graph. ``launch()`` replays it on the same stream. The
    pack's calls allocate nothing and record no memset, so they capture.
    """

    def __init__(self, stream: Stream, fn):
        self.stream = stream
        rt = runtime()
        check(rt.hipStreamBeginCapture(ctypes.c_void_p(stream.handle),
                                       HIP_STREAM_CAPTURE_RELAXED), "hipStreamBeginCapture")
        graph = ctypes.c_void_p()
        try:
            fn()
        finally:
            check(rt.hipStreamEndCapture(ctypes.c_void_p(stream.handle), ctypes.byref(graph)),
                  "hipStreamEndCapture")
        self.graph = graph.value
        exe = ctypes.c_void_p()
        check(rt.hipGraphInstantiate(ctypes.byref(exe), ctypes.c_void_p(self.graph), None, None,
                                     0), "hipGraphInstantiate")
        self.exec = exe.value

    def launch(self) -> None:
        check(runtime().hipGraphLaunch(ctypes.c_void_p(self.exec),
                                       ctypes.c_void_p(self.stream.handle)), "hipGraphLaunch")

    def destroy(self) -> None:
        rt = runtime()
        if getattr(self, "exec", None):
            rt.hipGraphExecDestroy(ctypes.c_void_p(self.exec))
            self.exec = None
        if getattr(self, "graph", None):
            rt.hipGraphDestroy(ctypes.c_void_p(self.graph))
            self.graph = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass
