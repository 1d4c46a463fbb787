"""HIP C++ candidate kernels: compiled at run time with hiprtc for gfx950.

The reference runner compiles each candidate's Metal source once and
dispatches it over a batch (kernelverify/runners/device.py:134-166,
:266-315). Here: hiprtc builds the source into a gfx950 code object with the
library's own device flags (packed fp32 off), hipModuleLoadData loads it, and
hipModuleLaunchKernel launches `entry_point` with the bindings as its
arguments in buffer-index order: a device pointer per tensor, the scalar
value per scalar binding (4 bytes; fp16 in the low half). Entry points must
be `extern "C" __global__` so the name is not mangled.
"""

from __future__ import annotations

import ctypes
from functools import lru_cache

import numpy as np

from kernelverify_amd import hip
from kernelverify_amd.hip import DeviceArray
from kernelverify_amd.runners.spec import (
    SCALAR_DTYPES,
    BindingKind,
    KernelSpec,
    LaunchMode,
    RunCase,
    SpecError,
)

ARCH = "gfx950"
OPTIONS = (f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-ffp-contract=fast",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops")
MAX_THREADS_PER_BLOCK = 1024


class CompileError(RuntimeError):
    """hiprtc rejected the source; the message carries its log."""


@lru_cache(maxsize=1)
def _hiprtc() -> ctypes.CDLL:
    for name in ("libhiprtc.so", "libhiprtc.so.7", "/opt/rocm/lib/libhiprtc.so"):
        try:
            rtc = ctypes.CDLL(name)
            break
        except OSError:
            continue
    else:
        raise CompileError("hiprtc is not loadable on this machine")
    vp, sz = ctypes.c_void_p, ctypes.c_size_t
    rtc.hiprtcCreateProgram.argtypes = [ctypes.POINTER(vp), ctypes.c_char_p, ctypes.c_char_p,
                                        ctypes.c_int, vp, vp]
    rtc.hiprtcCompileProgram.argtypes = [vp, ctypes.c_int, ctypes.POINTER(ctypes.c_char_p)]
    rtc.hiprtcGetProgramLogSize.argtypes = [vp, ctypes.POINTER(sz)]
    rtc.hiprtcGetProgramLog.argtypes = [vp, ctypes.c_char_p]
    rtc.hiprtcGetCodeSize.argtypes = [vp, ctypes.POINTER(sz)]
    rtc.hiprtcGetCode.argtypes = [vp, ctypes.c_char_p]
    rtc.hiprtcDestroyProgram.argtypes = [ctypes.POINTER(vp)]
    for fn in ("hiprtcCreateProgram", "hiprtcCompileProgram", "hiprtcGetProgramLogSize",
               "hiprtcGetProgramLog", "hiprtcGetCodeSize", "hiprtcGetCode",
               "hiprtcDestroyProgram"):
        getattr(rtc, fn).restype = ctypes.c_int
    return rtc


def compile_source(source: str, name: str = "candidate.hip") -> bytes:
    """gfx950 code object for `source`; CompileError with hiprtc's log."""
    rtc = _hiprtc()
    prog = ctypes.c_void_p()
    if rtc.hiprtcCreateProgram(ctypes.byref(prog), source.encode(), name.encode(), 0, None, None):
        raise CompileError("hiprtcCreateProgram failed")
    try:
        opts = (ctypes.c_char_p * len(OPTIONS))(*(o.encode() for o in OPTIONS))
        status = rtc.hiprtcCompileProgram(prog, len(OPTIONS), opts)
        n = ctypes.c_size_t(0)
        rtc.hiprtcGetProgramLogSize(prog, ctypes.byref(n))
        log = ctypes.create_string_buffer(max(n.value, 1))
        rtc.hiprtcGetProgramLog(prog, log)
        if status != 0:
            raise CompileError(log.value.decode(errors="replace") or f"hiprtc status {status}")
        rtc.hiprtcGetCodeSize(prog, ctypes.byref(n))
        code = ctypes.create_string_buffer(n.value)
        if rtc.hiprtcGetCode(prog, code):
            raise CompileError("hiprtcGetCode failed")
        return code.raw
    finally:
        rtc.hiprtcDestroyProgram(ctypes.byref(prog))


class Module:
    """A loaded code object and one function in it."""

    def __init__(self, code: bytes, entry_point: str):
        rt = hip.runtime()
        self._code = ctypes.create_string_buffer(code, len(code))
        self.handle = ctypes.c_void_p()
        hip.check(rt.hipModuleLoadData(ctypes.byref(self.handle), self._code), "hipModuleLoadData")
        self.function = ctypes.c_void_p()
        err = rt.hipModuleGetFunction(ctypes.byref(self.function), self.handle,
                                      entry_point.encode())
        if err:
            rt.hipGetLastError()  # the failed lookup's error is reported here, not later
            self.unload()
            raise CompileError(f"entry point {entry_point!r} not found in the code object "
                               "(declare it extern \"C\" __global__)")

    def unload(self) -> None:
        if self.handle:
            hip.runtime().hipModuleUnload(self.handle)
            self.handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.unload()
        except Exception:  # pragma: no cover - interpreter shutdown
            pass


def _scalar_bytes(value, dtype: str) -> ctypes.c_uint32:
    arr = np.asarray(value, dtype=SCALAR_DTYPES[dtype]).reshape(1)
    raw = arr.tobytes().ljust(4, b"\0")
    return ctypes.c_uint32(int.from_bytes(raw[:4], "little"))


class BoundKernel:
    """Device copies of a case's inputs, its output buffers, and the packed
    kernel arguments; `launch(stream)` returns a HIP status."""

    def __init__(self, module: Module, spec: KernelSpec, case: RunCase):
        grid, block, memory = spec.launch.resolve(case.params)
        if int(np.prod(block)) > MAX_THREADS_PER_BLOCK:
            raise SpecError(f"threadgroup {block} exceeds {MAX_THREADS_PER_BLOCK} threads")
        if spec.launch.mode is LaunchMode.THREADS:
            blocks = tuple(-(-g // t) for g, t in zip(grid, block))
        else:
            blocks = grid
        self.blocks, self.block = blocks, block
        self.shared = int(memory[0]) if memory else 0
        self.module = module
        by_index, self.outputs, self._keep = {}, [], []
        out_k = 0
        for position, binding in enumerate(spec.bindings):
            index = spec.buffer_index(position)
            if binding.kind is BindingKind.INPUT:
                arr = DeviceArray.from_host(np.ascontiguousarray(case.inputs[binding.name]))
                self._keep.append(arr)
                by_index[index] = ctypes.c_void_p(arr.ptr)
            elif binding.kind is BindingKind.OUTPUT:
                shape, dtype = case.output_shapes[out_k]
                out_k += 1
                arr = DeviceArray.zeros(shape, dtype)
                self.outputs.append(arr)
                by_index[index] = ctypes.c_void_p(arr.ptr)
            else:
                by_index[index] = _scalar_bytes(case.params[binding.name], binding.dtype)
        self._args = [by_index[i] for i in sorted(by_index)]
        self._ptrs = (ctypes.c_void_p * len(self._args))(
            *(ctypes.cast(ctypes.byref(a), ctypes.c_void_p) for a in self._args))

    def launch(self, stream) -> int:
        return hip.runtime().hipModuleLaunchKernel(
            self.module.function, *self.blocks, *self.block, self.shared, stream,
            self._ptrs, None)
