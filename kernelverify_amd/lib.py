"""ctypes binding of libkvpack.so, the C ABI declared in include/kvpack.h.

Loading never falls back: a missing or unloadable library raises
``LibraryMissing``, because the product path has no CPU implementation.
Build it with ``python -m kernelverify_amd.build``.

Status codes become exceptions here, one class per runner status
(kernelverify/runners/result.py:67-74): ``InvalidArgument`` (INVALID_SPEC),
``Unsupported`` (UNSUPPORTED), ``LaunchError`` (LAUNCH_ERROR), ``NoDevice``.
"""

from __future__ import annotations

import ctypes
from functools import lru_cache
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libkvpack.so"

KVP_OK, KVP_INVALID, KVP_UNSUPPORTED, KVP_LAUNCH_ERROR, KVP_NO_DEVICE = 0, -1, -2, -3, -4
KVP_F16, KVP_F32 = 1, 2


class KvpError(RuntimeError):
    status = None


class InvalidArgument(KvpError, ValueError):
    status = KVP_INVALID


class Unsupported(KvpError):
    status = KVP_UNSUPPORTED


class LaunchError(KvpError):
    status = KVP_LAUNCH_ERROR


class NoDevice(KvpError):
    status = KVP_NO_DEVICE


class LibraryMissing(RuntimeError):
    pass


_ERRORS = {c.status: c for c in (InvalidArgument, Unsupported, LaunchError, NoDevice)}

_vp, _sz, _i = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
_cp = ctypes.c_char_p
_ip = ctypes.POINTER(ctypes.c_int)
_szp = ctypes.POINTER(ctypes.c_size_t)

# name -> (restype, argtypes); the same order as include/kvpack.h.
SIGNATURES = {
    "kvp_version": (_cp, []),
    "kvp_last_error": (_sz, [_cp, _sz]),
    "kvp_device_info": (_i, [_i, _cp, _sz, _cp, _sz, _ip, _ip, _szp, _szp, _ip]),
    "kvp_quantize_affine": (_i, [_vp, _i, _i, _i, _vp, _vp, _vp, _vp]),
    "kvp_qmv": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp]),
    "kvp_kv_decode_workspace_bytes": (_sz, [_i, _i, _i, _i, _i]),
    "kvp_kv_decode": (_i, [_vp] * 11 + [_i] * 9 + [_vp, _sz, _vp]),
    "kvp_kv_decode_static_scratch_bytes": (_sz, []),
    "kvp_kv_decode_static": (_i, [_vp] * 11 + [_i] * 9 + [_vp]),
    "kvp_moe_route": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "kvp_moe_route_logits": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "kvp_moe_permute": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "kvp_moe_dispatch": (_i, [_vp] * 7 + [_i] * 7 + [_vp]),
    "kvp_moe_swiglu_workspace_bytes": (_sz, [_i] * 5),
    "kvp_moe_swiglu": (_i, [_vp] * 13 + [_i] * 7 + [_vp, _sz, _vp]),
    "kvp_moe_route_swiglu": (_i, [_vp] * 14 + [_i] * 7 + [_vp, _sz, _vp]),
    "kvp_set_tuning": (_i, [_cp, _i]),
    "kvp_get_tuning": (_i, [_cp, _ip]),
    "kvp_probe_stream_read": (_i, [_vp, _sz, _vp, _i, _vp]),
    "kvp_probe_stream_copy": (_i, [_vp, _vp, _sz, _i, _vp]),
    "kvp_probe_read_tiled": (_i, [_vp, _sz, _vp, _i, _i, _i, _i, _vp]),
    "kvp_probe_compute_flops": (ctypes.c_double, [_i, _i, _i]),
    "kvp_probe_compute": (_i, [_i, _i, _i, _vp, _vp]),
}


@lru_cache(maxsize=1)
def load() -> ctypes.CDLL:
    if not LIB_PATH.exists():
        raise LibraryMissing(
            f"{LIB_PATH} is not built; run `python -m kernelverify_amd.build` "
            "(the pack has no CPU fallback)")
    try:
        lib = ctypes.CDLL(str(LIB_PATH))
    except OSError as exc:
        raise LibraryMissing(f"cannot load {LIB_PATH}: {exc}") from exc
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def last_error() -> str:
    lib = load()
    n = lib.kvp_last_error(None, 0)
    buf = ctypes.create_string_buffer(n + 1)
    lib.kvp_last_error(buf, n + 1)
    return buf.value.decode(errors="replace")


def check(status: int) -> None:
    if status != KVP_OK:
        cls = _ERRORS.get(status, KvpError)
        raise cls(last_error() or f"libkvpack status {status}")


def set_tuning(key: str, value: int) -> None:
    """Override one kernel-selection choice (-1 restores the library's);
    see include/kvpack.h kvp_set_tuning."""
    check(load().kvp_set_tuning(key.encode(), int(value)))


def get_tuning(key: str) -> int:
    v = ctypes.c_int()
    check(load().kvp_get_tuning(key.encode(), ctypes.byref(v)))
    return v.value


def version() -> str:
    return load().kvp_version().decode()


def exported_symbols() -> list[str]:
    """Every name of SIGNATURES that the loaded library resolves."""
    lib = load()
    return [n for n in SIGNATURES if hasattr(lib, n)]
