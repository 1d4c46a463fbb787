"""Pack-library specs: a `KernelSpec` whose source is ``kvpack:<entry> K=V ...``.

The reference's pack modules hand the runner raw kernel source templates
(kernelverify/pack/wide_qmv.py:218-260, kv_attention.py:292-352,
moe_dispatch.py:161-234). Here the kernels are the prebuilt libkvpack entry
points, so a pack template is a descriptor: the entry family and its
compile-time constants (the same `$T $BITS $M $R ...` the reference's
templates carry), filled by `specialize`. The bindings keep the reference's
names and order, so a `RunCase` written for the reference door binds here.

Each family below turns (descriptor constants, case) into a bound call:
device copies of the inputs, output buffers, and a zero-argument launcher
on a stream. Shape and constant mismatches are `SpecError`s (INVALID_SPEC,
nothing runs); library status codes become LAUNCH_ERROR / UNSUPPORTED.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from kernelverify_amd import lib
from kernelverify_amd.hip import DeviceArray
from kernelverify_amd.runners.spec import LIBRARY_PREFIX, BindingKind, KernelSpec, RunCase, SpecError

_T = {"half": ("float16", lib.KVP_F16), "float16": ("float16", lib.KVP_F16),
      "float": ("float32", lib.KVP_F32), "float32": ("float32", lib.KVP_F32)}


def parse_descriptor(source: str) -> tuple[str, dict]:
    """``kvpack:<family> K=V K=V`` -> (family, {K: V})."""
    text = source.strip()
    if not text.startswith(LIBRARY_PREFIX):
        raise SpecError("not a pack-library descriptor")
    parts = text[len(LIBRARY_PREFIX):].split()
    if not parts:
        raise SpecError("pack-library descriptor names no entry")
    consts = {}
    for item in parts[1:]:
        if "=" not in item:
            raise SpecError(f"descriptor item {item!r} is not NAME=value")
        k, v = item.split("=", 1)
        consts[k] = v
    return parts[0], consts


def _int(consts: dict, key: str) -> int:
    try:
        return int(consts[key])
    except (KeyError, ValueError) as error:
        raise SpecError(f"descriptor constant {key} missing or not an integer") from error


def _dtype_of(consts: dict) -> tuple[str, int]:
    t = consts.get("T", "half")
    if t not in _T:
        raise SpecError(f"T={t!r}: the library writes half or float outputs")
    return _T[t]


@dataclass
class BoundCall:
    """Device state of one case and the launcher that runs it."""

    launch: object            # callable(stream_handle) -> int status
    outputs: list             # DeviceArray per output binding
    keep: tuple = ()


def _named(spec: KernelSpec, case: RunCase):
    """Inputs and scalars by binding name; output slots in binding order."""
    inputs, scalars = {}, {}
    for b in spec.bindings:
        if b.kind is BindingKind.INPUT:
            inputs[b.name] = np.ascontiguousarray(case.inputs[b.name])
        elif b.kind is BindingKind.SCALAR:
            scalars[b.name] = case.params[b.name]
    return inputs, scalars


def _need(inputs: dict, names) -> None:
    missing = [n for n in names if n not in inputs]
    if missing:
        raise SpecError(f"library entry needs inputs {missing}")


def _check_out(case: RunCase, k: int, shape, dtype: str) -> None:
    got = case.output_shapes[k]
    if tuple(got[0]) != tuple(shape) or got[1] != dtype:
        raise SpecError(f"output {k} must be {tuple(shape)} {dtype}, the case says {got}")


def _dev(a: np.ndarray) -> DeviceArray:
    return DeviceArray.from_host(np.ascontiguousarray(a))


# ---------------------------------------------------------------------------
def _bind_wide_qmv(consts: dict, spec: KernelSpec, case: RunCase) -> BoundCall:
    inputs, scalars = _named(spec, case)
    _need(inputs, ("x", "w_q", "scales", "biases"))
    bits, m = _int(consts, "BITS"), _int(consts, "M")
    out_dtype, code = _dtype_of(consts)
    x, w_q, s, b = (inputs[k] for k in ("x", "w_q", "scales", "biases"))
    d_out, d_in = s.shape[0], x.shape[1]
    if x.shape[0] != m:
        raise SpecError(f"M={m} but x has {x.shape[0]} rows")
    if "d_in_arg" in scalars and int(scalars["d_in_arg"]) != d_in:
        raise SpecError("d_in_arg disagrees with x")
    if "d_out_arg" in scalars and int(scalars["d_out_arg"]) != d_out:
        raise SpecError("d_out_arg disagrees with scales")
    if w_q.shape != (d_out, d_in * bits // 32) or x.dtype != np.float16:
        raise SpecError(f"w_q must be {(d_out, d_in * bits // 32)} uint32 and x fp16")
    _check_out(case, 0, (m, d_out), out_dtype)
    dx, dw, ds, db = (_dev(a) for a in (x, w_q, s, b))
    out = DeviceArray((m, d_out), out_dtype)
    fn = lib.load().kvp_qmv

    def launch(stream):
        return fn(dx.ptr, dw.ptr, ds.ptr, db.ptr, out.ptr, code, m, d_out, d_in, bits, stream)

    return BoundCall(launch, [out], (dx, dw, ds, db))


def _bind_kv_attention(consts: dict, spec: KernelSpec, case: RunCase) -> BoundCall:
    from kernelverify_amd.pack import kv_attention

    inputs, scalars = _named(spec, case)
    names = ("q", "k_wq", "k_scales", "k_biases", "v_wq", "v_scales", "v_biases", "new_k", "new_v")
    _need(inputs, names)
    bits, dh = _int(consts, "BITS"), _int(consts, "DH")
    out_dtype, code = _dtype_of(consts)
    q = inputs["q"]
    b, h, qdh = q.shape
    hkv, t_stride = inputs["k_wq"].shape[0], inputs["k_wq"].shape[1]
    if qdh != dh:
        raise SpecError(f"DH={dh} but q has head dim {qdh}")
    for key, want in (("n_heads", h), ("n_kv_heads", hkv), ("t_stride", t_stride)):
        if key in scalars and int(scalars[key]) != want:
            raise SpecError(f"{key}={scalars[key]} disagrees with the tensors ({want})")
    t_cached = int(scalars.get("t_cached", t_stride))
    _check_out(case, 0, (b, h, dh), out_dtype)
    dev = {k: _dev(inputs[k]) for k in names}
    dt = _dev(np.full(b, t_cached, dtype=np.int32))
    out = DeviceArray((b, h, dh), out_dtype)
    call = kv_attention.KvDecodeCall(*(dev[k] for k in names), dt, out, bits=bits)

    def launch(stream):
        return call._fn(*call._args, stream)

    return BoundCall(launch, [out], (dev, dt, call))


def _bind_moe_routing(consts: dict, spec: KernelSpec, case: RunCase) -> BoundCall:
    inputs, scalars = _named(spec, case)
    _need(inputs, ("x", "router"))
    e = _int(consts, "E")
    x, router = inputs["x"], inputs["router"]
    n, d = x.shape
    if router.shape != (e, d):
        raise SpecError(f"E={e} but router is {router.shape}")
    if "d_in_arg" in scalars and int(scalars["d_in_arg"]) != d:
        raise SpecError("d_in_arg disagrees with x")
    k = case.output_shapes[0][0][1]
    _check_out(case, 0, (n, k), "uint32")
    _check_out(case, 1, (n, k), "float32")
    dx, dr = _dev(x), _dev(router)
    idx, gate = DeviceArray((n, k), np.uint32), DeviceArray((n, k), np.float32)
    fn = lib.load().kvp_moe_route

    def launch(stream):
        return fn(dx.ptr, dr.ptr, idx.ptr, gate.ptr, n, d, e, k, stream)

    return BoundCall(launch, [idx, gate], (dx, dr))


def _bind_moe_dispatch(consts: dict, spec: KernelSpec, case: RunCase) -> BoundCall:
    inputs, scalars = _named(spec, case)
    names = ("x", "idx", "gate", "w_q", "scales", "biases")
    _need(inputs, names)
    bits = _int(consts, "BITS") if "BITS" in consts else 4
    out_dtype, code = _dtype_of(consts)
    x, idx = inputs["x"], inputs["idx"]
    n, d_in = x.shape
    k = idx.shape[1]
    e, d_out, _ = inputs["w_q"].shape
    for key, want in (("d_in_arg", d_in), ("d_out_arg", d_out)):
        if key in scalars and int(scalars[key]) != want:
            raise SpecError(f"{key}={scalars[key]} disagrees with the tensors ({want})")
    _check_out(case, 0, (n, d_out), out_dtype)
    dev = [_dev(inputs[k_].astype(np.uint32) if k_ == "idx" else inputs[k_]) for k_ in names]
    out = DeviceArray((n, d_out), out_dtype)
    fn = lib.load().kvp_moe_dispatch

    def launch(stream):
        return fn(*(a.ptr for a in dev), out.ptr, code, n, k, e, d_out, d_in, bits, stream)

    return BoundCall(launch, [out], tuple(dev))


FAMILIES = {
    "wide_qmv": _bind_wide_qmv,
    "kv_attention": _bind_kv_attention,
    "moe_routing": _bind_moe_routing,
    "moe_dispatch": _bind_moe_dispatch,
}


def bind(spec: KernelSpec, case: RunCase) -> BoundCall:
    family, consts = parse_descriptor(spec.source)
    if family not in FAMILIES:
        raise SpecError(f"the pack library has no entry family {family!r} "
                        f"(known: {sorted(FAMILIES)})")
    return FAMILIES[family](consts, spec, case)
