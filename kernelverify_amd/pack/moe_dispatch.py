"""Top-k MoE decode on MI355X: routing, permutation, expert gather-qmv.

Host side of the MoE entry points of libkvpack (kernelverify_amd/csrc/moe.hip),
mirroring the reference's pack module ``kernelverify/pack/moe_dispatch.py``:

- routing contract unchanged: fp32 logits (``x @ router^T``, or given), an fp32
  softmax over every expert, top-k BY PROBABILITY with ties to the lower
  expert index, renormalised over the k chosen (:39-79, and
  ``kernelverify/reference/native_kernels.py:92-101``);
- ``dispatch``: the reference's single-linear contract
  ``out[t] = sum_s gate[t, s] * (x_t . W_{idx[t, s]})`` (:84-138) at any k
  (the reference fixes k = 2, :27);
- ``swiglu``: BASELINE config 5's expert MLP (gate/up/down), where each
  routed expert's weights stream from HBM once per step whatever the number
  of tokens that chose it; tokens are grouped by a stable counting sort
  (``permute``), bit-exact and deterministic.
"""

from __future__ import annotations

import numpy as np

from kernelverify_amd import lib
from kernelverify_amd.hip import DeviceArray

SUPPORTED_BITS = (2, 3, 4, 8)
TOP_K = 8
MAX_K = 32
MAX_EXPERTS = 1024
GROUP = 64
OUT_DTYPES = {"float16": lib.KVP_F16, "float32": lib.KVP_F32}


def _h(stream):
    return getattr(stream, "handle", stream)


def expert_bytes(d_out: int, d_in: int, bits: int) -> int:
    """One quantized expert matrix: codes + fp16 scales and biases."""
    return d_out * d_in * bits // 8 + 2 * (d_out * d_in // GROUP) * 2


def algorithmic_bytes(idx: np.ndarray, n_experts: int, d_model: int, d_ffn: int, bits: int,
                      logits: bool = True, out_itemsize: int = 2) -> int:
    """Unique routed experts' gate/up/down weights once, logits, x and out."""
    unique = len(np.unique(np.asarray(idx)))
    per_expert = 2 * expert_bytes(d_ffn, d_model, bits) + expert_bytes(d_model, d_ffn, bits)
    n = idx.shape[0]
    return (unique * per_expert + (n * n_experts * 4 if logits else 0) + n * d_model * 2
            + n * d_model * out_itemsize)


def quantize_experts(experts: np.ndarray, bits: int):
    """(E, d_out, d_in) fp16 -> (codes (E, d_out, words), scales, biases) via
    the GPU quantizer (bench/pack_moe_dispatch.py:76-83 stacks the same)."""
    from kernelverify_amd.pack.quant import quantize

    return quantize(np.ascontiguousarray(experts, dtype=np.float16), bits)


def route_logits(logits: DeviceArray, idx: DeviceArray, gate: DeviceArray, k: int,
                 stream=None) -> None:
    n, e = logits.shape
    if logits.dtype != np.float32:
        raise lib.InvalidArgument("route: logits must be fp32 (n, E)")
    if idx.shape != (n, k) or idx.dtype != np.uint32 or gate.shape != (n, k) \
            or gate.dtype != np.float32:
        raise lib.InvalidArgument(f"route: idx uint32 and gate fp32 must be {(n, k)}")
    lib.check(lib.load().kvp_moe_route_logits(logits.ptr, idx.ptr, gate.ptr, n, e, k,
                                              _h(stream)))


def route_x(x: DeviceArray, router: DeviceArray, idx: DeviceArray, gate: DeviceArray, k: int,
            stream=None) -> None:
    n, d = x.shape
    e = router.shape[0]
    if x.dtype != np.float16 or router.dtype != np.float16 or router.shape != (e, d):
        raise lib.InvalidArgument("route: x (n, d) and router (E, d) must be fp16")
    lib.check(lib.load().kvp_moe_route(x.ptr, router.ptr, idx.ptr, gate.ptr, n, d, e, k,
                                       _h(stream)))


def permute(idx: DeviceArray, n_experts: int, stream=None):
    """-> (offsets int32 (E+1,), perm int32 (n*k,)) device arrays."""
    n, k = idx.shape
    offsets = DeviceArray((n_experts + 1,), np.int32)
    perm = DeviceArray((n * k,), np.int32)
    lib.check(lib.load().kvp_moe_permute(idx.ptr, offsets.ptr, perm.ptr, n, k, n_experts,
                                         _h(stream)))
    return offsets, perm


def dispatch(x: DeviceArray, idx: DeviceArray, gate: DeviceArray, w_q: DeviceArray,
             scales: DeviceArray, biases: DeviceArray, out: DeviceArray, *, bits: int,
             stream=None) -> None:
    n, d_in = x.shape
    k = idx.shape[1]
    e, d_out, words = w_q.shape
    if words * 32 != d_in * bits:
        raise lib.InvalidArgument(f"dispatch: {words} words per row for d_in={d_in} {bits}-bit")
    if out.shape != (n, d_out) or out.dtype.name not in OUT_DTYPES:
        raise lib.InvalidArgument(f"dispatch: out must be fp16/fp32 {(n, d_out)}")
    lib.check(lib.load().kvp_moe_dispatch(x.ptr, idx.ptr, gate.ptr, w_q.ptr, scales.ptr,
                                          biases.ptr, out.ptr, OUT_DTYPES[out.dtype.name], n, k,
                                          e, d_out, d_in, bits, _h(stream)))


def swiglu_workspace_bytes(n: int, k: int, n_experts: int, d_model: int, d_ffn: int) -> int:
    return int(lib.load().kvp_moe_swiglu_workspace_bytes(n, k, n_experts, d_model, d_ffn))


class SwigluCall:
    """One validated SwiGLU MoE step (bound arguments, own workspace).

    With ``logits`` (fp32 (n, E) on the device) the call routes too
    (``kvp_moe_route_swiglu``): ``idx`` and ``gate`` are then outputs, written
    as ``route_logits`` writes them."""

    def __init__(self, x: DeviceArray, idx: DeviceArray, gate: DeviceArray, gate_w, up_w,
                 down_w, out: DeviceArray, *, bits: int, workspace: DeviceArray | None = None,
                 logits: DeviceArray | None = None):
        n, d_model = x.shape
        k = idx.shape[1]
        e, d_ffn, words = gate_w[0].shape
        if words * 32 != d_model * bits or up_w[0].shape != gate_w[0].shape:
            raise lib.InvalidArgument("swiglu: gate/up weights must be (E, d_ffn, d_model*bits/32)")
        if down_w[0].shape != (e, d_model, d_ffn * bits // 32):
            raise lib.InvalidArgument("swiglu: down weights must be (E, d_model, d_ffn*bits/32)")
        if out.shape != (n, d_model) or out.dtype.name not in OUT_DTYPES:
            raise lib.InvalidArgument(f"swiglu: out must be fp16/fp32 {(n, d_model)}")
        need = swiglu_workspace_bytes(n, k, e, d_model, d_ffn)
        self.workspace = workspace if workspace is not None else DeviceArray((need,), np.uint8)
        if self.workspace.nbytes < need:
            raise lib.InvalidArgument(f"swiglu: workspace {self.workspace.nbytes} < {need}")
        args = (x.ptr, idx.ptr, gate.ptr, *(a.ptr for a in (*gate_w, *up_w, *down_w)),
                out.ptr, OUT_DTYPES[out.dtype.name], n, k, e, d_model, d_ffn, bits,
                self.workspace.ptr, self.workspace.nbytes)
        if logits is not None:
            if logits.shape != (n, e) or logits.dtype != np.float32:
                raise lib.InvalidArgument(f"swiglu: logits must be fp32 {(n, e)}")
            self._fn = lib.load().kvp_moe_route_swiglu
            self._args = (logits.ptr, *args)
        else:
            self._fn = lib.load().kvp_moe_swiglu
            self._args = args
        self._keep = (x, idx, gate, gate_w, up_w, down_w, out, logits)

    def __call__(self, stream=None) -> None:
        status = self._fn(*self._args, _h(stream))
        if status:
            lib.check(status)


# ---------------------------------------------------------------------------
# Host conveniences over numpy arrays
# ---------------------------------------------------------------------------
def _sync_get(*arrays):
    from kernelverify_amd import hip

    hip.synchronize()
    return tuple(a.to_host() for a in arrays)


def route(logits: np.ndarray | None = None, k: int = TOP_K, *, x: np.ndarray | None = None,
          router: np.ndarray | None = None):
    """(idx uint32 (n, k), gate fp32 (n, k)) from logits, or from x and router."""
    if logits is not None:
        n = logits.shape[0]
        idx, gate = DeviceArray((n, k), np.uint32), DeviceArray((n, k), np.float32)
        route_logits(DeviceArray.from_host(np.ascontiguousarray(logits, dtype=np.float32)), idx,
                     gate, k)
    else:
        n = x.shape[0]
        idx, gate = DeviceArray((n, k), np.uint32), DeviceArray((n, k), np.float32)
        route_x(DeviceArray.from_host(np.ascontiguousarray(x, dtype=np.float16)),
                DeviceArray.from_host(np.ascontiguousarray(router, dtype=np.float16)), idx, gate, k)
    return _sync_get(idx, gate)


def permute_host(idx: np.ndarray, n_experts: int):
    offsets, perm = permute(DeviceArray.from_host(np.ascontiguousarray(idx, dtype=np.uint32)),
                            n_experts)
    return _sync_get(offsets, perm)


def dispatch_host(x, idx, gate, w_q, scales, biases, *, bits: int, out_dtype: str = "float16"):
    dev = [DeviceArray.from_host(np.ascontiguousarray(a)) for a in
           (x.astype(np.float16), idx.astype(np.uint32), gate.astype(np.float32), w_q, scales,
            biases)]
    out = DeviceArray((x.shape[0], w_q.shape[1]), out_dtype)
    dispatch(*dev, out, bits=bits)
    return _sync_get(out)[0]


def swiglu_host(x, idx, gate, gate_w, up_w, down_w, *, bits: int, out_dtype: str = "float16"):
    up = lambda t: tuple(DeviceArray.from_host(np.ascontiguousarray(a)) for a in t)
    dx = DeviceArray.from_host(np.ascontiguousarray(x, dtype=np.float16))
    di = DeviceArray.from_host(np.ascontiguousarray(idx, dtype=np.uint32))
    dg = DeviceArray.from_host(np.ascontiguousarray(gate, dtype=np.float32))
    out = DeviceArray((x.shape[0], x.shape[1]), out_dtype)
    SwigluCall(dx, di, dg, up(gate_w), up(up_w), up(down_w), out, bits=bits)()
    return _sync_get(out)[0]


def route_swiglu_host(x, logits, k, gate_w, up_w, down_w, *, bits: int,
                      out_dtype: str = "float16"):
    """Routing from logits and the experts in one call: (out, idx, gate)."""
    up = lambda t: tuple(DeviceArray.from_host(np.ascontiguousarray(a)) for a in t)
    n = x.shape[0]
    dx = DeviceArray.from_host(np.ascontiguousarray(x, dtype=np.float16))
    dl = DeviceArray.from_host(np.ascontiguousarray(logits, dtype=np.float32))
    di, dg = DeviceArray((n, k), np.uint32), DeviceArray((n, k), np.float32)
    out = DeviceArray((n, x.shape[1]), out_dtype)
    SwigluCall(dx, di, dg, up(gate_w), up(up_w), up(down_w), out, bits=bits, logits=dl)()
    return _sync_get(out, di, dg)


# ---------------------------------------------------------------------------
# Runner-door templates (reference: kernelverify/pack/moe_dispatch.py:148-234)
# ---------------------------------------------------------------------------
ROUTING_NAME = "kvp_moe_route"
DISPATCH_NAME = "kvp_moe_dispatch"
BLOCK = 256


def routing_launch(n_tokens: int) -> tuple:
    """(grid, block): one block per token (the logits sit in LDS)."""
    return (n_tokens, 1, 1), (BLOCK, 1, 1)


def dispatch_launch(d_out: int, n_tokens: int) -> tuple:
    """(grid, block, rows per block): the single-linear dispatch kernel runs
    a block per (8 output rows, token)."""
    rows = 8
    return ((d_out + rows - 1) // rows, n_tokens, 1), (BLOCK, 1, 1), rows


def routing_spec():
    """Routing template: `specialize()` fills `E`; the top-k width is the
    outputs' width (the reference's k = 2); d_model is the `d_in_arg` scalar."""
    from kernelverify_amd.runners import Binding, BindingKind, KernelSpec, LaunchMode, LaunchSpec

    return KernelSpec(
        source="kvpack:moe_routing E=$E",
        entry_point=ROUTING_NAME,
        name=f"{ROUTING_NAME}-E$E",
        bindings=(Binding(BindingKind.INPUT, "x"),
                  Binding(BindingKind.INPUT, "router"),
                  Binding(BindingKind.OUTPUT),
                  Binding(BindingKind.OUTPUT),
                  Binding(BindingKind.SCALAR, "d_in_arg", "uint32")),
        launch=LaunchSpec(grid=("n_tokens", 1, 1), threadgroup=(BLOCK, 1, 1),
                          mode=LaunchMode.THREADGROUPS),
    )


def dispatch_spec(bits: int | None = None):
    """Dispatch template: `specialize()` fills `T` and `R` (R is recorded;
    the library tiles by its own rule). The reference kernel is 4-bit only;
    ``bits`` fixes another width in the descriptor."""
    from kernelverify_amd.runners import Binding, BindingKind, KernelSpec, LaunchMode, LaunchSpec

    width = "" if bits is None else f" BITS={int(bits)}"
    return KernelSpec(
        source=f"kvpack:moe_dispatch T=$T R=$R{width}",
        entry_point=DISPATCH_NAME,
        name=f"{DISPATCH_NAME}-R$R-$T",
        bindings=(Binding(BindingKind.INPUT, "x"),
                  Binding(BindingKind.INPUT, "idx"),
                  Binding(BindingKind.INPUT, "gate"),
                  Binding(BindingKind.INPUT, "w_q"),
                  Binding(BindingKind.INPUT, "scales"),
                  Binding(BindingKind.INPUT, "biases"),
                  Binding(BindingKind.OUTPUT),
                  Binding(BindingKind.SCALAR, "d_in_arg", "uint32"),
                  Binding(BindingKind.SCALAR, "d_out_arg", "uint32")),
        launch=LaunchSpec(grid=("row_blocks", "n_tokens", 1), threadgroup=(BLOCK, 1, 1),
                          mode=LaunchMode.THREADGROUPS),
    )
