"""Fused quantized-KV decode attention on MI355X, any context length.

Host side of ``kvp_kv_decode`` (kernelverify_amd/csrc/kv_decode.hip),
mirroring the reference's pack module ``kernelverify/pack/kv_attention.py``:
the same operator (one decode step; scores over T cached positions plus the
step's own new entry at full precision; fp32 softmax over T + 1), the same
cache layout per KV head ((T_stride, DH*bits/32) uint32 code rows plus
(T_stride, DH/64) fp16 scales and biases, the MLX affine artefact of
``quantize_cache``, :270-283) and the same GQA mapping (query head h reads
cache head h // (H / HKV), :99-103).

What the MI355X build adds (BASELINE configs 3 and 4):
- no capacity bound: the reference's ``TCAP = 1024`` (:77) is gone; the
  cache is split into chunks of positions whose partials (m, l, o) merge with
  a log-sum-exp combine, so ``should_dispatch`` accepts any T;
- per-sequence caches and lengths: ``cache_per_sequence=True`` takes caches
  shaped (B, HKV, T_stride, .) and a length per sequence; the reference's
  layout (one cache shared by every batch row) stays the default;
- each KV head is read once for its H/HKV query heads.
"""

from __future__ import annotations

import numpy as np

from kernelverify_amd import lib
from kernelverify_amd.hip import DeviceArray
from kernelverify_amd.pack.codes import pack_codes

KERNEL_NAME = "kvp_kv_decode"
SUPPORTED_BITS = (2, 3, 4, 8)
SUPPORTED_DH = (64, 128)
SUPPORTED_GQA = (1, 2, 4, 8)
GROUP = 64
OUT_DTYPES = {"float16": lib.KVP_F16, "float32": lib.KVP_F32}


def should_dispatch(t: int) -> bool:
    """Any cached length runs here (the reference routes T > 1024 away, :242-256)."""
    return t >= 0


def uses_matrix_cores(bits: int, gqa: int) -> bool:
    """4- and 8-bit caches with up to 8 query heads per KV head take the
    MFMA score kernel; 2- and 3-bit caches the all-VALU kernel."""
    return bits in (4, 8) and gqa <= 8


def max_chunk(bits: int, gqa: int = 4, batch: int = 1) -> int:
    """Largest chunk the library picks (positions per block): the MFMA
    kernel walks its slice tile by tile, longer slices for several sequences
    (whose lengths the host does not know); the VALU kernel holds its
    chunk's codes in registers. Mirrors ``pick_chunk`` in csrc/kv_decode.hip."""
    if uses_matrix_cores(bits, gqa):
        return 4096 if batch > 1 else 1024
    return 128


def launch_config(batch: int, n_kv_heads: int, t_stride: int, bits: int = 4,
                  chunk: int | None = None, gqa: int = 4):
    """(grid, block, chunk): one block per (chunk, KV head, sequence); the
    library's own chunk choice when ``chunk`` is None: about 256 blocks for
    the matrix-core kernel, about 1024 for the register-prefetched one."""
    if not chunk:
        target = batch * n_kv_heads * t_stride // (256 if uses_matrix_cores(bits, gqa) else 1024)
        chunk = 64
        while chunk < max_chunk(bits, gqa, batch) and chunk < target:
            chunk *= 2
    n_chunks = max(1, -(-t_stride // chunk))
    return (n_chunks, n_kv_heads, batch), (256, 1, 1), chunk


def cache_bytes(t: int, head_dim: int, bits: int) -> int:
    """One KV head's K or V cache for t positions: codes + fp16 scales/biases."""
    return t * (head_dim * bits // 8 + 2 * (head_dim // GROUP) * 2)


def algorithmic_bytes(lengths, n_heads: int, n_kv_heads: int, head_dim: int, bits: int,
                      out_itemsize: int = 2) -> int:
    """HBM bytes a step must move: each sequence's K and V once per KV head,
    q, new_k/new_v and the output."""
    caches = sum(2 * n_kv_heads * cache_bytes(int(t), head_dim, bits) for t in lengths)
    b = len(lengths)
    return (caches + b * n_heads * head_dim * 2 + 2 * b * n_kv_heads * head_dim * 2
            + b * n_heads * head_dim * out_itemsize)


def pack_cache(q_codes: np.ndarray, scales: np.ndarray, biases: np.ndarray, bits: int):
    """Artefact of an (..., T, DH) cache -> (codes uint32 (..., T, DH*bits/32),
    scales, biases) in the kernel layout (rows packed independently)."""
    lead = q_codes.shape[:-1]
    dh = q_codes.shape[-1]
    words = pack_codes(q_codes.reshape(-1, dh), bits).reshape(*lead, dh * bits // 32)
    return (np.ascontiguousarray(words),
            np.ascontiguousarray(scales.reshape(*lead, dh // GROUP)),
            np.ascontiguousarray(biases.reshape(*lead, dh // GROUP)))


def workspace_bytes(batch: int, n_heads: int, head_dim: int, t_stride: int, chunk: int) -> int:
    return int(lib.load().kvp_kv_decode_workspace_bytes(batch, n_heads, head_dim, t_stride, chunk))


class KvDecodeCall:
    """One validated decode step with its arguments bound (serving loops,
    graph capture). Buffers are DeviceArrays; the workspace is owned here."""

    def __init__(self, q, k_wq, k_s, k_b, v_wq, v_s, v_b, new_k, new_v, t_cached, out, *,
                 bits: int, cache_per_sequence: bool = False, chunk: int = 0,
                 workspace: DeviceArray | None = None):
        if bits not in SUPPORTED_BITS:
            raise lib.Unsupported(f"kv_decode: bits={bits} not in {SUPPORTED_BITS}")
        if len(q.shape) != 3 or q.dtype != np.float16:
            raise lib.InvalidArgument(f"kv_decode: q must be fp16 (B, H, DH), got {q.shape}")
        b, h, dh = q.shape
        lead = 4 if cache_per_sequence else 3
        if len(k_wq.shape) != lead:
            raise lib.InvalidArgument(f"kv_decode: k_wq must have {lead} dims, got {k_wq.shape}")
        if cache_per_sequence and k_wq.shape[0] != b:
            raise lib.InvalidArgument("kv_decode: per-sequence cache batch != q batch")
        hkv, t_stride, words = k_wq.shape[-3:]
        if words * 32 != dh * bits:
            raise lib.InvalidArgument(f"kv_decode: {words} words per row for DH={dh} {bits}-bit")
        for name, t, want in (("k_wq", k_wq, k_wq.shape), ("v_wq", v_wq, k_wq.shape)):
            if t.shape != want or t.dtype != np.uint32:
                raise lib.InvalidArgument(f"kv_decode: {name} must be uint32 {want}")
        sb_shape = k_wq.shape[:-1] + (dh // GROUP,)
        for name, t in (("k_scales", k_s), ("k_biases", k_b), ("v_scales", v_s),
                        ("v_biases", v_b)):
            if t.shape != sb_shape or t.dtype != np.float16:
                raise lib.InvalidArgument(f"kv_decode: {name} must be fp16 {sb_shape}")
        for name, t in (("new_k", new_k), ("new_v", new_v)):
            if t.shape != (b, hkv, dh) or t.dtype != np.float16:
                raise lib.InvalidArgument(f"kv_decode: {name} must be fp16 {(b, hkv, dh)}")
        if t_cached.shape != (b,) or t_cached.dtype != np.int32:
            raise lib.InvalidArgument("kv_decode: t_cached must be int32 (B,)")
        if out.shape != (b, h, dh) or out.dtype.name not in OUT_DTYPES:
            raise lib.InvalidArgument(f"kv_decode: out must be fp16/fp32 {(b, h, dh)}")
        _, _, chunk = launch_config(b, hkv, t_stride, bits, chunk or None, gqa=h // hkv)
        need = workspace_bytes(b, h, dh, t_stride, chunk)
        if workspace is None:
            workspace = DeviceArray((max(need, 4),), np.uint8)
        elif workspace.nbytes < need:
            raise lib.InvalidArgument(f"kv_decode: workspace {workspace.nbytes} < {need} bytes")
        self.workspace = workspace
        self._fn = lib.load().kvp_kv_decode
        self._args = (q.ptr, k_wq.ptr, k_s.ptr, k_b.ptr, v_wq.ptr, v_s.ptr, v_b.ptr, new_k.ptr,
                      new_v.ptr, t_cached.ptr, out.ptr, OUT_DTYPES[out.dtype.name], b, h, hkv, dh,
                      t_stride, bits, 1 if cache_per_sequence else 0, chunk, workspace.ptr,
                      workspace.nbytes)
        self._keep = (q, k_wq, k_s, k_b, v_wq, v_s, v_b, new_k, new_v, t_cached, out)

    def __call__(self, stream=None) -> None:
        status = self._fn(*self._args, getattr(stream, "handle", stream))
        if status:
            lib.check(status)


def kv_decode(q, k_wq, k_s, k_b, v_wq, v_s, v_b, new_k, new_v, t_cached, *, bits: int,
              cache_per_sequence: bool = False, out_dtype: str = "float16", chunk: int = 0):
    """Host convenience over numpy arrays: upload, one step, download."""
    from kernelverify_amd import hip

    dev = [DeviceArray.from_host(np.ascontiguousarray(a)) for a in
           (q, k_wq, k_s, k_b, v_wq, v_s, v_b, new_k, new_v,
            np.asarray(t_cached, dtype=np.int32))]
    out = DeviceArray(q.shape, out_dtype)
    KvDecodeCall(*dev, out, bits=bits, cache_per_sequence=cache_per_sequence, chunk=chunk)()
    hip.synchronize()
    return out.to_host()


def kernel_spec():
    """The runner-door template (reference: kernelverify/pack/kv_attention.py:292-352).

    A pack-library descriptor: `specialize()` fills `T`, `BITS` and `DH`;
    the bindings keep the reference's names and order (q, k_wq .. v_biases,
    new_k, new_v, out, then the scalars n_heads, t_cached, n_kv_heads,
    t_stride). The caches are the reference's shared (HKV, T_stride, ...)
    layout; `t_cached` is the logical length of every batch row, with no
    capacity bound. The grid's ``b_rows x n_heads`` extent is informational.
    """
    from kernelverify_amd.runners import Binding, BindingKind, KernelSpec, LaunchMode, LaunchSpec

    return KernelSpec(
        source="kvpack:kv_attention T=$T BITS=$BITS DH=$DH",
        entry_point=KERNEL_NAME,
        name=f"{KERNEL_NAME}-$BITS bit-DH$DH-$T",
        bindings=(Binding(BindingKind.INPUT, "q"),
                  Binding(BindingKind.INPUT, "k_wq"),
                  Binding(BindingKind.INPUT, "k_scales"),
                  Binding(BindingKind.INPUT, "k_biases"),
                  Binding(BindingKind.INPUT, "v_wq"),
                  Binding(BindingKind.INPUT, "v_scales"),
                  Binding(BindingKind.INPUT, "v_biases"),
                  Binding(BindingKind.INPUT, "new_k"),
                  Binding(BindingKind.INPUT, "new_v"),
                  Binding(BindingKind.OUTPUT),
                  Binding(BindingKind.SCALAR, "n_heads", "uint32"),
                  Binding(BindingKind.SCALAR, "t_cached", "uint32"),
                  Binding(BindingKind.SCALAR, "n_kv_heads", "uint32"),
                  Binding(BindingKind.SCALAR, "t_stride", "uint32")),
        launch=LaunchSpec(grid=(1, 1, ["b_rows", "n_heads"]), threadgroup=(256, 1, 1),
                          mode=LaunchMode.THREADGROUPS),
    )
