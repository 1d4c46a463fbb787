"""The serving door on PyTorch-ROCm (reference: bench/serve_sub4bit.py:201-260
`_RoutedLinear`, `Patch` 271-340; bench/spike_mlx_e2e.py:126-172, the fused
KV decode door; docs/adr/0018-flattened-row-serving-dispatch.md).

Torch is plumbing here: device memory, the current stream and the module
tree a server already has. The compute of a routed call is the library's
C entry point on the tensors' device pointers (`kvp_qmv`, `kvp_kv_decode`,
`kvp_quantize_affine`), enqueued on torch's current stream.

- `QuantizedLinear`: an MLX-affine quantized linear (uint32 code stream,
  fp16 scales and biases per 64-column group) with a stock forward, the
  incumbent a server runs when the pack does not serve a call.
- `RoutedLinear` wraps one and routes a call to `kvp_qmv` when
  `ineligible(x)` returns None. M is the flattened row count at every input
  rank (ADR 0018): (1, 7, d), (7, 1, d) and (7, d) are the same seven rows
  and the same M = 7 call, and `should_dispatch(m, bits, d_out, d_in)` is
  the only judge of M. Every refused call names its reason.
- `Patch(model)` replaces every `QuantizedLinear` of a module tree in place
  and counts routed calls and fallbacks by reason; `mode = "stock"` makes
  the same decision and discards it (the A/B's forced-stock arm).
  `uninstall()` restores the tree.
- `QuantizedKVCache` keeps a logical length (`offset`, the cached
  positions) apart from the padded stride (`max_len`) it was allocated
  with; `KvDoor` runs one decode step over the `offset` cached positions
  plus the step's own new entry at full precision on `kvp_kv_decode`, or
  names why not and runs the stock attention.
"""

from __future__ import annotations

import math

import torch
from torch import nn

from kernelverify_amd import lib
from kernelverify_amd.pack import kv_attention, wide_qmv

GROUP = 64


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def unpack_codes(w_q: torch.Tensor, bits: int, cols: int) -> torch.Tensor:
    """int64 codes (rows, cols) of an LSB-first code stream held as int32
    words (rows, cols * bits / 32); a code may straddle two words (3-bit)."""
    words = w_q.to(torch.int64) & 0xFFFFFFFF
    bit = torch.arange(cols, device=w_q.device, dtype=torch.int64) * bits
    word, shift = bit >> 5, bit & 31
    low = words[:, word] >> shift
    nxt = torch.clamp(word + 1, max=words.shape[1] - 1)
    high = (words[:, nxt] << (32 - shift)) * ((shift + bits) > 32)
    return (low | high) & ((1 << bits) - 1)


class QuantizedLinear(nn.Module):
    """y = x @ dequant(W)^T (+ bias): MLX-affine codes, group 64 along d_in."""

    def __init__(self, w_q: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, bits: int,
                 bias: torch.Tensor | None = None, group_size: int = GROUP, mode: str = "affine"):
        super().__init__()
        self.bits, self.group_size, self.mode = bits, group_size, mode
        self.register_buffer("weight", w_q.to(torch.int32) if w_q.dtype != torch.int32 else w_q)
        self.register_buffer("scales", scales)
        self.register_buffer("biases", biases)
        self.register_buffer("bias", bias)

    @property
    def d_out(self) -> int:
        return self.scales.shape[0]

    @property
    def d_in(self) -> int:
        # scales are (d_out, d_in / group): rows are the OUTPUT dimension
        return self.scales.shape[1] * self.group_size

    def dequantized(self) -> torch.Tensor:
        codes = unpack_codes(self.weight, self.bits, self.d_in).to(torch.float32)
        s = self.scales.to(torch.float32).repeat_interleave(self.group_size, dim=1)
        b = self.biases.to(torch.float32).repeat_interleave(self.group_size, dim=1)
        return s * codes + b

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        y = x.to(torch.float32) @ self.dequantized().T
        if self.bias is not None:
            y = y + self.bias.to(torch.float32)
        return y.to(x.dtype)


class RoutedLinear(nn.Module):
    """One wrapped QuantizedLinear; `patch` holds the mode and the counters."""

    def __init__(self, inner: QuantizedLinear, patch: "Patch"):
        super().__init__()
        self.inner = inner
        self._patch = patch

    def ineligible(self, x: torch.Tensor) -> str | None:
        """None when the kernel takes this call, else the reason."""
        inner = self.inner
        if not str(inner.mode).endswith("affine"):
            return f"mode-{inner.mode}"
        if inner.bits not in wide_qmv.SUPPORTED_BITS or inner.group_size != GROUP:
            return f"quant-{inner.bits}b-gs{inner.group_size}"
        if inner.bias is not None:
            return "bias-term"
        if x.dtype != torch.float16 or inner.scales.dtype != torch.float16:
            return f"dtype-{x.dtype}-{inner.scales.dtype}"
        if inner.biases.dtype != torch.float16:
            return f"biases-dtype-{inner.biases.dtype}"
        d_in = x.shape[-1]
        if d_in % GROUP or d_in != inner.d_in:
            return f"din-{d_in}"
        # the kernel reads these buffers raw: (d_out, d_in * bits / 32) words
        # and (d_out, d_in / 64) scales and biases, densely packed
        words = d_in * inner.bits // 32
        if (inner.weight.dim() != 2 or tuple(inner.weight.shape) != (inner.d_out, words)
                or inner.weight.element_size() != 4):
            return f"weight-shape-{tuple(inner.weight.shape)}"
        if tuple(inner.biases.shape) != tuple(inner.scales.shape):
            return f"biases-shape-{tuple(inner.biases.shape)}"
        if not all(t.is_contiguous() for t in (inner.weight, inner.scales, inner.biases)):
            return "noncontiguous"
        m = x.numel() // d_in
        if not wide_qmv.should_dispatch(m, inner.bits, inner.d_out, d_in):
            return f"m-{m}-outside-dispatch-{inner.d_out}x{d_in}"
        if not x.is_cuda or any(p.device != x.device
                                for p in (inner.weight, inner.scales, inner.biases)):
            return f"device-{x.device}"
        return None

    def fused(self, x: torch.Tensor) -> torch.Tensor:
        inner = self.inner
        x2 = x.reshape(-1, x.shape[-1]).contiguous()
        m = x2.shape[0]
        out = torch.empty((m, inner.d_out), dtype=torch.float16, device=x.device)
        lib.check(lib.load().kvp_qmv(x2.data_ptr(), inner.weight.data_ptr(),
                                     inner.scales.data_ptr(), inner.biases.data_ptr(),
                                     out.data_ptr(), lib.KVP_F16, m, inner.d_out, inner.d_in,
                                     inner.bits, _stream()))
        return out.reshape(*x.shape[:-1], inner.d_out)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        patch = self._patch
        why = self.ineligible(x)
        if why is None:
            if patch.mode == "fused":
                patch.calls += 1
                return self.fused(x)
            why = "forced-stock"
        patch.fallbacks[why] = patch.fallbacks.get(why, 0) + 1
        return self.inner(x)


class Patch:
    """The installed interception over one module tree."""

    def __init__(self, model: nn.Module, mode: str = "fused"):
        if getattr(model, "_kvp_patch", None) is not None:
            raise RuntimeError("a patch is already installed on this model")
        if mode not in ("fused", "stock"):
            raise ValueError(f"mode {mode!r} not in ('fused', 'stock')")
        self.mode = mode
        self.calls = 0
        self.fallbacks: dict[str, int] = {}
        self._model = model
        self._sites: list[tuple] = []
        for parent in list(model.modules()):
            for name, child in list(parent.named_children()):
                if isinstance(child, QuantizedLinear):
                    setattr(parent, name, RoutedLinear(child, self))
                    self._sites.append((parent, name, child))
        model._kvp_patch = self
        self.n_wrapped = len(self._sites)
        # the routing cell of every wrapped site, (bits, d_out, d_in)
        self.site_cells = [(q.bits, q.d_out, q.d_in) for _, _, q in self._sites]

    def uninstall(self) -> None:
        for parent, name, original in self._sites:
            setattr(parent, name, original)
        self._sites = []
        self._model._kvp_patch = None


class QuantizedKVCache:
    """One layer's K/V cache as MLX-affine artefacts, (1, HKV, max_len, ...)
    with `offset` positions filled; `max_len` is the padded stride the
    kernel walks by, `offset` the logical length it reads."""

    def __init__(self, n_kv_heads: int, head_dim: int, bits: int, max_len: int,
                 device="cuda", group_size: int = GROUP):
        if head_dim % group_size:
            raise ValueError(f"head_dim {head_dim} is not a multiple of {group_size}")
        self.n_kv_heads, self.head_dim, self.bits = n_kv_heads, head_dim, bits
        self.group_size, self.max_len, self.offset = group_size, max_len, 0
        words, groups = head_dim * bits // 32, head_dim // group_size
        shape = (1, n_kv_heads, max_len)
        self.keys = (torch.zeros(shape + (words,), dtype=torch.int32, device=device),
                     torch.zeros(shape + (groups,), dtype=torch.float16, device=device),
                     torch.zeros(shape + (groups,), dtype=torch.float16, device=device))
        self.values = tuple(torch.zeros_like(t) for t in self.keys)

    def _quantize_into(self, dst: tuple, x: torch.Tensor, at: int) -> None:
        hkv, n, dh = x.shape[1], x.shape[2], x.shape[3]
        dev = dst[0].device
        src = x.reshape(hkv * n, dh).to(device=dev, dtype=torch.float16).contiguous()
        parts = (torch.empty((hkv * n, dh * self.bits // 32), dtype=torch.int32, device=dev),
                 torch.empty((hkv * n, dh // self.group_size), dtype=torch.float16, device=dev),
                 torch.empty((hkv * n, dh // self.group_size), dtype=torch.float16, device=dev))
        lib.check(lib.load().kvp_quantize_affine(src.data_ptr(), hkv * n, dh, self.bits,
                                                 parts[0].data_ptr(), parts[1].data_ptr(),
                                                 parts[2].data_ptr(), _stream()))
        for d, p in zip(dst, parts):
            d[0, :, at:at + n] = p.reshape(hkv, n, -1)

    def append(self, keys: torch.Tensor, values: torch.Tensor) -> None:
        """Quantize (1, HKV, L, DH) new entries into positions offset .. offset + L
        with the library's GPU quantizer (the cache must be on a cuda device;
        the entries move there)."""
        if not self.keys[0].is_cuda:
            raise ValueError(f"append quantizes on the GPU: this cache is on {self.keys[0].device}")
        want = (1, self.n_kv_heads, keys.shape[2], self.head_dim)
        if tuple(keys.shape) != want or tuple(values.shape) != want:
            raise ValueError(f"append takes keys and values of shape {want}, got "
                             f"{tuple(keys.shape)} and {tuple(values.shape)}")
        n = keys.shape[2]
        if n == 0:
            return
        if self.offset + n > self.max_len:
            raise ValueError(f"cache of {self.max_len} positions cannot take {n} more at "
                             f"{self.offset}")
        self._quantize_into(self.keys, keys, self.offset)
        self._quantize_into(self.values, values, self.offset)
        self.offset += n

    def dequantized(self) -> tuple[torch.Tensor, torch.Tensor]:
        """fp32 (1, HKV, offset, DH) K and V (the stock path's view)."""
        out = []
        for wq, s, b in (self.keys, self.values):
            rows = wq[0, :, :self.offset].reshape(-1, wq.shape[-1])
            codes = unpack_codes(rows, self.bits, self.head_dim).to(torch.float32)
            sc = s[0, :, :self.offset].reshape(-1, s.shape[-1]).to(torch.float32)
            bi = b[0, :, :self.offset].reshape(-1, b.shape[-1]).to(torch.float32)
            deq = (sc.repeat_interleave(self.group_size, 1) * codes
                   + bi.repeat_interleave(self.group_size, 1))
            out.append(deq.reshape(1, self.n_kv_heads, self.offset, self.head_dim))
        return out[0], out[1]


class KvDoor:
    """One decode step of quantized-KV attention, routed or named fallback."""

    def __init__(self, mode: str = "fused"):
        if mode not in ("fused", "stock"):
            raise ValueError(f"mode {mode!r} not in ('fused', 'stock')")
        self.mode = mode
        self.calls = 0
        self.fallbacks: dict[str, int] = {}

    @staticmethod
    def ineligible(queries, cache, scale: float, mask=None) -> str | None:
        b, h, length, d = queries.shape
        if length != 1:
            return f"prefill-L{length}"
        if not isinstance(cache, QuantizedKVCache):
            return "cache-not-quantized"
        if b != 1:
            return f"batch-B{b}"
        if d not in kv_attention.SUPPORTED_DH or d != cache.head_dim:
            return f"head-dim-{d}"
        if cache.bits not in kv_attention.SUPPORTED_BITS or cache.group_size != GROUP:
            return f"quant-{cache.bits}b-gs{cache.group_size}"
        if h % cache.n_kv_heads or h // cache.n_kv_heads not in (1, 2, 4, 8):
            return f"gqa-{h}/{cache.n_kv_heads}"
        if mask is not None and not (isinstance(mask, str) and mask == "causal"):
            return "mask-array"
        if queries.dtype != torch.float16:
            return f"dtype-{queries.dtype}"
        if abs(scale * math.sqrt(d) - 1.0) > 1e-6:
            return "nonstandard-scale"
        if not queries.is_cuda:
            return f"device-{queries.device}"
        if any(p.device != queries.device for p in (*cache.keys, *cache.values)):
            return f"cache-device-{cache.keys[0].device}"
        return None

    @staticmethod
    def fused(queries, cache: QuantizedKVCache, new_k, new_v) -> torch.Tensor:
        b, h, _, d = queries.shape
        hkv = cache.n_kv_heads
        q = queries.reshape(b, h, d).contiguous()
        nk, nv = (t.reshape(b, hkv, d).to(device=queries.device, dtype=torch.float16).contiguous()
                  for t in (new_k, new_v))
        t_cached = torch.full((b,), cache.offset, dtype=torch.int32, device=queries.device)
        out = torch.empty((b, h, d), dtype=torch.float16, device=queries.device)
        L = lib.load()
        need = L.kvp_kv_decode_workspace_bytes(b, h, d, cache.max_len, 0)
        ws = torch.empty((max(int(need), 4),), dtype=torch.uint8, device=queries.device)
        (kw, ks, kb), (vw, vs, vb) = cache.keys, cache.values
        lib.check(L.kvp_kv_decode(q.data_ptr(), kw.data_ptr(), ks.data_ptr(), kb.data_ptr(),
                                  vw.data_ptr(), vs.data_ptr(), vb.data_ptr(), nk.data_ptr(),
                                  nv.data_ptr(), t_cached.data_ptr(), out.data_ptr(),
                                  lib.KVP_F16, b, h, hkv, d, cache.max_len, cache.bits, 0, 0,
                                  ws.data_ptr(), ws.numel(), _stream()))
        return out.reshape(b, h, 1, d)

    @staticmethod
    def stock(queries, cache: QuantizedKVCache, new_k, new_v, scale: float) -> torch.Tensor:
        """fp32 attention over the dequantized cache plus the new entry."""
        b, h, length, d = queries.shape
        k, v = cache.dequantized()
        k = torch.cat([k.expand(b, -1, -1, -1), new_k.to(torch.float32)], dim=2)
        v = torch.cat([v.expand(b, -1, -1, -1), new_v.to(torch.float32)], dim=2)
        rep = h // k.shape[1]
        k = k.repeat_interleave(rep, dim=1).contiguous()
        v = v.repeat_interleave(rep, dim=1).contiguous()
        scores = torch.matmul(queries.to(torch.float32), k.transpose(-1, -2).contiguous())
        scores = scores * scale
        t = k.shape[2]
        if length > 1:  # causal over the new entries
            pos = torch.arange(t, device=queries.device)
            rows = t - length + torch.arange(length, device=queries.device)
            allowed = pos[None, :] <= rows[:, None]
            scores = scores.masked_fill(~allowed, float("-inf"))
        p = torch.softmax(scores, dim=-1)
        return torch.matmul(p, v).to(queries.dtype)

    def __call__(self, queries, cache, new_k, new_v, scale: float, mask=None):
        why = self.ineligible(queries, cache, scale, mask)
        if why is None:
            if self.mode == "fused":
                self.calls += 1
                return self.fused(queries, cache, new_k, new_v)
            why = "forced-stock"
        self.fallbacks[why] = self.fallbacks.get(why, 0) + 1
        return self.stock(queries, cache, new_k, new_v, scale)
