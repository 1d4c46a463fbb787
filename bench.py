"""Bench the quantized decode pack on one MI355X; prints ONE JSON line.

Workload of ``value`` (the metric's headline case):
4-bit affine qmv, W 14336 x 4096, group 64, batch M = 1, fp16 x and out.
A "step" is one ``kvp_qmv`` launch over one weight artefact.

Protocol (kernelverify bench/interleave.py:38-103, bench/pack_wide_qmv.py:282-329,
re-targeted to HIP):
- verify first: the GPU output of every timed configuration is checked
  against the CPU baseline's output on the same inputs before any timing
  (the CPU leg doubles as the checker; no timing is printed for a failing
  configuration);
- weights rotate over >= 1 GiB of distinct artefact copies, more than the
  256 MB Infinity Cache, so every launch reads HBM;
- W warmup launches, then a HIP graph holding EXACTLY K launches
  back-to-back on one stream, bracketed by event-record nodes inside the
  graph (the host's graph-launch latency stays out of the window), replayed
  for ROUNDS >= 7 rounds between device synchronisations; ms_per_step is the
  median over rounds of elapsed / K, and ``timing`` carries every round's
  min, max and max/min spread (a row over 1.5 is re-timed once, then
  flagged, bench/interleave.py:48, :77-103). ``timing_5ms_samples`` repeats
  the headline with rounds of at least 5 ms of launches (interleave.py:38)
  as a cross-check; every other row is timed that way;
- ``roofline.achieved`` = algorithmic bytes per launch / ms_per_step, with
  the bytes of ``kernelverify_amd.pack.wide_qmv.algorithmic_bytes``;
  ``roofline.frac`` is against the 8 TB/s spec and
  ``roofline.measured_ceiling`` against back-to-back probe reads of the same
  bytes per launch (each KV and MoE row carries ``frac_measured_ceiling``
  alike);
- ``valu_bound`` on every row (and on ``roofline``): min(HBM, VALU, matrix
  core), the time the call's bytes need at 8 TB/s beside the time its
  hardware-counted instructions need at the issue rates the compute probes
  measure in this run (kernelverify_amd/counters.py; the counts come from
  ``profiles/issue_counts_bench.json``, made by rocprofv3 over
  ``--issue-profile``), the resource that binds and the achieved fraction
  of its cap.

The other BASELINE configurations ride in the same line: the qmv ones
(config 1's 4096 x 4096, config 2's 8-bit, M = 4/8 and 4096 x 14336) under
"secondary", KV decode (configs 3 and 4 and the 32k case) under "kv_decode",
and the MoE expert layer (config 5) under "moe".

CPU paths (skipped with ``--no-cpu``): ``cpu_baseline`` times the numpy
control path of the headline (fp32 dequant + BLAS) and adds
``matmul_only_value``, BLAS alone on weights dequantized beforehand (an upper
bound for any CPU path), and the BLAS vendor. Every KV and MoE row carries
``cpu``: a numpy port of the reference CPU path on the same stored
artefacts, dequantized per call as the GPU path does, checked against the
verified GPU output and timed over a bounded sample.

``--gpus N`` with N > 1 exits: this build measures one GPU.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_HBM_GBS = 8000.0
ROTATION_BYTES = 1 << 30
METRIC = "achieved HBM GB/s (% of 8 TB/s) + µs/call, 4-bit qmv & quant-KV decode attn"


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


# ---------------------------------------------------------------------------
# qmv workload
# ---------------------------------------------------------------------------
class QmvWorkload:
    def __init__(self, d_out, d_in, bits, m, seed=0):
        from kernelverify_amd.hip import DeviceArray
        from kernelverify_amd.pack import wide_qmv
        from kernelverify_amd.pack.codes import pack_codes

        self.d_out, self.d_in, self.bits, self.m = d_out, d_in, bits, m
        self.name = f"qmv {bits}b {d_out}x{d_in} M{m}"
        rng = np.random.default_rng(seed)
        self.q = rng.integers(0, 1 << bits, size=(d_out, d_in), dtype=np.int32)
        g = d_in // 64
        self.scales = np.abs(rng.standard_normal((d_out, g)) * 0.02).astype(np.float16)
        self.biases = (rng.standard_normal((d_out, g)) * 0.01).astype(np.float16)
        self.x = rng.standard_normal((m, d_in)).astype(np.float16)
        self.w_q = pack_codes(self.q, bits)
        self.bytes = wide_qmv.algorithmic_bytes(m, d_out, d_in, bits)
        art = wide_qmv.artefact_bytes(d_out, d_in, bits)
        copies = max(2, -(-ROTATION_BYTES // art))
        self.dx = DeviceArray.from_host(self.x)
        self.copies = []
        for _ in range(copies):
            self.copies.append((DeviceArray.from_host(self.w_q), DeviceArray.from_host(self.scales),
                                DeviceArray.from_host(self.biases)))
        self.out = DeviceArray((m, d_out), np.float16)
        self.calls = [wide_qmv.QmvCall(self.dx, w, s, b, self.out, bits=bits)
                      for w, s, b in self.copies]
        self.i = 0

    def step(self, stream):
        self.calls[self.i % len(self.calls)](stream)
        self.i += 1

    def gpu_output(self):
        from kernelverify_amd import hip

        self.step(None)
        hip.synchronize()
        return self.out.to_host()

    def cpu_reference(self):
        """The reference CPU path on this artefact: fp32 dequant then BLAS
        (kernelverify/reference/native_kernels.py:66-83)."""
        from oracle.extensions import artefact_from_arrays
        from oracle.native_kernels import quantized_matmul_artefact

        art = artefact_from_arrays(self.q, self.scales, self.biases, self.bits)
        return lambda: quantized_matmul_artefact(self.x, art)


class KvWorkload:
    """One decode step of quantized-KV attention (BASELINE configs 3/4 and
    the 32k-context target): K, V ~ N(0, 1) fp16 quantized on the GPU
    (``kvp_quantize_affine``), rotated over >= 1 GiB of device copies."""

    def __init__(self, lengths, n_heads=32, n_kv_heads=8, head_dim=128, bits=4,
                 per_sequence=False, t_stride=None, seed=0, chunk=None):
        from kernelverify_amd import hip
        from kernelverify_amd.hip import DeviceArray
        from kernelverify_amd.pack import kv_attention
        from kernelverify_amd.pack.quant import quantize_affine

        self.lengths = [int(t) for t in lengths]
        b = len(self.lengths)
        t_stride = t_stride or max(self.lengths)
        self.bits, self.b, self.h, self.hkv, self.dh = bits, b, n_heads, n_kv_heads, head_dim
        self.per_sequence = per_sequence
        c = b if per_sequence else 1
        lens = "x".join(map(str, self.lengths)) if b <= 2 else f"{b} seqs"
        self.name = f"kv {bits}b B{b} H{n_heads}/{n_kv_heads} DH{head_dim} T{lens}"
        rng = np.random.default_rng(seed)
        self.q = rng.standard_normal((b, n_heads, head_dim)).astype(np.float16)
        self.nk = rng.standard_normal((b, n_kv_heads, head_dim)).astype(np.float16)
        self.nv = rng.standard_normal((b, n_kv_heads, head_dim)).astype(np.float16)
        self.k_raw = rng.standard_normal((c, n_kv_heads, t_stride, head_dim)).astype(np.float16)
        self.v_raw = rng.standard_normal((c, n_kv_heads, t_stride, head_dim)).astype(np.float16)
        shape = (c, n_kv_heads, t_stride, head_dim) if per_sequence else (n_kv_heads, t_stride,
                                                                          head_dim)
        k = quantize_affine(DeviceArray.from_host(self.k_raw.reshape(shape)), bits)
        v = quantize_affine(DeviceArray.from_host(self.v_raw.reshape(shape)), bits)
        hip.synchronize()
        self._parts = (k, v)
        self.bytes = kv_attention.algorithmic_bytes(self.lengths, n_heads, n_kv_heads, head_dim,
                                                    bits)
        cache_bytes = sum(a.nbytes for a in (*k, *v))
        copies = max(2, -(-ROTATION_BYTES // cache_bytes))
        self.dq = DeviceArray.from_host(self.q)
        self.dnk, self.dnv = DeviceArray.from_host(self.nk), DeviceArray.from_host(self.nv)
        self.dt = DeviceArray.from_host(np.array(self.lengths, dtype=np.int32))
        self.out = DeviceArray((b, n_heads, head_dim), np.float16)
        self.calls = []
        ws = None
        for i in range(copies):
            parts = [a if i == 0 else DeviceArray.from_host(a.to_host()) for a in (*k, *v)]
            call = kv_attention.KvDecodeCall(self.dq, *parts[:3], *parts[3:], self.dnk, self.dnv,
                                             self.dt, self.out, bits=bits,
                                             cache_per_sequence=per_sequence, workspace=ws,
                                             chunk=chunk or 0)
            ws = call.workspace
            self.calls.append(call)
        self.i = 0

    def step(self, stream):
        self.calls[self.i % len(self.calls)](stream)
        self.i += 1

    def gpu_output(self):
        from kernelverify_amd import hip

        self.step(None)
        hip.synchronize()
        return self.out.to_host()

    def cpu_fn(self):
        """The CPU decode step on the same stored caches (downloaded once)."""
        k, v = ([a.to_host() for a in parts] for parts in self._parts)
        return lambda: kv_cpu_path(self.q, self.nk, self.nv, k, v, self.lengths, self.bits,
                                   self.per_sequence)

    def check(self, got):
        """max |gpu - fp64 reference| against 4 eps16 max|ref|, per sequence."""
        from oracle.extensions import kv_reference_gqa

        worst = 0.0
        for i, t in enumerate(self.lengths):
            c = i if self.per_sequence else 0
            ref = kv_reference_gqa(self.q[i:i + 1], self.k_raw[c][:, :t], self.v_raw[c][:, :t],
                                   self.nk[i:i + 1], self.nv[i:i + 1], self.bits)
            err = float(np.max(np.abs(got[i:i + 1].astype(np.float64) - ref)))
            worst = max(worst, err / (4 * 9.77e-4 * float(np.max(np.abs(ref)))))
        return worst


class MoeWorkload:
    """One MoE decode step of BASELINE config 5: route top-8 of 128 experts
    from fp32 N(0, 1) logits, then the SwiGLU experts (gate/up 768 x 2048,
    down 2048 x 768, 4-bit) for n tokens, as one kvp_moe_route_swiglu call.
    Expert sets rotate over >= 1 GiB."""

    def __init__(self, n, n_experts=128, k=8, d_model=2048, d_ffn=768, bits=4, seed=0):
        from kernelverify_amd import hip
        from kernelverify_amd.hip import DeviceArray
        from kernelverify_amd.pack import moe_dispatch as moe
        from kernelverify_amd.pack.quant import quantize_affine

        self.n, self.e, self.k, self.dm, self.df, self.bits = n, n_experts, k, d_model, d_ffn, bits
        self.name = f"moe {bits}b E{n_experts} top{k} {d_model}/{d_ffn} n{n}"
        rng = np.random.default_rng(seed)
        self.x = rng.standard_normal((n, d_model)).astype(np.float16)
        self.logits = rng.standard_normal((n, n_experts)).astype(np.float32)
        self.raw = [(rng.standard_normal(shape) * 0.02).astype(np.float16)
                    for shape in ((n_experts, d_ffn, d_model), (n_experts, d_ffn, d_model),
                                  (n_experts, d_model, d_ffn))]
        mats = [quantize_affine(DeviceArray.from_host(w), bits) for w in self.raw]
        hip.synchronize()
        self._mats = mats
        set_bytes = sum(a.nbytes for m in mats for a in m)
        copies = max(2, -(-ROTATION_BYTES // set_bytes))
        self.dx = DeviceArray.from_host(self.x)
        self.dl = DeviceArray.from_host(self.logits)
        self.idx = DeviceArray((n, k), np.uint32)
        self.gate = DeviceArray((n, k), np.float32)
        self.out = DeviceArray((n, d_model), np.float16)
        self.calls = []
        ws = None
        for i in range(copies):
            m = mats if i == 0 else [tuple(DeviceArray.from_host(a.to_host()) for a in t)
                                     for t in mats]
            call = moe.SwigluCall(self.dx, self.idx, self.gate, *m, self.out, bits=bits,
                                  workspace=ws, logits=self.dl)
            ws = call.workspace
            self.calls.append(call)
        moe.route_logits(self.dl, self.idx, self.gate, k)
        hip.synchronize()
        self.routed = self.idx.to_host()
        self.bytes = moe.algorithmic_bytes(self.routed, n_experts, d_model, d_ffn, bits)
        self.unique = len(np.unique(self.routed))
        self.i = 0

    def step(self, stream):
        # routing from the logits and the experts: one kvp_moe_route_swiglu
        self.calls[self.i % len(self.calls)](stream)
        self.i += 1

    def gpu_output(self):
        from kernelverify_amd import hip

        self.step(None)
        hip.synchronize()
        return self.out.to_host()

    def cpu_fn(self):
        """The CPU MoE step from the same logits and stored experts."""
        host = [tuple(a.to_host() for a in m) for m in self._mats]
        return lambda: moe_cpu_path(self.x, self.logits, self.k, *host, self.bits)

    def check(self, got, tokens=(0,)):
        """Error over 4 eps16 max|ref| on a few tokens (fp64 SwiGLU reference)."""
        from oracle.extensions import artefact_from_arrays, route_topk, swiglu_reference
        from oracle.quant_contract import QuantContract, canonical_quantize

        idx, gate = route_topk(self.logits, self.k)
        worst = 0.0
        for t in tokens:
            used = sorted(set(int(e) for e in idx[t]))
            arts = []
            for w in self.raw:
                per = {}
                for e in used:
                    per[e] = canonical_quantize(w[e], QuantContract(bits=self.bits, group_size=64))
                arts.append(per)
            ref = swiglu_reference(self.x[t:t + 1], idx[t:t + 1], gate[t:t + 1], *arts)
            err = float(np.max(np.abs(got[t:t + 1].astype(np.float64) - ref)))
            worst = max(worst, err / (4 * 9.77e-4 * float(np.max(np.abs(ref)))))
        return worst


# The rows beside the headline, in bench order.
SECONDARY_QMV = ((4096, 4096, 4, 1), (14336, 4096, 8, 1), (14336, 4096, 4, 4),
                 (14336, 4096, 4, 8), (4096, 14336, 4, 1))
MOE_TOKENS = (1, 8, 32)


def kv_rows() -> list[dict]:
    """KvWorkload arguments: the 32k target, config 3, config 4 (seed-0 lengths)."""
    return [dict(lengths=[32768], bits=4), dict(lengths=[8192], bits=8),
            dict(lengths=list(np.random.default_rng(0).integers(1024, 32769, 8)), bits=4,
                 per_sequence=True, t_stride=32768)]


def row_factories() -> list:
    """One constructor per bench row, headline first."""
    rows = [lambda: QmvWorkload(14336, 4096, 4, 1)]
    rows += [lambda c=c: QmvWorkload(*c, seed=1) for c in SECONDARY_QMV]
    rows += [lambda kw=kw: KvWorkload(**kw) for kw in kv_rows()]
    rows += [lambda n=n: MoeWorkload(n) for n in MOE_TOKENS]
    return rows


ROUNDS = 7          # replays of one K-launch graph per row (bench/interleave.py:38-103)
SPREAD_LIMIT = 1.5  # max/min of a row's rounds above which the row is re-timed, then rejected
MIN_SAMPLE_MS = 5.0  # the reference's floor for one timed sample (interleave.py:38)


class Timing:
    """Rounds of one row: per-call ms of each replay of a graph of exactly
    ``steps`` launches, timed by event-record nodes inside the graph."""

    def __init__(self, steps: int, round_ms: list[float], in_graph: bool, retried: bool):
        self.steps = steps
        self.round_ms = round_ms
        self.in_graph = in_graph
        self.retried = retried

    @property
    def ms(self) -> float:
        return float(np.median(self.round_ms))

    @property
    def spread(self) -> float:
        return max(self.round_ms) / min(self.round_ms)

    @property
    def ok(self) -> bool:
        return self.spread <= SPREAD_LIMIT

    def summary(self) -> dict:
        return {"rounds": len(self.round_ms), "launches_per_round": self.steps,
                "median_us": round(self.ms * 1e3, 3),
                "min_us": round(min(self.round_ms) * 1e3, 3),
                "max_us": round(max(self.round_ms) * 1e3, 3),
                "spread": round(self.spread, 4), "spread_ok": self.ok,
                "events": "inside the graph" if self.in_graph else "around the graph launch"}


def time_rounds(workload, steps: int, warmup: int, rounds: int = ROUNDS) -> Timing:
    """ms per call: ``rounds`` replays of one HIP graph holding EXACTLY
    ``steps`` back-to-back launches (the weights rotating over >= 1 GiB).

    The start and stop events are event-record nodes inside the graph, so
    the host's graph-launch latency is outside the window: each round is the
    device's own time for ``steps`` calls, as a serving loop that replays a
    captured decode step sees it. The value is the median over rounds; a row
    whose max/min over rounds exceeds SPREAD_LIMIT is timed again once and
    reported with ``spread_ok`` false if it still does (the reference's
    reference-arm rule, bench/interleave.py:48, :77-103).
    """
    from kernelverify_amd import hip

    stream = hip.Stream()
    for _ in range(warmup):
        workload.step(stream)
    hip.synchronize()
    start, stop = hip.Event(), hip.Event()

    def body(external: bool):
        (start.record_external if external else start.record)(stream)
        for _ in range(steps):
            workload.step(stream)
        (stop.record_external if external else stop.record)(stream)

    in_graph = True
    try:
        g = hip.Graph(stream, lambda: body(True))
    except hip.HipError as exc:  # a runtime without event nodes: events around the launch
        log(f"[bench] event nodes unavailable ({exc}); timing around the graph launch")
        in_graph = False
        g = hip.Graph(stream, lambda: [workload.step(stream) for _ in range(steps)])

    def one_round() -> float:
        if in_graph:
            g.launch()
        else:
            start.record(stream)
            g.launch()
            stop.record(stream)
        stream.synchronize()
        return start.elapsed_ms(stop) / steps

    one_round()  # the replay itself warmed once
    hip.synchronize()
    t = Timing(steps, [one_round() for _ in range(rounds)], in_graph, False)
    if not t.ok:
        t = Timing(steps, [one_round() for _ in range(rounds)], in_graph, True)
    hip.synchronize()
    g.destroy()
    return t


def sample_steps(workload, warmup: int, floor: int) -> int:
    """Launches per round for a secondary row: at least ``floor`` and at
    least MIN_SAMPLE_MS of back-to-back launches (one short probe round)."""
    probe = time_rounds(workload, 20, warmup, rounds=1)
    return max(floor, int(np.ceil(MIN_SAMPLE_MS / max(probe.ms, 1e-6))))


def cpu_baseline(fn, budget_s: float = 12.0, min_reps: int = 20):
    """Best and median wall time of the CPU path: at least ``min_reps`` calls
    (the reference found best-of-5 unstable on CPU), more while ``budget_s``
    lasts, at most 50."""
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < min_reps or (time.perf_counter() < t_end and len(times) < 50):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return min(times), float(np.median(times)), len(times)


def host_dequant(words: np.ndarray, scales: np.ndarray, biases: np.ndarray, bits: int):
    """fp32 s * q + b of an MLX-affine artefact held on the host (4- or 8-bit
    code streams: byte j holds codes 2j, 2j+1 at 4 bits, code j at 8)."""
    b = np.ascontiguousarray(words).view(np.uint8)
    if bits == 4:
        q = np.empty(b.shape[:-1] + (2 * b.shape[-1],), dtype=np.float32)
        q[..., 0::2] = b & 15
        q[..., 1::2] = b >> 4
    elif bits == 8:
        q = b.astype(np.float32)
    else:
        raise ValueError(f"host_dequant: bits={bits}")
    s = np.repeat(scales.astype(np.float32), 64, axis=-1)
    return q * s + np.repeat(biases.astype(np.float32), 64, axis=-1)


def kv_cpu_path(q, new_k, new_v, k_parts, v_parts, lengths, bits, per_sequence):
    """The CPU decode step (reference/native_kernels.py:168-221 semantics, fp32
    numpy + BLAS) from the stored quantized caches: per sequence, dequantize
    its T rows, scores over T + 1 with the new entry, softmax, values.
    q (B, H, DH); caches (C, HKV, T_stride, ...) or (HKV, T_stride, ...)."""
    b, h, dh = q.shape
    hkv = new_k.shape[1]
    g = h // hkv
    scale = np.float32(1.0 / np.sqrt(dh))
    out = np.empty((b, h, dh), dtype=np.float32)
    for i, t in enumerate(lengths):
        sel = (lambda a: a[i][:, :t]) if per_sequence else (lambda a: a[:, :t])
        kd = host_dequant(*(sel(a) for a in k_parts), bits)          # (HKV, T, DH)
        vd = host_dequant(*(sel(a) for a in v_parts), bits)
        qg = q[i].astype(np.float32).reshape(hkv, g, dh)
        s = np.matmul(qg, kd.transpose(0, 2, 1)) * scale             # (HKV, G, T)
        s_new = np.einsum("kgd,kd->kg", qg, new_k[i].astype(np.float32)) * scale
        m = np.maximum(s.max(axis=-1), s_new)
        p = np.exp(s - m[..., None])
        p_new = np.exp(s_new - m)
        o = np.matmul(p, vd) + p_new[..., None] * new_v[i].astype(np.float32)[:, None, :]
        out[i] = (o / (p.sum(axis=-1) + p_new)[..., None]).reshape(h, dh)
    return out


def moe_cpu_path(x, logits, k, gate_parts, up_parts, down_parts, bits):
    """The CPU MoE step (reference/native_kernels.py:104-147 semantics at top-k,
    SwiGLU experts; fp32 numpy + BLAS): softmax over all experts, top-k by
    probability (ties low), renormalised; each routed expert's three
    projections dequantized once per step and applied to its tokens."""
    p = np.exp(logits - logits.max(axis=-1, keepdims=True))
    p /= p.sum(axis=-1, keepdims=True)
    top = np.argsort(-p, axis=-1, kind="stable")[:, :k]
    w = np.take_along_axis(p, top, axis=-1)
    w /= w.sum(axis=-1, keepdims=True)
    xf = x.astype(np.float32)
    out = np.zeros((x.shape[0], down_parts[0].shape[1]), dtype=np.float32)
    for e in np.unique(top):
        rows, slots = np.nonzero(top == e)
        wg = host_dequant(*(a[e] for a in gate_parts), bits)
        wu = host_dequant(*(a[e] for a in up_parts), bits)
        wd = host_dequant(*(a[e] for a in down_parts), bits)
        gx, ux = xf[rows] @ wg.T, xf[rows] @ wu.T
        hidden = gx / (1.0 + np.exp(-gx)) * ux
        np.add.at(out, rows, w[rows, slots][:, None] * (hidden @ wd.T))
    return out


def blas_vendor() -> str:
    try:
        return str(np.show_config(mode="dicts")["Build Dependencies"]["blas"]["name"])
    except Exception:
        return "unknown"


def cpu_row(workload, gpu_out, what: str) -> dict | None:
    """The CPU path of a KV or MoE row on the same inputs, a bounded sample
    (at least 20 calls), after a check of its output against the
    verified GPU output; None (logged) if they disagree."""
    fn = workload.cpu_fn()
    ref = np.asarray(gpu_out, dtype=np.float64)
    got = np.asarray(fn(), dtype=np.float64).reshape(ref.shape)
    if not np.max(np.abs(got - ref)) <= 4 * 9.77e-4 * np.max(np.abs(ref)):
        log(f"[bench] CPU path of {workload.name} disagrees with the GPU output; not timed")
        return None
    best, med, n = cpu_baseline(fn, budget_s=4.0, min_reps=20)
    return {"us_per_call": round(best * 1e6, 1), "median_us": round(med * 1e6, 1),
            "GBps": round(workload.bytes / best / 1e9, 3), "calls": n, "cores": blas_threads(),
            "kind": "port", "path": what}


TRAFFIC_FILE = ROOT / "profiles" / "qmv_4b_14336x4096_m1.traffic.json"


def measured_traffic():
    """HBM bytes per headline launch from the committed rocprofv3 --pmc runs
    (FETCH_SIZE + WRITE_SIZE per dispatch, each scaled by the same counter's
    reading on a copy kernel of known size); None before that profile exists."""
    try:
        return json.loads(TRAFFIC_FILE.read_text())["traffic_bytes"]
    except (OSError, KeyError, ValueError):
        return None


def blas_threads() -> int:
    try:
        from threadpoolctl import threadpool_info

        info = [i for i in threadpool_info() if i.get("user_api") == "blas"]
        return int(info[0]["num_threads"]) if info else 1
    except Exception:
        return int(os.environ.get("OMP_NUM_THREADS", "1"))


ISSUE_FILE = ROOT / "profiles" / "issue_counts_bench.json"


def trace_steps(steps: int, replays: int = 3) -> int:
    """The program the kernel-trace profile runs: every row's step captured
    ``steps`` times back to back in one HIP graph with no event nodes (the
    profiler does not follow event-record nodes), replayed ``replays``
    times, so each kernel runs as it does inside the timed region."""
    from kernelverify_amd import hip

    stream = hip.Stream()
    for make in row_factories():
        w = make()
        w.step(stream)
        stream.synchronize()
        g = hip.Graph(stream, lambda: [w.step(stream) for _ in range(steps)])
        for _ in range(replays):
            g.launch()
        stream.synchronize()
        g.destroy()
        log(f"[trace] {w.name}: {replays} x {steps} steps")
        del w
    print(json.dumps({"trace_steps": steps, "replays": replays}), flush=True)
    return 0


def issue_profile(steps: int) -> int:
    """The program the instruction-count passes profile: every row's step
    ``steps`` times between tag launches (kernelverify_amd/counters.py reads
    the dispatches back by the tags), then the manifest line."""
    from kernelverify_amd import counters, hip, lib

    L = lib.load()
    sink = hip.DeviceArray((len(row_factories()) + 1,), np.float32)
    names = []
    for i, make in enumerate(row_factories()):
        w = make()
        hip.synchronize()
        lib.check(L.kvp_probe_compute(0, i + 1, 1, sink.ptr, None))  # open tag: row i
        for _ in range(steps):
            w.step(None)
            hip.synchronize()
        lib.check(L.kvp_probe_compute(1, 1, 1, sink.ptr, None))  # close tag
        hip.synchronize()
        names.append(w.name)
        log(f"[issue] row {i}: {w.name}, {steps} steps")
        del w
    print(json.dumps({"issue_rows": names, "steps": steps,
                      "kernel_source_sha256": counters.library_source_sha256()}), flush=True)
    return 0


class IssueBounds:
    """min(HBM, VALU, matrix core) per row: the committed per-call
    instruction counts (rocprofv3 over ``--issue-profile``) at the issue
    rates the compute probes measure in this run."""

    def __init__(self):
        from kernelverify_amd import counters, roofline

        self.counters = counters
        try:
            data = json.loads(ISSUE_FILE.read_text())
        except (OSError, ValueError):
            data = {"rows": {}}
        self.rows = data.get("rows", {})
        self.current = data.get("kernel_source_sha256") == counters.library_source_sha256()
        c = roofline.compute_ceilings(blocks=256 * 8, iters=1024)
        fma = c[roofline.COMPUTE_KINDS[0]]["TFLOPs"] * 1e12
        dot2 = c[roofline.COMPUTE_KINDS[1]]["TFLOPs"] * 1e12
        self.rates = {"valu_wave_insts_per_s": fma / (2 * 64),
                      "dot2_wave_insts_per_s": dot2 / (4 * 64),
                      "mfma_f16_flops_per_s": c[roofline.COMPUTE_KINDS[2]]["TFLOPs"] * 1e12}

    def summary(self) -> dict:
        return {"rates": {k: round(v / 1e9, 1) for k, v in self.rates.items()},
                "rates_unit": "G per s (wave-instructions, flops)",
                "counts": ISSUE_FILE.name, "counts_match_source": self.current,
                "valu_rate_from": "fp32 FMA probe (the fastest VALU instruction measured; "
                                  "valu_us is a lower bound)"}

    def row(self, name: str, nbytes: int, achieved_GBps: float) -> dict | None:
        work = self.counters.issue_work(self.rows.get(name, {}).get("per_call", {}))
        if work is None:
            return None
        out = self.counters.issue_bound(nbytes, achieved_GBps, work, self.rates, PEAK_HBM_GBS)
        if not self.current:
            out["counts_stale"] = True
        return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-secondary", action="store_true",
                    help="skip the other BASELINE qmv configs (configs 1 and 2 beside the headline)")
    ap.add_argument("--headline-only", action="store_true",
                    help="time only the headline qmv workload (profiling runs)")
    ap.add_argument("--trace-steps", type=int, default=0, metavar="K",
                    help="kernel-trace program: every row's step K times in a graph, then exit")
    ap.add_argument("--issue-profile", type=int, default=0, metavar="S",
                    help="run every row S times between tag launches, for rocprofv3 counter "
                         "passes (kernelverify_amd/counters.py); no timing")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported by this build "
              "(every GPU box has one MI355X; the multi-GPU sharding is a design note)",
              file=sys.stderr)
        return 2

    from kernelverify_amd import hip, lib, roofline

    if hip.device_count() == 0:
        print("bench.py: no HIP device visible", file=sys.stderr)
        return 3
    lib.load()
    if args.issue_profile:
        return issue_profile(args.issue_profile)
    if args.trace_steps:
        return trace_steps(args.trace_steps)

    head = row_factories()[0]()
    log(f"[bench] {head.name}: {len(head.copies)} artefact copies, "
        f"{head.bytes} algorithmic bytes/launch")

    # Verify first: GPU output against the CPU path on the same inputs.
    got = head.gpu_output()
    ref_fn = head.cpu_reference()
    ref = ref_fn()
    err = float(np.max(np.abs(got.astype(np.float64) - ref.astype(np.float64))))
    tol = 4 * 9.77e-4 * float(np.max(np.abs(ref.astype(np.float64))))
    log(f"[bench] verify {head.name}: max|gpu-cpu| {err:.3e} (bound {tol:.3e})")
    if not err <= tol:
        print(f"bench.py: verification failed for {head.name}", file=sys.stderr)
        return 1

    timing = time_rounds(head, args.steps, args.warmup)
    ms = timing.ms
    us = ms * 1e3
    log(f"[bench] {head.name} rounds: {timing.summary()}")
    # the same kernel over samples of at least MIN_SAMPLE_MS, as a cross-check
    # of the K-launch figure (not the value)
    long = time_rounds(head, sample_steps(head, 0, args.steps), 0)
    gbs = head.bytes / (ms * 1e-3) / 1e9
    log(f"[bench] {head.name}: {us:.3f} us/call, {gbs:.1f} GB/s ({100 * gbs / PEAK_HBM_GBS:.1f}%)")

    # The measured ceiling for the same shape of work: back-to-back probe
    # reads of the headline's bytes per launch (scored against its own
    # ceiling as well as the spec).
    ceiling = None
    bounds = IssueBounds()
    log(f"[bench] issue rates: {bounds.summary()}")
    if not args.headline_only:
        c_gbs, c_us, c_shape = roofline.best_read_like(head.bytes)
        ceiling = {"GBps": round(c_gbs, 1), "us_per_launch": round(c_us, 3),
                   "frac": round(gbs / c_gbs, 4), "probe_shape": c_shape,
                   "probe": "kvp_probe_read_tiled, back-to-back launches reading the same bytes "
                            "per launch from a >= 1 GiB rotation, fastest of the sweep's leading "
                            "shapes (roofline.best_read_like)"}
        log(f"[bench] measured read ceiling at {head.bytes} B/launch: {ceiling}")

    secondary = []
    if not (args.no_secondary or args.headline_only):
        for c in SECONDARY_QMV:
            w = QmvWorkload(*c, seed=1)
            g = w.gpu_output()
            r = w.cpu_reference()()
            e = float(np.max(np.abs(g.astype(np.float64) - r)))
            t = 4 * 9.77e-4 * float(np.max(np.abs(r)))
            if not e <= t:
                log(f"[bench] verify FAILED {w.name}: {e:.3e} > {t:.3e}")
                continue
            t2 = time_rounds(w, sample_steps(w, args.warmup, max(200, args.steps // 2)), 0)
            ms2 = t2.ms
            secondary.append({"workload": w.name, "us_per_call": round(ms2 * 1e3, 3),
                              "GBps": round(w.bytes / (ms2 * 1e-3) / 1e9, 1),
                              "frac_8TBps": round(w.bytes / (ms2 * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                              "timing": t2.summary(),
                              "valu_bound": bounds.row(w.name, w.bytes,
                                                       w.bytes / (ms2 * 1e-3) / 1e9)})
            log(f"[bench] {secondary[-1]}")
            del w

    kv = []
    for kw in () if args.headline_only else kv_rows():
        w = KvWorkload(**kw)
        got = w.gpu_output()
        ratio = w.check(got)
        if not ratio <= 1.0:
            log(f"[bench] verify FAILED {w.name}: error {ratio:.2f} x bound")
            continue
        t2 = time_rounds(w, sample_steps(w, args.warmup, max(200, args.steps // 2)), 0)
        ms2 = t2.ms
        gbs2 = w.bytes / (ms2 * 1e-3) / 1e9
        kv.append({"workload": w.name, "us_per_call": round(ms2 * 1e3, 3), "GBps": round(gbs2, 1),
                   "frac_8TBps": round(gbs2 / PEAK_HBM_GBS, 4), "bytes": w.bytes,
                   "verify_err_over_bound": round(ratio, 4), "timing": t2.summary()})
        kv[-1]["frac_measured_ceiling"] = round(gbs2 / roofline.best_read_like(w.bytes)[0], 4)
        kv[-1]["valu_bound"] = bounds.row(w.name, w.bytes, gbs2)
        if not args.no_cpu:
            kv[-1]["cpu"] = cpu_row(w, got, "dequantize the stored caches, fp32 scores, "
                                    "softmax over T + 1, values (native_kernels.py:168-221)")
        log(f"[bench] {kv[-1]}")
        del w

    moe_rows = []
    for n in () if args.headline_only else MOE_TOKENS:
        w = MoeWorkload(n)
        got = w.gpu_output()
        ratio = w.check(got, tokens=(0, n - 1) if n > 1 else (0,))
        if not ratio <= 1.0:
            log(f"[bench] verify FAILED {w.name}: error {ratio:.2f} x bound")
            continue
        t3 = time_rounds(w, sample_steps(w, args.warmup, max(100, args.steps // 4)), 0)
        ms3 = t3.ms
        gbs3 = w.bytes / (ms3 * 1e-3) / 1e9
        moe_rows.append({"workload": w.name, "us_per_call": round(ms3 * 1e3, 3),
                         "GBps": round(gbs3, 1), "frac_8TBps": round(gbs3 / PEAK_HBM_GBS, 4),
                         "unique_experts": w.unique, "bytes": w.bytes,
                         "verify_err_over_bound": round(ratio, 4), "timing": t3.summary()})
        moe_rows[-1]["frac_measured_ceiling"] = round(gbs3 / roofline.best_read_like(w.bytes)[0], 4)
        moe_rows[-1]["valu_bound"] = bounds.row(w.name, w.bytes, gbs3)
        if not args.no_cpu:
            moe_rows[-1]["cpu"] = cpu_row(w, got, "softmax top-8 routing, each routed expert's "
                                          "gate/up/down dequantized once, fp32 SwiGLU "
                                          "(native_kernels.py:104-147 at top-k)")
        log(f"[bench] {moe_rows[-1]}")
        del w

    cpu = None
    if not args.no_cpu:
        best, med, n = cpu_baseline(ref_fn)
        cpu = {"value": round(head.bytes / best / 1e9, 3), "unit": "GB/s",
               "cores": blas_threads(), "kind": "port",
               "sample": f"{n} calls of the numpy control path (fp32 dequant + BLAS sgemv, "
                         f"native_kernels.py:66-83) on the same 14336x4096 4-bit artefact; "
                         f"best {best * 1e3:.1f} ms, median {med * 1e3:.1f} ms; "
                         f"host {platform.processor() or platform.machine()}, "
                         f"os.cpu_count()={os.cpu_count()}"}
        wdq = host_dequant(head.w_q, head.scales, head.biases, 4)
        x32 = head.x.astype(np.float32)
        best_mm, _, n_mm = cpu_baseline(lambda: x32 @ wdq.T, budget_s=3.0)
        del wdq
        cpu["matmul_only_value"] = round(head.bytes / best_mm / 1e9, 3)
        cpu["blas"] = blas_vendor()
        cpu["sample"] += (f"; upper bound: BLAS sgemv alone on the weights dequantized "
                          f"beforehand, best of {n_mm}, {best_mm * 1e3:.1f} ms "
                          f"(matmul_only_value)")
        log(f"[bench] cpu baseline: {cpu}")

    line = {
        "metric": METRIC, "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 6),
        "us_per_call": round(us, 3), "timing": timing.summary(),
        "timing_5ms_samples": long.summary(), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "u4 codes x f16 -> f32 accumulate",
        "data": "synthetic (BASELINE configs[1] distributions, seed 0)",
        "config": {"workload": head.name, "d_out": 14336, "d_in": 4096, "bits": 4, "group": 64,
                   "batch": 1, "rotation_copies": len(head.copies)},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                     "traffic": measured_traffic(), "measured_ceiling": ceiling,
                     "valu_bound": bounds.row(head.name, head.bytes, gbs),
                     "issue_rates": bounds.summary()},
        "cpu_baseline": cpu,
    }
    if secondary:
        line["secondary"] = secondary
    if kv:
        line["kv_decode"] = kv
    if moe_rows:
        line["moe"] = moe_rows
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
