"""Price the qmv routing boundary on MI355X (reference:
bench/price_qmv_boundary.py, whose classify rule is :221-250).

`wide_qmv.should_dispatch(m, bits, d_out, d_in)` routes a (tile width, bit
width, shape) cell to the pack only where a recording says the pack wins
there. This probe makes that recording. Two arms per cell:

- ours: `kvp_qmv` on the resident artefact (codes + fp16 scales/biases);
- the incumbent: what a ROCm server runs for the same layer when the pack
  does not serve it, the vendor fp16 GEMM on fp16 weights held in HBM
  (rocBLAS `gemm_ex`, fp16 in/out, fp32 compute, `out = x @ W^T`). Its
  weights are the fp16 matrix the artefact was quantized from: a
  dequantized copy has the same shape and dtype, and a GEMM's time does not
  depend on the values. The incumbent's numerics are not judged here.

Verification precedes timing, as in the reference (:1-20): for every
(shape, bits) the GPU quantizer's artefact is checked byte-identical to the
canonical quantizer on a row subset, and every M = 1..16 is judged against
the oracle's quantized_matmul reference and tolerance on that row subset
(rows are independent: a row's output depends on its own weights only). One
failure and the run writes nothing.

Timing, after the reference's discipline: both arms are captured as HIP
graphs of back-to-back launches (so the host's launch cost, which differs
between a ctypes call and a BLAS call, is not what gets timed), each sample
is one replay of at least MIN_SAMPLE_MS over a rotation of distinct weight
copies totalling >= 1 GiB (more than the 256 MB Infinity Cache), the two
arms alternate within each of ROUNDS rounds, and `classify` applies the
interval rule: REJECTED when the incumbent's own spread exceeds
MAX_CANARY_SPREAD, WIN / LOSS only when the whole ratio interval
[min(incumbent)/max(ours), max(incumbent)/min(ours)] clears 1.0, else
REFUSED.

    python -m tests.gates.price_qmv_boundary --out /tmp/qmv-boundary-pricing-mi355x.json
"""

from __future__ import annotations

import argparse
import ctypes
import datetime as _dt
import json
import math
import statistics
import sys
import time
from dataclasses import asdict, dataclass

import numpy as np

from kernelverify_amd import hip, lib
from kernelverify_amd.pack import wide_qmv
from kernelverify_amd.pack.codes import pack_codes
from kernelverify_amd.pack.quant import quantize_affine
from oracle.quant_contract import QuantContract, canonical_quantize
from oracle.verify import judge, qmv_inputs, reference_and_tolerance

# The six decode dispatch shapes the reference priced (Qwen3-4B, its
# recording bench/results/qmv-boundary-pricing-2026-08-15.json) and the
# three BASELINE qmv shapes.
SITES = (
    ("q_proj", 4096, 2560),
    ("k_proj/v_proj", 1024, 2560),
    ("o_proj", 2560, 4096),
    ("gate_proj/up_proj", 9728, 2560),
    ("down_proj", 2560, 9728),
    ("lm_head", 151936, 2560),
    ("baseline 4096x4096", 4096, 4096),
    ("baseline 14336x4096", 14336, 4096),
    ("baseline 4096x14336", 4096, 14336),
)
BITS = (2, 3, 4, 8)
M_SWEEP = tuple(range(1, 17))
ROUNDS = 7
MIN_SAMPLE_MS = 5.0
WORKING_SET_BYTES = 1 << 30
MAX_CANARY_SPREAD = 1.5
CHECK_ROWS = 256
MAX_LAUNCHES = 20000
INCUMBENT = ("rocBLAS gemm_ex fp16 x fp16 -> fp16, fp32 compute, out = x @ W^T with W "
             "(d_out, d_in) fp16 resident; HIP-graph replay")


@dataclass(frozen=True)
class PricedPoint:
    site: str
    bits: int
    d_out: int
    d_in: int
    m: int
    r: int
    verdict: str
    ratio: float
    ratio_lo: float
    ratio_hi: float
    spread_ours: float
    spread_incumbent: float
    ours_us: float
    incumbent_us: float
    samples_ours_us: tuple
    samples_incumbent_us: tuple


def classify(ours: list, incumbent: list, *, site: str = "", bits: int = 0, d_out: int = 0,
             d_in: int = 0, m: int = 0, r: int = 0) -> PricedPoint:
    """The verdict for one cell from the two arms' per-round samples
    (seconds per call). Ratio = incumbent time / our time: above 1 we win."""
    spread_ours = max(ours) / min(ours)
    spread_inc = max(incumbent) / min(incumbent)
    ratio = statistics.median(incumbent) / statistics.median(ours)
    ratio_lo = min(incumbent) / max(ours)
    ratio_hi = max(incumbent) / min(ours)
    if spread_inc > MAX_CANARY_SPREAD:
        verdict = "REJECTED"
    elif ratio_lo > 1.0:
        verdict = "WIN"
    elif ratio_hi < 1.0:
        verdict = "LOSS"
    else:
        verdict = "REFUSED"
    return PricedPoint(site=site, bits=bits, d_out=d_out, d_in=d_in, m=m, r=r, verdict=verdict,
                       ratio=ratio, ratio_lo=ratio_lo, ratio_hi=ratio_hi,
                       spread_ours=spread_ours, spread_incumbent=spread_inc,
                       ours_us=statistics.median(ours) * 1e6,
                       incumbent_us=statistics.median(incumbent) * 1e6,
                       samples_ours_us=tuple(s * 1e6 for s in ours),
                       samples_incumbent_us=tuple(s * 1e6 for s in incumbent))


# ---------------------------------------------------------------------------
# The incumbent arm
# ---------------------------------------------------------------------------
_OP_N, _OP_T = 111, 112            # rocblas_operation
_F16, _F32 = 150, 151              # rocblas_datatype


class VendorGemm:
    """`out (M, N) = x (M, K) @ W^T`, W (N, K) row-major, through rocBLAS.

    Column-major view: out^T (N x M, ld N) = W^T-op (W is K x N, ld K,
    transposed) times x^T (K x M, ld K). A user workspace is set so no call
    allocates (the calls are captured into graphs)."""

    def __init__(self, stream: hip.Stream, workspace_bytes: int = 128 << 20):
        for name in ("librocblas.so.5", "librocblas.so", "/opt/rocm/lib/librocblas.so"):
            try:
                self.rb = ctypes.CDLL(name)
                break
            except OSError:
                continue
        else:
            raise RuntimeError("rocBLAS is not loadable")
        vp, i = ctypes.c_void_p, ctypes.c_int
        self.rb.rocblas_create_handle.argtypes = [ctypes.POINTER(vp)]
        self.rb.rocblas_set_stream.argtypes = [vp, vp]
        self.rb.rocblas_set_workspace.argtypes = [vp, vp, ctypes.c_size_t]
        self.rb.rocblas_gemm_ex.argtypes = [vp, i, i, i, i, i, vp, vp, i, i, vp, i, i, vp, vp, i,
                                            i, vp, i, i, i, i, ctypes.c_int32, ctypes.c_uint32]
        self.rb.rocblas_destroy_handle.argtypes = [vp]
        self.handle = vp()
        self._check(self.rb.rocblas_create_handle(ctypes.byref(self.handle)), "create_handle")
        self._check(self.rb.rocblas_set_stream(self.handle, ctypes.c_void_p(stream.handle)),
                    "set_stream")
        self.workspace = hip.DeviceArray((workspace_bytes,), np.uint8)
        self._check(self.rb.rocblas_set_workspace(self.handle, ctypes.c_void_p(self.workspace.ptr),
                                                  workspace_bytes), "set_workspace")
        self.alpha, self.beta = ctypes.c_float(1.0), ctypes.c_float(0.0)

    @staticmethod
    def _check(status: int, what: str) -> None:
        if status != 0:
            raise RuntimeError(f"rocBLAS {what}: status {status}")

    def __call__(self, x_ptr: int, w_ptr: int, out_ptr: int, m: int, n: int, k: int) -> None:
        vp = ctypes.c_void_p
        self._check(self.rb.rocblas_gemm_ex(
            self.handle, _OP_T, _OP_N, n, m, k, ctypes.byref(self.alpha), vp(w_ptr), _F16, k,
            vp(x_ptr), _F16, k, ctypes.byref(self.beta), vp(out_ptr), _F16, n, vp(out_ptr), _F16,
            n, _F32, 0, 0, 0), "gemm_ex")

    def close(self) -> None:
        if self.handle:
            self.rb.rocblas_destroy_handle(self.handle)
            self.handle = ctypes.c_void_p()


# ---------------------------------------------------------------------------
# Timing
# ---------------------------------------------------------------------------
def _replay_seconds(graph: hip.Graph, stream: hip.Stream, launches: int) -> float:
    start, stop = hip.Event(), hip.Event()
    start.record(stream)
    graph.launch()
    stop.record(stream)
    stop.synchronize()
    return start.elapsed_ms(stop) * 1e-3 / launches


def _sized_graph(stream: hip.Stream, launch, copies: int) -> tuple[hip.Graph, int]:
    """A graph of enough back-to-back launches (cycling the weight copies) to
    last MIN_SAMPLE_MS, sized from a 64-launch trial graph."""
    trial = hip.Graph(stream, lambda: [launch(i % copies) for i in range(64)])
    trial.launch()
    stream.synchronize()
    per_call = min(_replay_seconds(trial, stream, 64) for _ in range(3))
    trial.destroy()
    n = int(min(MAX_LAUNCHES, max(64, math.ceil(MIN_SAMPLE_MS * 1e-3 / max(per_call, 1e-9)))))
    n = max(n, copies)  # every copy appears in every sample
    graph = hip.Graph(stream, lambda: [launch(i % copies) for i in range(n)])
    graph.launch()
    stream.synchronize()
    return graph, n


def price_cell(site, bits, m, d_out, d_in, ours_copies, inc_copies, gemm, stream):
    x = hip.DeviceArray.from_host(
        (np.random.default_rng(100 + m).standard_normal((m, d_in)).astype(np.float32)
         .astype(np.float16)))
    out_ours = hip.DeviceArray((m, d_out), np.float16)
    out_inc = hip.DeviceArray((m, d_out), np.float16)
    calls = [wide_qmv.QmvCall(x, wq, s, b, out_ours, bits=bits) for wq, s, b in ours_copies]

    def ours(i):
        calls[i](stream)

    def incumbent(i):
        gemm(x.ptr, inc_copies[i].ptr, out_inc.ptr, m, d_out, d_in)

    g_ours, n_ours = _sized_graph(stream, ours, len(calls))
    g_inc, n_inc = _sized_graph(stream, incumbent, len(inc_copies))
    a, b = [], []
    for _ in range(ROUNDS):
        a.append(_replay_seconds(g_ours, stream, n_ours))
        b.append(_replay_seconds(g_inc, stream, n_inc))
    g_ours.destroy()
    g_inc.destroy()
    return classify(a, b, site=site, bits=bits, d_out=d_out, d_in=d_in, m=m,
                    r=wide_qmv.rows_per_wave(m, bits, d_out, d_in))


# ---------------------------------------------------------------------------
# Verification
# ---------------------------------------------------------------------------
def check_rows(d_out: int) -> np.ndarray:
    rng = np.random.default_rng(d_out)
    edge = np.r_[np.arange(min(64, d_out)), np.arange(max(0, d_out - 64), d_out)]
    pick = rng.choice(d_out, size=min(CHECK_ROWS, d_out), replace=False)
    return np.unique(np.r_[edge, pick])


def verify_shape(w: np.ndarray, bits: int, artefact, out=print) -> dict:
    """Artefact identity and every M on the row subset; raises on a failure."""
    d_out, d_in = w.shape
    rows = check_rows(d_out)
    wq, s, b = (a.to_host() for a in artefact)
    art = canonical_quantize(w[rows], QuantContract(bits=bits, group_size=64))
    if not (np.array_equal(wq[rows], pack_codes(art.q, bits))
            and np.array_equal(s[rows], art.scales) and np.array_equal(b[rows], art.biases)):
        raise AssertionError(f"{d_out}x{d_in} {bits}-bit: GPU artefact differs from the "
                             "canonical quantizer")
    worst, cases = 0.0, 0
    rng = np.random.default_rng(11)
    for m in M_SWEEP:
        for scale in (1.0, 10.0):
            x = (rng.standard_normal((m, d_in)).astype(np.float32) * scale).astype(np.float16)
            x_dev, out_dev = hip.DeviceArray.from_host(x), hip.DeviceArray((m, d_out), np.float16)
            wide_qmv.run_qmv(x_dev, *artefact, out_dev, bits=bits)
            got = out_dev.to_host()
            ref, tol = reference_and_tolerance("quantized_matmul", qmv_inputs(x, w[rows], bits))
            v = judge(got[:, rows], ref, tol)
            cases += 1
            worst = max(worst, v.err / v.tol)
            if not v.ok:
                raise AssertionError(f"{d_out}x{d_in} {bits}-bit M={m} x{scale:g}: err "
                                     f"{v.err:.3e} > tol {v.tol:.3e}")
    out(f"  verified {d_out}x{d_in} {bits}-bit: artefact identical on {len(rows)} rows, "
        f"{cases} cases green (worst err/tol {worst:.3f})")
    return {"rows_checked": int(len(rows)), "cases": cases, "worst_err_over_tol": worst}


# ---------------------------------------------------------------------------
def machine() -> dict:
    name = ctypes.create_string_buffer(256)
    arch = ctypes.create_string_buffer(64)
    cus, threads, clock = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    lds, mem = ctypes.c_size_t(), ctypes.c_size_t()
    lib.check(lib.load().kvp_device_info(0, name, 256, arch, 64, ctypes.byref(cus),
                                         ctypes.byref(threads), ctypes.byref(lds),
                                         ctypes.byref(mem), ctypes.byref(clock)))
    ver = ctypes.c_int()
    rt = hip.runtime()
    rt.hipRuntimeGetVersion.argtypes = [ctypes.POINTER(ctypes.c_int)]
    rt.hipRuntimeGetVersion(ctypes.byref(ver))
    return {"device": name.value.decode(), "arch": arch.value.decode(),
            "compute_units": cus.value, "memory_bytes": mem.value, "clock_khz": clock.value,
            "hip_runtime_version": ver.value}


def run(sites=SITES, bits_list=BITS, out=print) -> dict:
    stream = hip.Stream()
    gemm = VendorGemm(stream)
    points, verification = [], {}
    started = time.time()
    for site, d_out, d_in in sites:
        rng = np.random.default_rng(7)
        w = (rng.standard_normal((d_out, d_in), dtype=np.float32) * 0.02).astype(np.float16)
        w_dev = hip.DeviceArray.from_host(w)
        inc_copies = [w_dev] + [hip.DeviceArray.from_host(w) for _ in
                                range(max(2, -(-WORKING_SET_BYTES // w.nbytes)) - 1)]
        for bits in bits_list:
            first = quantize_affine(w_dev, bits)
            verification[f"{site} {bits}-bit"] = verify_shape(w, bits, first, out=out)
            per_copy = wide_qmv.artefact_bytes(d_out, d_in, bits)
            n_copies = max(2, -(-WORKING_SET_BYTES // per_copy))
            ours = [first] + [quantize_affine(w_dev, bits) for _ in range(n_copies - 1)]
            hip.synchronize()
            for m in M_SWEEP:
                p = price_cell(site, bits, m, d_out, d_in, ours, inc_copies, gemm, stream)
                points.append(p)
                out(f"  {site:22s} {bits}-bit M={m:2d}  ours {p.ours_us:8.2f} us  incumbent "
                    f"{p.incumbent_us:8.2f} us  ratio {p.ratio:5.2f} "
                    f"[{p.ratio_lo:5.2f}, {p.ratio_hi:5.2f}]  {p.verdict}")
            del ours, first
        del inc_copies, w_dev
    gemm.close()
    return {
        "probe": "price_qmv_boundary",
        "date": _dt.date.today().isoformat(),
        "bits": list(bits_list),
        "rounds": ROUNDS,
        "min_sample_ms": MIN_SAMPLE_MS,
        "working_set_mb": WORKING_SET_BYTES >> 20,
        "max_canary_spread": MAX_CANARY_SPREAD,
        "incumbent": INCUMBENT,
        "shape_provenance": "six Qwen3-4B decode shapes of the reference's pricing recording "
                            "plus the three BASELINE qmv shapes",
        "kernel_source_sha256": wide_qmv.kernel_source_sha256(),
        "rows_per_wave": {f"{bits}b {d_out}x{d_in} M{m}": wide_qmv.rows_per_wave(m, bits, d_out, d_in)
                          for _, d_out, d_in in sites for bits in bits_list for m in M_SWEEP},
        "machine": machine(),
        "elapsed_s": round(time.time() - started, 1),
        "verification": verification,
        "points": [asdict(p) for p in points],
    }


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--out", required=True)
    ap.add_argument("--sites", default="", help="comma-separated site indices (default: all)")
    ap.add_argument("--bits", default=",".join(map(str, BITS)))
    args = ap.parse_args(argv)
    sites = SITES if not args.sites else tuple(SITES[int(i)] for i in args.sites.split(","))
    bits = tuple(int(b) for b in args.bits.split(","))
    record = run(sites, bits, out=lambda s: print(s, flush=True))
    with open(args.out, "w") as f:
        json.dump(record, f, indent=1)
        f.write("\n")
    wins = sum(1 for p in record["points"] if p["verdict"] == "WIN")
    print(f"wrote {args.out}: {len(record['points'])} cells, {wins} WIN", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
