"""The runner door on the GPU: run-time compiled candidates, the pack-library
specs, statuses and interleaved comparison (reference runner behaviour:
kernelverify/runners/metal.py:105-251, compare.py:190-249)."""

import numpy as np
import pytest

from kernelverify_amd.pack import wide_qmv
from kernelverify_amd.pack.codes import pack_codes
from kernelverify_amd.runners import (
    Binding,
    BindingKind,
    HipRunner,
    KernelSpec,
    LaunchSpec,
    RunCase,
    RunStatus,
    compare,
    specialize,
)
from tests.test_runners import SAXPY, saxpy_spec

pytestmark = pytest.mark.gpu


def saxpy_case(n=1000, a=3.0, seed=0):
    x = np.random.default_rng(seed).standard_normal(n).astype(np.float32)
    return x, RunCase(inputs={"x": x}, params={"a": a, "n": n}, output_shapes=[((n,), "float32")],
                      label=f"saxpy n={n}")


def test_probe_finds_gfx950():
    info = HipRunner().probe()
    assert info is not None and info.arch.startswith("gfx950") and info.compute_units > 0


def test_candidate_source_runs_with_timing():
    x, case = saxpy_case()
    res = HipRunner(repeats=3).run_one(saxpy_spec(), case)
    assert res.ok, res.detail
    assert np.array_equal(res.outputs[0], np.float32(3.0) * x)
    assert res.timing.repeats == 3 and res.timing.gpu_best > 0


def test_statuses_not_exceptions():
    _, case = saxpy_case()
    broken = KernelSpec(source='extern "C" __global__ void saxpy(float* y) { y[0] = nope; }',
                        entry_point="saxpy", bindings=saxpy_spec().bindings,
                        launch=saxpy_spec().launch)
    missing = KernelSpec(source=SAXPY, entry_point="not_there", bindings=saxpy_spec().bindings,
                         launch=saxpy_spec().launch)
    runner = HipRunner()
    assert runner.run_one(broken, case).status is RunStatus.COMPILE_ERROR
    assert runner.run_one(missing, case).status is RunStatus.COMPILE_ERROR
    qmv = specialize(wide_qmv.kernel_spec(), {"T": "half", "BITS": 4, "M": 2, "R": 2})
    x = np.ones((1, 128), np.float16)  # M = 2 in the spec, 1 row here
    bad = RunCase(inputs={"x": x, "w_q": np.zeros((8, 16), np.uint32),
                          "scales": np.zeros((8, 2), np.float16),
                          "biases": np.zeros((8, 2), np.float16)},
                  params={"d_in_arg": 128, "d_out_arg": 8, "row_blocks": 1},
                  output_shapes=[((1, 8), "float16")])
    assert runner.run_one(qmv, bad).status is RunStatus.INVALID_SPEC
    five = specialize(wide_qmv.kernel_spec(), {"T": "half", "BITS": 5, "M": 1, "R": 2})
    res = runner.run_one(five, bad)
    assert res.status in (RunStatus.UNSUPPORTED, RunStatus.INVALID_SPEC), res


def test_library_spec_equals_the_direct_call():
    """Also a regression test: a failed symbol lookup just before must not
    surface as this launch's error (the library clears the runtime's stale
    per-thread error on entry)."""
    _, saxpy = saxpy_case()
    missing = KernelSpec(source=SAXPY, entry_point="not_there", bindings=saxpy_spec().bindings,
                         launch=saxpy_spec().launch)
    assert HipRunner().run_one(missing, saxpy).status is RunStatus.COMPILE_ERROR
    rng = np.random.default_rng(3)
    d_out, d_in, m, bits = 300, 512, 3, 4
    q = rng.integers(0, 16, (d_out, d_in))
    s = np.abs(rng.standard_normal((d_out, d_in // 64)) * 0.02).astype(np.float16)
    b = (rng.standard_normal((d_out, d_in // 64)) * 0.01).astype(np.float16)
    x = rng.standard_normal((m, d_in)).astype(np.float16)
    w = pack_codes(q, bits)
    grid, _, r = wide_qmv.launch_config(d_out, m)
    spec = specialize(wide_qmv.kernel_spec(), {"T": "float", "BITS": bits, "M": m, "R": r})
    case = RunCase(inputs={"x": x, "w_q": w, "scales": s, "biases": b},
                   params={"d_in_arg": d_in, "d_out_arg": d_out, "row_blocks": grid[0]},
                   output_shapes=[((m, d_out), "float32")])
    res = HipRunner().run_one(spec, case)
    assert res.ok, res.detail
    assert np.array_equal(res.outputs[0], wide_qmv.qmv(x, w, s, b, bits=bits, out_dtype="float32"))


def test_interleaved_compare_reports_rounds():
    _, case = saxpy_case(n=1 << 20)
    spec_b = KernelSpec(source=SAXPY.replace("a * x[i]", "x[i] * a"), entry_point="saxpy",
                        bindings=saxpy_spec().bindings, launch=saxpy_spec().launch)
    report = compare(saxpy_spec(), spec_b, [case], rounds=3, warmup=1, repeats=3,
                     spread_limit=100.0)
    assert not report.failure, report.failure
    assert len(report.cases[0].samples) == 3
    assert np.isfinite(report.cases[0].speedup)


# A kernel that waits a bounded time on the device's constant 100 MHz wall
# clock, then writes its output: it always finishes (at most `ticks` ticks
# and at most 2^26 polls), but longer than the runner's deadline below.
WAIT = """
extern "C" __global__ void wait_then_write(float* y, unsigned ticks) {
  const unsigned long long t0 = wall_clock64();
  unsigned polls = 0;
  while (wall_clock64() - t0 < ticks && polls < (1u << 26)) ++polls;
  y[threadIdx.x] = 1.0f + (float)min(polls, 1u);  // 1 or 2: the kernel ran
}
"""


def test_a_case_still_running_at_its_deadline_is_timeout_and_wedges_the_runner():
    """case_timeout is a host deadline checked while the work is queued: a
    case whose kernel outlives it is TIMEOUT, and the runner refuses the
    rest of its cases without touching the device."""
    spec = KernelSpec(source=WAIT, entry_point="wait_then_write",
                      bindings=(Binding(BindingKind.OUTPUT),
                                Binding(BindingKind.SCALAR, "ticks", "uint32")),
                      launch=LaunchSpec(grid=(64, 1, 1), threadgroup=(64, 1, 1)))
    slow = RunCase(inputs={}, params={"ticks": 20_000_000}, output_shapes=[((64,), "float32")],
                   label="200 ms")
    quick = RunCase(inputs={}, params={"ticks": 1}, output_shapes=[((64,), "float32")],
                    label="quick")
    ok = HipRunner(warmup=0, repeats=1).run(spec, [quick])
    assert ok[0].ok and np.all(ok[0].outputs[0] >= 1.0)
    runner = HipRunner(case_timeout=0.02, warmup=0, repeats=1)
    res = runner.run(spec, [slow, quick])
    assert res[0].status is RunStatus.TIMEOUT and "still running" in res[0].detail
    assert res[1].status is RunStatus.TIMEOUT and res[1].detail.startswith("not run")
    assert runner.wedged
    from kernelverify_amd import hip

    hip.synchronize()  # the slow kernel ends by itself (bounded above)
