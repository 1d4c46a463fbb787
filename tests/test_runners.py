"""The runner door's host side on the CPU (no GPU needed): spec and case
validation, extents, JSON wire forms, `specialize`, pack-library
descriptors, and the statuses a runner returns without a device.

Mirrors the reference's runner tests in spirit (tests/test_runners_spec.py,
tests/test_specialize.py): every misuse is a SpecError or an INVALID_SPEC
status, never a crash, and `specialize` refuses missing and unused keys.
"""

import numpy as np
import pytest

from kernelverify_amd.pack import kv_attention, moe_dispatch, wide_qmv
from kernelverify_amd.runners import (
    Binding,
    BindingKind,
    HipRunner,
    KernelSpec,
    LaunchMode,
    LaunchSpec,
    RunCase,
    RunResult,
    RunStatus,
    SpecError,
    Timing,
    specialize,
)
from kernelverify_amd.runners.library import parse_descriptor
from kernelverify_amd.runners.spec import resolve_extent

SAXPY = """
extern "C" __global__ void saxpy(const float* x, float* y, float a, unsigned n) {
  unsigned i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = a * x[i];
}
"""


def saxpy_spec():
    return KernelSpec(source=SAXPY, entry_point="saxpy",
                      bindings=(Binding(BindingKind.INPUT, "x"), Binding(BindingKind.OUTPUT),
                                Binding(BindingKind.SCALAR, "a", "float32"),
                                Binding(BindingKind.SCALAR, "n", "uint32")),
                      launch=LaunchSpec(grid=("n", 1, 1), threadgroup=(64, 1, 1)))


def test_extents_resolve_ints_names_and_products():
    assert resolve_extent(4, {}, "g") == 4
    assert resolve_extent("n", {"n": 7}, "g") == 7
    assert resolve_extent(["b", "h", 2], {"b": 3, "h": 5}, "g") == 30
    for bad in (True, 0, [], "missing", 1.5):
        with pytest.raises(SpecError):
            resolve_extent(bad, {"x": 1}, "g")


def test_spec_validation_refuses_unrunnable_specs():
    with pytest.raises(SpecError):
        KernelSpec(source="", entry_point="k", bindings=(Binding(BindingKind.OUTPUT),))
    with pytest.raises(SpecError):
        KernelSpec(source="x", entry_point="k", bindings=(Binding(BindingKind.INPUT, "a"),))
    with pytest.raises(SpecError):
        KernelSpec(source="x", entry_point="k",
                   bindings=(Binding(BindingKind.OUTPUT, index=1), Binding(BindingKind.OUTPUT)))
    with pytest.raises(SpecError):
        Binding(BindingKind.SCALAR, "n", "float64")
    with pytest.raises(SpecError):
        LaunchSpec(grid=(1, 1))


def test_case_validation_names_every_missing_piece():
    spec = saxpy_spec()
    good = RunCase(inputs={"x": np.ones(8, np.float32)}, params={"a": 2.0, "n": 8},
                   output_shapes=[((8,), "float32")])
    good.validate_against(spec)
    for case in (RunCase(inputs={}, params={"a": 2.0, "n": 8}, output_shapes=[((8,), "float32")]),
                 RunCase(inputs={"x": np.ones(8, np.float32)}, params={"n": 8},
                         output_shapes=[((8,), "float32")]),
                 RunCase(inputs={"x": np.ones(8, np.float32)}, params={"a": 1.0},
                         output_shapes=[((8,), "float32")]),
                 RunCase(inputs={"x": np.ones(8, np.float64)}, params={"a": 1.0, "n": 8},
                         output_shapes=[((8,), "float32")])):
        with pytest.raises(SpecError):
            case.validate_against(spec)
    with pytest.raises(SpecError):
        RunCase(inputs={}, output_shapes=[((0,), "float32")])
    with pytest.raises(SpecError):
        RunCase(inputs={}, output_shapes=())


def test_json_wire_forms_round_trip():
    spec = saxpy_spec()
    assert KernelSpec.from_json(spec.to_json()) == spec
    x = np.arange(12, dtype=np.float16).reshape(3, 4)
    case = RunCase(inputs={"x": x}, params={"n": 3}, output_shapes=[((3, 4), "float16")],
                   label="c")
    back = RunCase.from_json(case.to_json())
    assert np.array_equal(back.inputs["x"], x) and back.inputs["x"].dtype == x.dtype
    assert back.params == {"n": 3} and back.output_shapes == case.output_shapes
    res = RunResult(status=RunStatus.OK, outputs=[x], timing=Timing((1e-6, 2e-6), (3e-6,), 1),
                    label="c")
    back = RunResult.from_json(res.to_json())
    assert back.status is RunStatus.OK and np.array_equal(back.outputs[0], x)
    assert back.timing.gpu_best == 1e-6 and back.timing.gpu_spread == 2.0


def test_specialize_fills_and_refuses():
    spec = specialize(wide_qmv.kernel_spec(), {"T": "half", "BITS": 4, "M": 1, "R": 2})
    assert spec.source == "kvpack:wide_qmv T=half BITS=4 M=1 R=2"
    assert spec.name == "kvp_qmv-4 bit-M1-R2-half"
    assert spec.bindings == wide_qmv.kernel_spec().bindings
    with pytest.raises(SpecError):
        specialize(wide_qmv.kernel_spec(), {"T": "half", "BITS": 4, "M": 1})
    with pytest.raises(SpecError):
        specialize(wide_qmv.kernel_spec(), {"T": "half", "BITS": 4, "M": 1, "R": 2, "Q": 0})


def test_pack_templates_keep_the_reference_bindings():
    """Binding names and order of the reference's templates
    (pack/wide_qmv.py:247-253, kv_attention.py:333-346, moe_dispatch.py:186-189,
    :222-230), so cases written for the reference door bind here."""
    names = lambda s: [(b.kind.value, b.name) for b in s.bindings]
    assert names(wide_qmv.kernel_spec()) == [
        ("input", "x"), ("input", "w_q"), ("input", "scales"), ("input", "biases"),
        ("output", ""), ("scalar", "d_in_arg"), ("scalar", "d_out_arg")]
    assert [n for k, n in names(kv_attention.kernel_spec()) if k == "scalar"] == [
        "n_heads", "t_cached", "n_kv_heads", "t_stride"]
    assert [k for k, _ in names(moe_dispatch.routing_spec())] == [
        "input", "input", "output", "output", "scalar"]
    assert names(moe_dispatch.dispatch_spec())[:6] == [
        ("input", n) for n in ("x", "idx", "gate", "w_q", "scales", "biases")]
    family, consts = parse_descriptor(
        specialize(kv_attention.kernel_spec(), {"T": "float", "BITS": 8, "DH": 64}).source)
    assert family == "kv_attention" and consts == {"T": "float", "BITS": "8", "DH": "64"}


def test_no_device_is_unsupported_and_bad_cases_are_invalid(monkeypatch):
    monkeypatch.setenv("KV_FORCE_NO_GPU", "1")
    runner = HipRunner()
    assert runner.probe() is None
    spec = saxpy_spec()
    good = RunCase(inputs={"x": np.ones(8, np.float32)}, params={"a": 2.0, "n": 8},
                   output_shapes=[((8,), "float32")], label="good")
    bad = RunCase(inputs={}, params={"a": 2.0, "n": 8}, output_shapes=[((8,), "float32")],
                  label="bad")
    res = runner.run_candidate([(spec, [good]), (spec, [bad])])
    assert res[0][0].status is RunStatus.UNSUPPORTED
    assert res[1][0].status is RunStatus.INVALID_SPEC and "input 'x' is missing" in res[1][0].detail


def test_launch_modes_round_trip():
    ls = LaunchSpec(grid=(["a", "b"], 1, 1), threadgroup=(64, 1, 1),
                    mode=LaunchMode.THREADGROUPS, threadgroup_memory=("lds",))
    assert LaunchSpec.from_json(ls.to_json()) == ls
    assert ls.resolve({"a": 2, "b": 3, "lds": 512}) == ((6, 1, 1), (64, 1, 1), (512,))


def test_hiprtc_builds_candidates_and_reports_compile_errors():
    """hiprtc compiles HIP source for gfx950 without a device; a broken
    source is a CompileError carrying the compiler's diagnostic."""
    from kernelverify_amd.runners import rtc

    code = rtc.compile_source(SAXPY)
    assert code[:4] == b"\x7fELF"
    with pytest.raises(rtc.CompileError, match="undeclared identifier"):
        rtc.compile_source('extern "C" __global__ void k(float* y) { y[0] = nothing_here; }')


def test_specialize_reports_every_problem_and_keeps_escaped_dollars():
    from kernelverify_amd.runners.specialize import placeholders

    tmpl = KernelSpec(source="k<$T, ${N}> costs $$5 // $T again", entry_point="k_$T",
                      bindings=(Binding(BindingKind.OUTPUT),), name="t")
    assert placeholders(tmpl.source) == ["T", "N"]
    spec = specialize(tmpl, {"T": "half", "N": 3})
    assert spec.source == "k<half, 3> costs $5 // half again" and spec.entry_point == "k_half"
    with pytest.raises(SpecError) as err:
        specialize(tmpl, {"T": "half", "M": 1})
    assert "$N" in str(err.value) and "['M']" in str(err.value)
    bad = KernelSpec(source="x = $1", entry_point="k", bindings=(Binding(BindingKind.OUTPUT),))
    with pytest.raises(SpecError):
        specialize(bad, {})
