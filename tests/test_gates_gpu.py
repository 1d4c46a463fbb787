"""The pack gates through the runner door (the reference's
bench/pack_*.py verify() drivers, here tests/gates/): each must come back
green, and the quantizer faults of the contract (oracle FAULTS, the
reference's negative controls, tests/test_pack_verify.py:47-54) must each
turn the qmv gate red when the kernel is fed the faulted artefact."""

import pytest

from kernelverify_amd.runners import HipRunner
from oracle.quant_contract import FAULTS
from tests.gates import pack_kv_attention, pack_moe_dispatch, pack_wide_qmv

pytestmark = pytest.mark.gpu


def quiet(*_):
    pass


def test_qmv_gate_green_every_width():
    """The qmv gate at one of its shapes, every width, M in {1, 4} (the full
    policy is `python -m tests.gates.pack_wide_qmv`)."""
    ev = pack_wide_qmv.verify(HipRunner(repeats=1), shapes=[(2560, 2560)], ms=[1, 4], out=quiet)
    assert ev.cases_run == 16
    assert ev.ok, [c for s in ev.specializations for c in s.cases if not c.passed] + \
        [c for c in ev.checks if not c.passed]


def test_kv_gate_green():
    ev = pack_kv_attention.verify(HipRunner(repeats=1), out=quiet)
    assert ev.cases_run == 10 and ev.ok, [c for s in ev.specializations for c in s.cases
                                        if not c.passed] + [c for c in ev.checks if not c.passed]


def test_moe_gate_green():
    ev = pack_moe_dispatch.verify(HipRunner(repeats=1), out=quiet)
    assert ev.cases_run == 12 and ev.ok, [c for s in ev.specializations for c in s.cases
                                         if not c.passed]


@pytest.mark.parametrize("fault", sorted(FAULTS))
def test_each_quantizer_fault_turns_the_qmv_gate_red(fault):
    ev = pack_wide_qmv.verify(HipRunner(repeats=1), shapes=[(512, 1024)], bits_list=(4,),
                              ms=[1], artefact_fault=FAULTS[fault], out=quiet)
    assert ev.cases_run == 2
    assert ev.cases_passed == 0, (fault, [c for s in ev.specializations for c in s.cases])


def test_a_green_gate_certifies_and_a_faulted_one_is_refused(tmp_path):
    """Certificates from real gate evidence: one per specialization when the
    gate is green; the family withheld when the artefact is faulted."""
    import json

    from tests.gates import emit_pack_certificates as emitter

    runner = HipRunner(repeats=1)
    ev = pack_wide_qmv.verify(runner, shapes=[(512, 1024)], bits_list=(4,), ms=[1, 4],
                              out=quiet)
    report = emitter.certify([ev], tmp_path / "green", commit="test", chip="gfx950")
    assert report.ok and len(report.written) == 2, report.refused
    body = json.loads(report.written[0].read_text())
    assert body["protocol_bound"]["cases_passed"] == body["protocol_bound"]["cases_run"] == 2
    bad = pack_wide_qmv.verify(runner, shapes=[(512, 1024)], bits_list=(4,), ms=[1],
                               artefact_fault=FAULTS[sorted(FAULTS)[0]], out=quiet)
    refused = emitter.certify([bad], tmp_path / "faulted", commit="test", chip="gfx950")
    assert not refused.written and "kvp_qmv" in refused.refused


def test_mutation_battery_catches_every_blatant_fault():
    """The qmv gate's cases against run-time compiled mutants: the control
    passes and every fault of the operator's formula is caught; the fp16
    rounding of group partials is reported either way (a precision fault
    the cases may not separate)."""
    from tests.gates import battery_qmv

    table = battery_qmv.run_battery(HipRunner(repeats=1))
    assert not table["control"]["caught"], table["control"]
    for name in ("fp16-accumulate", "drop-bias", "wrong-group-scale", "complemented-codes",
                 "shifted-activations"):
        assert table[name]["caught"], (name, table[name])
    print({n: (r["caught"], round(r["worst_err_over_tol"], 3)) for n, r in table.items()})


def test_kv_mutation_battery():
    """The KV gate's cases against run-time compiled mutants: the control
    passes, every fault of the formula and the GQA mapping is caught; the
    unshifted softmax (C4) escapes these cases, as the battery documents."""
    from tests.gates import battery_kv

    table = battery_kv.run_battery(HipRunner(repeats=1))
    print({n: (r["caught"], round(r["worst_err_over_tol"], 3)) for n, r in table.items()})
    assert not table["control"]["caught"], table["control"]
    for name in ("new-entry-dropped", "v-bias-dropped", "v-position-shifted", "scale-1-over-dh",
                 "gqa-modulo"):
        assert table[name]["caught"], (name, table[name])
    assert not table["no-max-shift"]["caught"], table["no-max-shift"]


def test_moe_mutation_battery():
    """The MoE gate's cases against run-time compiled routers: the control
    passes; the unnormalised gates, the off-by-one expert, top-1 and the
    high-index tie-break are caught; softmax over the chosen logits is the
    equivalent mutant and escapes."""
    from tests.gates import battery_moe

    table = battery_moe.run_battery(HipRunner(repeats=1))
    print({n: (r["caught"], r["by"], round(r["worst_err_over_tol"], 3)) for n, r in table.items()})
    assert not table["control"]["caught"], table["control"]
    for name in ("not-renormalised", "expert-offset", "top-1", "ties-high"):
        assert table[name]["caught"], (name, table[name])
    assert "dispatch" in table["ties-high"]["by"]
    assert not table["softmax-after-topk"]["caught"], table["softmax-after-topk"]
