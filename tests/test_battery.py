"""The mutation batteries' host side: every mutant differs from the
control by its own fault and compiles for gfx950 (hiprtc, no device). The
scoring on the GPU is tests/test_gates_gpu.py."""

import pytest

from kernelverify_amd.runners import rtc
from tests.gates import battery_qmv as B


def test_each_mutant_is_the_control_plus_one_fault():
    control = B.mutant_spec("control", 4).source
    sources = {name: B.mutant_spec(name, 4).source for name in B.MUTANTS}
    assert len(set(sources.values())) == len(B.MUTANTS)
    for name, src in sources.items():
        assert src.endswith(B.TEMPLATE) and (name == "control") == (src == control)


@pytest.mark.parametrize("name", sorted(B.MUTANTS))
def test_every_mutant_compiles_for_gfx950(name):
    try:
        code = rtc.compile_source(B.mutant_spec(name, 8).source)
    except rtc.CompileError as error:
        if "not loadable" in str(error):
            pytest.skip(str(error))
        raise
    assert len(code) > 0


def test_each_kv_mutant_is_the_control_plus_one_fault():
    from tests.gates import battery_kv as K

    sources = {name: K.mutant_spec(name, 4, 128).source for name in K.MUTANTS}
    assert len(set(sources.values())) == len(K.MUTANTS)
    for src in sources.values():
        assert src.endswith(K.TEMPLATE)


@pytest.mark.parametrize("name", ["control", "new-entry-dropped", "fp16-scores", "gqa-modulo"])
def test_kv_mutants_compile_for_gfx950(name):
    from tests.gates import battery_kv as K

    try:
        code = rtc.compile_source(K.mutant_spec(name, 3, 128).source)
    except rtc.CompileError as error:
        if "not loadable" in str(error):
            pytest.skip(str(error))
        raise
    assert len(code) > 0


def test_each_moe_mutant_is_the_control_plus_one_fault():
    from tests.gates import battery_moe as M

    sources = {name: M.mutant_spec(name, 16).source for name in M.MUTANTS}
    assert len(set(sources.values())) == len(M.MUTANTS)
    for src in sources.values():
        assert src.endswith(M.TEMPLATE)
    with pytest.raises(AssertionError):
        M.mutant_spec("control", M.MAX_E + 1)


@pytest.mark.parametrize("name", ["control", "top-1", "ties-high", "softmax-after-topk"])
def test_moe_mutants_compile_for_gfx950(name):
    from tests.gates import battery_moe as M

    try:
        code = rtc.compile_source(M.mutant_spec(name, 8).source)
    except rtc.CompileError as error:
        if "not loadable" in str(error):
            pytest.skip(str(error))
        raise
    assert len(code) > 0


def test_moe_battery_plan_is_the_gates():
    """Same shapes and modes as the gate; constant_rows rows are all near-ties
    (so only the dispatch rule can see a tie-break fault there)."""
    from tests.gates import battery_moe as M
    from tests.gates.pack_moe_dispatch import VERIFY_SHAPES

    plan = M.cases()
    metas = [m for ms in plan.values() for m in ms]
    assert len(metas) == 2 * len(VERIFY_SHAPES)
    for m in metas:
        if m["label"].startswith("constant_rows"):
            assert not m["clean"].any()
        assert m["want"].shape == (m["n"], M.TOP_K)
