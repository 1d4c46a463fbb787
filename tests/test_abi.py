"""The C-ABI library: it loads, and exports every entry point the header declares.

No compute call here: this runs without a GPU.
"""

import re
from pathlib import Path

import pytest

from kernelverify_amd import lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "kvpack.h"


def declared_symbols():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(kvp_\w+)\s*\(", text)))


def test_header_declares_the_pack():
    names = declared_symbols()
    for must in ("kvp_qmv", "kvp_kv_decode", "kvp_moe_route", "kvp_moe_permute",
                 "kvp_moe_dispatch", "kvp_moe_swiglu", "kvp_last_error"):
        assert must in names


def test_library_exports_every_declared_symbol():
    cdll = lib.load()
    missing = [n for n in declared_symbols() if not hasattr(cdll, n)]
    assert not missing, missing


def test_binding_table_matches_header():
    assert sorted(lib.SIGNATURES) == declared_symbols()


def test_version_names_the_target():
    assert "gfx950" in lib.version()


def test_argument_errors_are_statuses_not_crashes():
    """Argument checks run on the host before anything touches a device."""
    cdll = lib.load()
    rc = cdll.kvp_qmv(None, None, None, None, None, lib.KVP_F16, 1, 16, 64, 4, None)
    assert rc == lib.KVP_INVALID
    assert "null pointer" in lib.last_error()
    with pytest.raises(lib.InvalidArgument):
        lib.check(rc)


def declared_arities():
    """name -> number of parameters, parsed from the header's prototypes."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for name, params in re.findall(r"\b(kvp_\w+)\s*\(([^)]*)\)\s*;", text):
        params = params.strip()
        out[name] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def test_binding_arities_match_header():
    """Every ctypes prototype takes exactly the header's parameter count."""
    arities = declared_arities()
    assert set(arities) == set(lib.SIGNATURES)
    for name, (_, args) in lib.SIGNATURES.items():
        assert len(args) == arities[name], (name, len(args), arities[name])


def test_tuning_keys_are_explicit_and_restorable():
    """Kernel selection changes only through kvp_set_tuning (no environment
    variable is read); unknown keys are refused and -1 restores the
    library's choice."""
    assert lib.get_tuning("qmv_path") == -1
    lib.set_tuning("qmv_path", 5)
    try:
        assert lib.get_tuning("qmv_path") == 5
    finally:
        lib.set_tuning("qmv_path", -1)
    assert lib.get_tuning("qmv_path") == -1
    with pytest.raises(lib.InvalidArgument):
        lib.set_tuning("no_such_key", 1)
    with pytest.raises(lib.InvalidArgument):
        lib.set_tuning("moe_kq", -2)

    src = Path(__file__).resolve().parents[1] / "kernelverify_amd" / "csrc"
    for f in src.iterdir():
        if f.suffix in (".hip", ".h"):
            assert "getenv" not in f.read_text(), f.name
