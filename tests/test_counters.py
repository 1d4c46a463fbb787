"""The counter-pass reader behind the bench rows' issue bounds
(kernelverify_amd/counters.py), on synthetic rocprofv3 CSVs: dispatches are
given to the row whose tag launches bracket them, counts become per-call
sums, derived fractions per-dispatch means, and the bound picks the
slowest resource."""

import csv

import pytest

from kernelverify_amd import counters

FIELDS = ["Correlation_Id", "Dispatch_Id", "Agent_Id", "Queue_Id", "Process_Id", "Thread_Id",
          "Grid_Size", "Kernel_Id", "Kernel_Name", "Workgroup_Size", "LDS_Block_Size",
          "Scratch_Size", "VGPR_Count", "Accum_VGPR_Count", "SGPR_Count", "Counter_Name",
          "Counter_Value", "Start_Timestamp", "End_Timestamp"]


def write_pass(path, dispatches):
    """dispatches: (kernel, grid, {counter: value}) in dispatch order."""
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, FIELDS)
        w.writeheader()
        for i, (kernel, grid, values) in enumerate(dispatches, start=1):
            for name, value in values.items():
                w.writerow({"Correlation_Id": i, "Dispatch_Id": i, "Agent_Id": "Agent 1",
                            "Queue_Id": 1, "Process_Id": 1, "Thread_Id": 1, "Grid_Size": grid,
                            "Kernel_Id": 1, "Kernel_Name": kernel, "Workgroup_Size": 256,
                            "LDS_Block_Size": 0, "Scratch_Size": 0, "VGPR_Count": 32,
                            "Accum_VGPR_Count": 0, "SGPR_Count": 16, "Counter_Name": name,
                            "Counter_Value": value, "Start_Timestamp": 0, "End_Timestamp": 1})


def open_tag(row):
    return ("_ZN3kvp12_GLOBAL__N_116probe_fma_kernelEifPf", 256 * (row + 1), {"SQ_WAVES": 4})


CLOSE = ("_ZN3kvp12_GLOBAL__N_117probe_dot2_kernelEifPf", 256, {"SQ_WAVES": 4})


def test_dispatches_go_to_the_bracketing_row(tmp_path):
    steps = 2
    a = tmp_path / "a.csv"
    write_pass(a, [
        ("setup_kernel", 64, {"SQ_INSTS_VALU": 999.0}),          # before any tag: dropped
        open_tag(0),
        ("split", 1024, {"SQ_INSTS_VALU": 100.0, "SQ_INSTS_MFMA": 10.0}),
        ("combine", 512, {"SQ_INSTS_VALU": 20.0, "SQ_INSTS_MFMA": 0.0}),
        ("split", 1024, {"SQ_INSTS_VALU": 102.0, "SQ_INSTS_MFMA": 10.0}),
        ("combine", 512, {"SQ_INSTS_VALU": 22.0, "SQ_INSTS_MFMA": 0.0}),
        CLOSE,
        ("next_rows_setup", 64, {"SQ_INSTS_VALU": 777.0}),       # between rows: dropped
        open_tag(1),
        ("qmv", 2048, {"SQ_INSTS_VALU": 50.0, "SQ_INSTS_MFMA": 0.0}),
        ("qmv", 2048, {"SQ_INSTS_VALU": 50.0, "SQ_INSTS_MFMA": 0.0}),
        CLOSE,
    ])
    b = tmp_path / "b.csv"
    write_pass(b, [open_tag(0), ("split", 1024, {"VALUBusy": 40.0}),
                   ("combine", 512, {"VALUBusy": 10.0}), ("split", 1024, {"VALUBusy": 60.0}),
                   ("combine", 512, {"VALUBusy": 30.0}), CLOSE,
                   open_tag(1), ("qmv", 2048, {"VALUBusy": 70.0}),
                   ("qmv", 2048, {"VALUBusy": 80.0}), CLOSE])
    manifest = {"issue_rows": ["kv row", "qmv row"], "steps": steps}
    got = counters.summarize(manifest, [a, b])["rows"]
    kv = got["kv row"]
    assert kv["per_call"]["SQ_INSTS_VALU"] == pytest.approx((100 + 20 + 102 + 22) / steps)
    assert kv["per_call"]["SQ_INSTS_MFMA"] == pytest.approx(10.0)
    assert "VALUBusy" not in kv["per_call"]          # fractions are not summed
    split = next(k for k in kv["kernels"] if k["grid"] == 1024)
    assert split["VALUBusy"] == pytest.approx(50.0)  # the mean over dispatches
    assert split["SQ_INSTS_VALU"] == pytest.approx(101.0)
    assert split["dispatches_per_call"] == 1.0
    qmv = got["qmv row"]
    assert qmv["per_call"]["SQ_INSTS_VALU"] == pytest.approx(50.0)
    assert qmv["kernels"][0]["VALUBusy"] == pytest.approx(75.0)


def test_issue_bound_picks_the_slowest_resource():
    rates = {"valu_wave_insts_per_s": 1e12, "mfma_f16_flops_per_s": 2e15}
    nbytes = 8_000_000  # 1 us at 8 TB/s
    hbm = counters.issue_bound(nbytes, 4000.0, {"valu_wave_insts": 5e5, "mfma_f16_flops": 0.0},
                               rates, 8000.0)
    assert hbm["binding"] == "hbm" and hbm["cap_GBps"] == pytest.approx(8000.0)
    assert hbm["valu_us"] == pytest.approx(0.5) and hbm["frac_cap"] == pytest.approx(0.5)
    valu = counters.issue_bound(nbytes, 4000.0, {"valu_wave_insts": 2e6, "mfma_f16_flops": 0.0},
                                rates, 8000.0)
    assert valu["binding"] == "valu" and valu["cap_GBps"] == pytest.approx(4000.0)
    assert valu["frac_cap"] == pytest.approx(1.0)
    mfma = counters.issue_bound(nbytes, 1000.0, {"valu_wave_insts": 0.0, "mfma_f16_flops": 8e9},
                                rates, 8000.0)
    assert mfma["binding"] == "mfma" and mfma["mfma_us"] == pytest.approx(4.0)


def test_issue_work_separates_matrix_core_instructions():
    w = counters.issue_work({"SQ_INSTS_VALU": 1000.0, "SQ_INSTS_MFMA": 200.0,
                             "SQ_INSTS_VALU_MFMA_MOPS_F16": 3.0})
    assert w == {"valu_wave_insts": 800.0, "mfma_insts": 200.0, "mfma_f16_flops": 1536.0}
    assert counters.issue_work({"VALUBusy": 3.0}) is None
