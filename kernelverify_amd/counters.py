"""Per-call instruction counts and busy fractions of the bench rows, from
rocprofv3 counter passes over ``bench.py --issue-profile``.

The issue bound of a row (the time its instructions need at the measured
issue rates, beside the time its bytes need at the HBM rate) rests on what
the kernels really execute, counted by the hardware:

- ``SQ_INSTS_VALU`` counts VALU wave-instructions, matrix-core ones
  included, and ``SQ_INSTS_MFMA`` the matrix-core ones alone, so their
  difference is the VALU issue work of the call;
- ``SQ_INSTS_VALU_MFMA_MOPS_F16`` counts the fp16 matrix-core work in units
  of 512 flops;
- the busy and occupancy fractions (``VALUBusy``, ``MfmaUtil``,
  ``OccupancyPercent``) are rocprofv3's derived counters, one value per
  dispatch.

``bench.py --issue-profile S`` builds each row's workload, then launches a
tag kernel (``probe_fma_kernel`` with ``row + 1`` blocks), S steps of the
row with a device synchronisation after each, and a closing tag
(``probe_dot2_kernel``, 1 block); it prints the row names in order as one
JSON line (the manifest). Here the dispatches of each counter pass are
walked in dispatch order and given to the row whose tags bracket them.
Counts are summed over the row's dispatches and divided by S (per call);
the derived percentages are averaged per kernel, weighted by dispatches.

    python -m kernelverify_amd.counters MANIFEST PASS.csv [PASS.csv ...] > issue.json
"""

from __future__ import annotations

import csv
import hashlib
import json
import re
import shutil
import subprocess
import sys
from collections import defaultdict
from pathlib import Path

from kernelverify_amd import build

OPEN_TAG = "probe_fma_kernel"
CLOSE_TAG = "probe_dot2_kernel"
TAG_BLOCK = 256  # threads per block of the tag kernels

# derived counters that are fractions of a dispatch's time: averaged, not summed
AVERAGED = {"OccupancyPercent", "VALUBusy", "MfmaUtil", "VALUUtilization",
            "MeanOccupancyPerCU", "MeanOccupancyPerActiveCU"}


def library_source_sha256() -> str:
    """sha256 over every libkvpack source (csrc/*.hip and *.h, by name) and
    the device flags: the kernels whose instructions a set of counts
    describes."""
    csrc = Path(__file__).resolve().parent / "csrc"
    h = hashlib.sha256()
    for f in sorted(list(csrc.glob("*.hip")) + list(csrc.glob("*.h"))):
        h.update(f.name.encode())
        h.update(f.read_bytes())
    h.update(build.flags_fingerprint())
    return h.hexdigest()


_TEMPLATE_ARG = re.compile(r"L([ib])(\d+)E|DF16_")


def _short_name(mangled: str) -> str:
    """``name<args>`` of a kernel in namespace kvp::(anonymous) read straight
    from its mangled name (integer, bool and _Float16 template arguments),
    for names a demangler leaves alone."""
    m = re.match(r"_ZN3kvp12_GLOBAL__N_1(\d+)", mangled)
    if not m:
        return mangled
    start = m.end()
    name = mangled[start:start + int(m.group(1))]
    rest = mangled[start + int(m.group(1)):]
    if not rest.startswith("I"):
        return name
    args = []
    for a in _TEMPLATE_ARG.finditer(rest[:rest.find("EEv") + 1 if "EEv" in rest else None]):
        if a.group(0) == "DF16_":
            args.append("f16")
        else:
            args.append(a.group(2) if a.group(1) == "i" else ("true" if a.group(2) == "1"
                                                               else "false"))
    return f"{name}<{','.join(args)}>"


def demangle(names: list[str]) -> dict[str, str]:
    """{mangled: readable}: c++filt when it is installed and understands
    the name, else the name and template arguments read directly."""
    tool = shutil.which("c++filt") or shutil.which("llvm-cxxfilt")
    out = []
    if tool and names:
        out = subprocess.run([tool], input="\n".join(names), capture_output=True, text=True,
                             check=False).stdout.splitlines()
    if len(out) != len(names):
        out = list(names)
    readable = {}
    for n, d in zip(names, out):
        if d.startswith("_Z"):  # still mangled
            readable[n] = _short_name(d)
            continue
        # rocprofv3 writes most names demangled already: drop the return
        # type, the namespace and the parameter list
        d = d.replace("kvp::(anonymous namespace)::", "").removeprefix("void ")
        readable[n] = d.split("(")[0]
    return readable


def _is(kernel: str, tag: str) -> bool:
    return tag in kernel


def read_pass(path: Path, rows: list[str]) -> dict:
    """{row: {kernel: {"dispatches": n, "grid": g, "workgroup": w, "vgpr": v,
    "agpr": a, "lds": l, counter: summed value}}} for one counter pass."""
    by_dispatch: dict[int, dict] = {}
    with open(path, newline="") as f:
        for rec in csv.DictReader(f):
            d = by_dispatch.setdefault(int(rec["Dispatch_Id"]), {
                "kernel": rec["Kernel_Name"], "grid": int(rec["Grid_Size"]),
                "workgroup": int(rec["Workgroup_Size"]), "vgpr": int(rec["VGPR_Count"]),
                "agpr": int(rec.get("Accum_VGPR_Count") or 0),
                "lds": int(rec["LDS_Block_Size"]), "counters": {}})
            d["counters"][rec["Counter_Name"]] = float(rec["Counter_Value"])
    out: dict = {r: {} for r in rows}
    current = None
    for _, d in sorted(by_dispatch.items()):
        k = d["kernel"]
        if _is(k, OPEN_TAG):
            i = d["grid"] // TAG_BLOCK - 1
            current = rows[i] if 0 <= i < len(rows) else None
            continue
        if _is(k, CLOSE_TAG):
            current = None
            continue
        if current is None:
            continue
        key = (k, d["grid"])
        e = out[current].setdefault(key, {"dispatches": 0, "grid": d["grid"],
                                          "workgroup": d["workgroup"], "vgpr": d["vgpr"],
                                          "agpr": d["agpr"], "lds": d["lds"]})
        e["dispatches"] += 1
        for name, value in d["counters"].items():
            e[name] = e.get(name, 0.0) + value
    return out


def summarize(manifest: dict, passes: list[Path]) -> dict:
    """Per row: per-call totals of every summed counter and, per kernel,
    the per-dispatch values (counts and the averaged fractions)."""
    rows, steps = manifest["issue_rows"], int(manifest["steps"])
    merged: dict = {r: {} for r in rows}
    for p in passes:
        for row, kernels in read_pass(Path(p), rows).items():
            for key, e in kernels.items():
                m = merged[row].setdefault(key, {k: e[k] for k in
                                                 ("dispatches", "grid", "workgroup", "vgpr",
                                                  "agpr", "lds")})
                for name, value in e.items():
                    if name not in m:
                        m[name] = value
    names = demangle(sorted({k for r in merged.values() for k, _ in r}))
    result = {"steps": steps, "kernel_source_sha256": manifest.get("kernel_source_sha256"),
              "rows": {}}
    for row in rows:
        totals: dict = defaultdict(float)
        kernels = []
        for (k, grid), e in merged[row].items():
            n = e["dispatches"]
            per = {"kernel": names.get(k, k), "grid": grid, "workgroup": e["workgroup"],
                   "vgpr": e["vgpr"], "agpr": e["agpr"], "lds": e["lds"],
                   "dispatches_per_call": n / steps}
            for name, value in e.items():
                if name in ("dispatches", "grid", "workgroup", "vgpr", "agpr", "lds"):
                    continue
                per[name] = value / n  # per dispatch: a mean for AVERAGED, a count otherwise
                if name not in AVERAGED:
                    totals[name] += value / steps
            kernels.append(per)
        result["rows"][row] = {"per_call": dict(totals), "kernels": kernels}
    return result


def issue_work(per_call: dict) -> dict | None:
    """(VALU wave-instructions, fp16 matrix-core flops) of one call, or None
    when the counts were not collected."""
    if "SQ_INSTS_VALU" not in per_call:
        return None
    mfma = per_call.get("SQ_INSTS_MFMA", 0.0)
    return {"valu_wave_insts": per_call["SQ_INSTS_VALU"] - mfma, "mfma_insts": mfma,
            "mfma_f16_flops": 512.0 * per_call.get("SQ_INSTS_VALU_MFMA_MOPS_F16", 0.0)}


def issue_bound(nbytes: int, achieved_GBps: float, work: dict, rates: dict,
                hbm_GBps: float) -> dict:
    """min(HBM, VALU, matrix core) for one row: the time each resource needs
    for the call's work at its rate, the cap the slowest one sets on the
    throughput, and the achieved fraction of that cap.

    ``rates``: ``valu_wave_insts_per_s`` (the fastest VALU instruction the
    compute probes measure, so the VALU time is a lower bound),
    ``mfma_f16_flops_per_s`` and, optionally, ``dot2_wave_insts_per_s``."""
    t = {"hbm_us": nbytes / (hbm_GBps * 1e9) * 1e6,
         "valu_us": work["valu_wave_insts"] / rates["valu_wave_insts_per_s"] * 1e6,
         "mfma_us": work["mfma_f16_flops"] / rates["mfma_f16_flops_per_s"] * 1e6}
    binding = max(t, key=t.get)
    cap = nbytes / (t[binding] * 1e-6) / 1e9
    out = {"valu_wave_insts_per_call": round(work["valu_wave_insts"]),
           "mfma_f16_flops_per_call": round(work["mfma_f16_flops"]),
           **{k: round(v, 3) for k, v in t.items()},
           "binding": binding.split("_")[0], "cap_GBps": round(cap, 1),
           "frac_cap": round(achieved_GBps / cap, 4)}
    if "dot2_wave_insts_per_s" in rates:
        # every VALU instruction at the dot-product's rate: the issue time
        # if the inner loop's instruction set the pace of the whole stream
        out["valu_us_at_dot2_rate"] = round(
            work["valu_wave_insts"] / rates["dot2_wave_insts_per_s"] * 1e6, 3)
    return out


def main(argv: list[str]) -> int:
    if len(argv) < 2:
        print(__doc__, file=sys.stderr)
        return 2
    manifest = None
    for line in Path(argv[0]).read_text().splitlines():
        if line.startswith("{") and "issue_rows" in line:
            manifest = json.loads(line)
    if manifest is None:
        print(f"{argv[0]}: no issue_rows manifest line", file=sys.stderr)
        return 1
    print(json.dumps(summarize(manifest, [Path(p) for p in argv[1:]]), indent=1))
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
