"""Write tests/golden/quant_device_adequacy.records.json from the reference's
committed evidence file bench/results/quant_device_adequacy.json.

Run once in the build container (the reference tree is not present on the GPU
box). The output keeps, per record, the fields the oracle tests check: the
record key (bits, shape, draw, seed, mode, dtype), ref_scale, base_tol, the
six CPU member errors, the three Metal device-member errors (advisory), the six
fault errors and the fp16-dequant boundary error. Inputs are not stored: they
regenerate from default_rng(10000 + seed) -> make_w -> make_x per (mode, dtype).
"""

import json
import sys
from pathlib import Path

SRC = Path("/root/reference/bench/results/quant_device_adequacy.json")
DST = Path(__file__).with_name("quant_device_adequacy.records.json")
KEEP = ("bits", "shape", "draw", "seed", "mode", "dtype", "ref_scale", "base_tol",
        "members", "faults", "boundary_fp16_dequant")


def main() -> int:
    raw = json.loads(SRC.read_text())
    out = {"source": "vladmt06/kernelverify bench/results/quant_device_adequacy.json",
           "shapes": raw["shapes"], "k_shipped": raw["k_shipped"], "records": []}
    for bits in sorted(raw["records"], key=int):
        for rec in raw["records"][bits]:
            out["records"].append({k: rec[k] for k in KEEP})
    DST.write_text(json.dumps(out, separators=(",", ":")))
    print(f"wrote {len(out['records'])} records to {DST}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
