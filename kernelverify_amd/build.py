"""Build libkvpack.so for gfx950 from kernelverify_amd/csrc with hipcc.

One shared library, compiled in-tree so it travels with the repository
snapshot. Each .hip file is compiled to an object in parallel, then linked.

Flags:
- ``--offload-arch=gfx950`` only: the library is CDNA4 code, no other target.
- ``-Xclang -target-feature -Xclang -packed-fp32-ops`` keeps the compiler from
  forming packed-fp32 VALU instructions from scalar float code.
- ``-ffp-contract=fast`` lets a*b+c fuse to FMA (a single rounding, within the
  fp32 contract); no fast-math: exp, division and sqrt stay IEEE-accurate.
- ``-amdgpu-kernarg-preload-count=16`` hands kernel arguments to a wave in
  SGPRs at launch.

Run: ``python -m kernelverify_amd.build`` (or ``__graft_entry__.build()``).
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
INCLUDE = PKG.parent / "include"
LIB = PKG / "libkvpack.so"
OBJ_DIR = PKG / "_build"

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=fast",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # matrix-core accumulators in ordinary VGPRs: the KV kernels rescale them
    # on the VALU, which cannot operate on AGPRs in place
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    # kernel arguments arrive in SGPRs when a wave starts instead of through a
    # scalar load (the compiler keeps a prologue that loads them on firmware
    # without preloading); struct arguments, passed by reference, are not
    # preloaded. Measured on MI355X, 4-bit qmv at M = 1: 14336x4096 8.56 ->
    # 8.47 us, 4096x4096 4.29 -> 4.09, outputs bit-identical.
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
    f"-I{INCLUDE}",
]


def flags_fingerprint() -> bytes:
    """The device flags that shape the machine code, include paths aside (they
    differ between machines): hashed with the sources wherever a measurement
    is pinned to a kernel body, so a changed flag voids it like a changed
    line."""
    return " ".join(f for f in DEVICE_FLAGS if not f.startswith("-I")).encode()


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path, extra: list[str]) -> Path:
    obj = OBJ_DIR / (src.stem + ".o")
    cmd = [HIPCC, *DEVICE_FLAGS, *extra, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{' '.join(cmd)}\n{proc.stderr}")
    return obj


def build(verbose: bool = True, extra_flags: list[str] | None = None) -> Path:
    """Compile every csrc/*.hip and link libkvpack.so; returns its path."""
    if not Path(HIPCC).exists() and shutil.which("hipcc") is None:
        raise RuntimeError("hipcc not found: the HIP toolchain is required to build libkvpack")
    OBJ_DIR.mkdir(exist_ok=True)
    extra = list(extra_flags or [])
    srcs = sources()
    workers = min(len(srcs), int(os.environ.get("MAX_JOBS", "8")), 16)
    with cf.ThreadPoolExecutor(max_workers=max(1, workers)) as pool:
        objs = list(pool.map(lambda s: _compile(s, extra), srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{proc.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources", flush=True)
    return LIB


if __name__ == "__main__":
    build(extra_flags=sys.argv[1:])
