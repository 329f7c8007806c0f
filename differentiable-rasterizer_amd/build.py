"""Builds libdiffrast_hip.so (gfx950) in-tree with hipcc.

Usage: python build.py [--verbose]. The library lands next to this file, where
`diffrast._lib` loads it from.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
CSRC = HERE / "csrc"
LIB = HERE / "libdiffrast_hip.so"
ARCH = os.environ.get("DIFFRAST_OFFLOAD_ARCH", "gfx950")

SOURCES = [CSRC / "kernels.hip", CSRC / "runtime.hip", CSRC / "fit.hip", CSRC / "scratch.hip", CSRC / "resize.hip"]
HEADERS = [CSRC / "kernels.h", CSRC / "runtime.h", ROOT / "include" / "diffrast_hip.h"]

# -ffp-contract=off: the kernels state every FMA explicitly; plain a*b+c must
# round twice, as the reference's arithmetic does.
# -packed-fp32-ops: no v_pk_*_f32 instructions in the generated code.
# -structurizecfg-skip-uniform-regions: regions whose branches are all
# wave-uniform (scalar-condition branches) keep their control flow as written;
# the default structurizer rewrites them as it does divergent ones, carrying
# path flags (scalar mask operations and extra branches) through the sweeps'
# per-entry code. Regions with a divergent branch are structurized as before.
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-structurizecfg-skip-uniform-regions=true",
    "-Wall",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]


def hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found")


def build(verbose: bool = False) -> Path:
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), *FLAGS, *map(str, SOURCES), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "packed-fp32-ops"
    err = "\n".join(l for l in (res.stderr or "").splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{err}")
    if verbose and err.strip():
        print(err)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="--verbose" in sys.argv))
