"""Builds x_amd/csrc/libatl_hip.so for gfx950 with hipcc (in-tree, no JIT cache).

Flags: -ffp-contract=off keeps every fp32 expression rounded op by op (the index and cut-off arithmetic must
match the reference's CPU rounding), -munsafe-fp-atomics emits hardware float atomics, and packed FP32 is
disabled (-Xclang -target-feature -Xclang -packed-fp32-ops)."""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
SOURCES = ["abi.hip", "events.hip", "tiles.hip", "pairs.hip", "fastpair.hip", "knn.hip"]
OUT = HERE / "libatl_hip.so"
ARCH = os.environ.get("ATL_HIP_ARCH", "gfx950")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if cand and (Path(cand).exists() or cand == "hipcc"):
            return cand
    raise RuntimeError("hipcc not found")


def build(verbose: bool = False) -> Path:
    srcs = [str(HERE / s) for s in SOURCES if (HERE / s).exists()]
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared", "-ffp-contract=off",
           "-munsafe-fp-atomics", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-Wno-unused-command-line-argument", f"-I{ROOT / 'include'}", "-o", str(tmp)] + srcs
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
