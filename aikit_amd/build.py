"""Build recipe for libenchip.so (gfx950) -- used by __graft_entry__.build().

One translation unit, compiled by hipcc for gfx950 only, linked as a plain C-ABI
shared library next to this file. Flags that matter for correctness:

* ``-ffp-contract=off`` -- the epilogue must round after every multiply and add,
  as aikit's Go amd64 arithmetic does (no FMA contraction).
* ``-fhip-fp32-correctly-rounded-divide-sqrt`` -- the quantizer's maxAbs/127 and
  1/s and the erf tail's 1/(1+p*x) must be IEEE-correct divisions.
* ``-Xclang -target-feature -Xclang -packed-fp32-ops`` -- no packed-FP32 VALU ops
  (the host pass warns that it does not know the feature; harmless).
"""
from __future__ import annotations

import os
import shutil
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SRC = os.path.join(HERE, "csrc", "enchip.hip")
OUT = os.path.join(HERE, "libenchip.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]


def hipcc() -> str:
    p = os.path.join(ROCM, "bin", "hipcc")
    return p if os.path.exists(p) else (shutil.which("hipcc") or "hipcc")


def build(verbose: bool = False) -> str:
    """Compile libenchip.so in-tree; returns its path. Always recompiles."""
    tmp = OUT + ".tmp"
    cmd = [hipcc(), *HIPCC_FLAGS,
           "-I", os.path.join(ROOT, "include"), "-I", os.path.join(HERE, "csrc"),
           SRC, "-o", tmp, f"-Wl,-rpath,{ROCM}/lib"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{err}")
    if verbose and err.strip():
        print(err)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
