"""Build the gfx950 sampler library in-tree: ferro_amd/libferro_sampler.so (C ABI of include/ferro_sampler.h)."""
from __future__ import annotations

import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
SRC = os.path.join(PKG, "csrc", "sampler_kernels.hip")
LIB = os.path.join(PKG, "libferro_sampler.so")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    # penalties must round exactly as ferro's scalar float ops: no FMA contraction, no fast-math
    "-ffp-contract=off",
    # packed-FP32 instructions are kept out of the device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # the persistent kernel's loop would otherwise hoist exp()'s constants and lane masks out of it and spill them
    "-mllvm", "-disable-machine-licm",
    "-I" + os.path.join(ROOT, "include"),
]


def build(verbose: bool = False) -> str:
    cmd = [HIPCC, *FLAGS, "-o", LIB, SRC]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"hipcc failed ({r.returncode}) building {LIB}")
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
