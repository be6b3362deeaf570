"""Build the gfx950 sampler library in-tree: ferro_amd/libferro_sampler.so (C ABI of include/ferro_sampler.h)."""
from __future__ import annotations

import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
SRC = os.path.join(PKG, "csrc", "sampler_kernels.hip")
LIB = os.path.join(PKG, "libferro_sampler.so")
# the same source with phase timestamps compiled in (-DFS_TRACE, fs_trace_set): read by ferro_amd/trace_phases.py
TRACE_LIB = os.path.join(PKG, "libferro_sampler_trace.so")
# C++ drop-in test driver (tests/cpp): host code over include/ferro_sampler.hpp, linked against LIB
SHIM_SRC = os.path.join(ROOT, "tests", "cpp", "shim_replay.cpp")
SHIM_BIN = os.path.join(ROOT, "tests", "cpp", "shim_replay")
# launch and streaming-read floors for the rocprofv3 traces (profiles/launch_floor.md)
FLOOR_SRC = os.path.join(PKG, "csrc", "launch_floor.hip")
FLOOR_BIN = os.path.join(PKG, "launch_floor")
# per-call timing of the C++ drop-in (bench.py --workload dropin)
DROPIN_SRC = os.path.join(PKG, "csrc", "dropin_bench.cpp")
DROPIN_BIN = os.path.join(PKG, "dropin_bench")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    # penalties must round exactly as ferro's scalar float ops: no FMA contraction, no fast-math
    "-ffp-contract=off",
    # packed-FP32 instructions are kept out of the device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # the persistent kernel's loop would otherwise hoist exp()'s constants and lane masks out of it and spill them
    "-mllvm", "-disable-machine-licm",
    # the kernels' leading scalar parameters arrive in SGPRs at wave launch (no argument loads before the first
    # memory requests)
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-I" + os.path.join(ROOT, "include"),
]


def _run(cmd, what, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"{cmd[0]} failed ({r.returncode}) building {what}")


def build(verbose: bool = False, trace: bool = False) -> str:
    jobs = [([HIPCC, *FLAGS, "-o", LIB, SRC], LIB)]
    if os.path.exists(FLOOR_SRC):
        jobs.append(([HIPCC, *[f for f in FLAGS if f not in ("-shared", "-fPIC")], "-o", FLOOR_BIN, FLOOR_SRC],
                     FLOOR_BIN))
    if trace:
        jobs.append(([HIPCC, *FLAGS, "-DFS_TRACE", "-o", TRACE_LIB, SRC], TRACE_LIB))
    procs = []
    for cmd, what in jobs:                         # the two libraries compile side by side
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True), cmd, what))
    for p, cmd, what in procs:
        out, _ = p.communicate()
        if p.returncode != 0:
            sys.stderr.write(out)
            raise RuntimeError(f"{cmd[0]} failed ({p.returncode}) building {what}")
    for src, out, rpath in ((SHIM_SRC, SHIM_BIN, "$ORIGIN/../../ferro_amd"), (DROPIN_SRC, DROPIN_BIN, "$ORIGIN")):
        if os.path.exists(src):
            _run(["g++", "-O2", "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I" + os.path.join(ROOT, "include"),
                  "-I" + os.path.join(ROCM, "include"), src, "-o", out, "-L" + PKG, "-lferro_sampler",
                  "-L" + os.path.join(ROCM, "lib"), "-lamdhip64", "-Wl,-rpath," + rpath,
                  "-Wl,-rpath," + os.path.join(ROCM, "lib")], out, verbose)
    return LIB


if __name__ == "__main__":
    # `python ferro_amd/build.py --trace` also builds the phase-timestamp library that ferro_amd/trace_phases.py loads
    print(build(verbose=True, trace="--trace" in sys.argv[1:]))
