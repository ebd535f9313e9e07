"""Build recipe for libpkv_hip.so (gfx950), invoked by __graft_entry__.build().

hipcc compiles the kernels and the host half together; -ffp-contract=off keeps
every multiply-add rounded twice (the reference's Rust arithmetic), and packed
FP32 instructions are disabled for the device code.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libpkv_hip.so")
SOURCES = ["pkv_kernels.hip", "pkv_records.hip", "pkv_blake3.hip", "pkv_lloyd.hip", "pkv_capi.cpp", "pkv_profile.cpp",
           "pkv_json.cpp"]

FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-ffp-contract=off",
    "-fno-fast-math",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in VGPRs (gfx950 allows it): no v_accvgpr_read per
    # result element in the fib encode scoring loop
    "-mllvm", "-amdgpu-mfma-vgpr-form",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    return "hipcc"


def build(verbose: bool = False) -> str:
    srcs = []
    for s in SOURCES:
        p = os.path.join(CSRC, s)
        srcs += (["-x", "hip", p] if s.endswith(".cpp") else [p])
    tmp = LIB + ".tmp"
    cmd = [hipcc()] + FLAGS + srcs + ["-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print(LIB)
