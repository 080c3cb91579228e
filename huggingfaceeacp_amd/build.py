"""Build recipe for libgemma_q8.so: hipcc, gfx950 only, in-tree.

Run as ``python -m huggingfaceeacp_amd.build`` (or through
``__graft_entry__.build()``).  The library is written next to this file so it
travels with the source tree.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIBRARY = os.path.join(HERE, "libgemma_q8.so")

SOURCES = ["gq8_kernels.hip", "gq8_decode.hip", "gq8_persist.hip", "gq8_gemm.hip",
           "gq8_batch.hip", "gq8_prefill_attention.hip", "gq8_checkpoint.hip", "gq8_sample.hip",
           "gq8_tokenizer.cpp", "gq8_gemma.cpp",
           "gq8_runtime.hip"]

# Packed FP32 instructions are switched off for every kernel; the compiler
# otherwise forms them from ordinary float code.
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if candidate and os.path.exists(candidate):
            return candidate
    raise RuntimeError("hipcc not found: the gfx950 library cannot be built")


def build(verbose: bool = False) -> str:
    objects = []
    tmp = LIBRARY + ".tmp"
    cmd = [hipcc(), *HIP_FLAGS, "-I", INCLUDE, "-I", CSRC,
           *[os.path.join(CSRC, s) for s in SOURCES], "-o", tmp, "-lpthread"]
    if verbose:
        print(" ".join(cmd), flush=True)
    result = subprocess.run(cmd, capture_output=True, text=True)
    noise = [line for line in (result.stderr or "").splitlines()
             if "packed-fp32-ops' is not a recognized feature" not in line]
    if result.returncode != 0:
        sys.stderr.write("\n".join(noise) + "\n")
        raise RuntimeError("hipcc failed building libgemma_q8.so")
    if verbose and noise:
        sys.stderr.write("\n".join(noise) + "\n")
    os.replace(tmp, LIBRARY)
    del objects
    return LIBRARY


if __name__ == "__main__":
    print(build(verbose=True))
