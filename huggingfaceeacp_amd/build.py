"""Build recipe for libgemma_q8.so: hipcc, gfx950 only, in-tree.

Run as ``python -m huggingfaceeacp_amd.build`` (or through
``__graft_entry__.build()``).  The library is written next to this file so it
travels with the source tree.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIBRARY = os.path.join(HERE, "libgemma_q8.so")

SOURCES = ["gq8_kernels.hip", "gq8_decode.hip", "gq8_gemm.hip",
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


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    result = subprocess.run(cmd, capture_output=True, text=True)
    noise = [line for line in (result.stderr or "").splitlines()
             if "packed-fp32-ops' is not a recognized feature" not in line]
    return result.returncode, noise


def build(verbose: bool = False, jobs: int = 0) -> str:
    """Compiles every source to an object (in parallel: each translation unit
    holds its own kernels), then links the shared library."""
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    base = [hipcc(), *HIP_FLAGS, "-I", INCLUDE, "-I", CSRC]
    compiles = []
    for source in SOURCES:
        obj = os.path.join(objdir, os.path.splitext(source)[0] + ".o")
        cmd = [*[a for a in base if a != "-shared"], "-c", os.path.join(CSRC, source), "-o", obj]
        compiles.append((source, obj, cmd))
    workers = jobs if jobs > 0 else min(len(compiles), os.cpu_count() or 1, 16)
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        results = list(pool.map(lambda c: _run(c[2], verbose), compiles))
    failed = False
    for (source, _, _), (code, noise) in zip(compiles, results):
        if code != 0 or (verbose and noise):
            sys.stderr.write(f"--- {source}\n" + "\n".join(noise) + "\n")
        failed |= code != 0
    if failed:
        raise RuntimeError("hipcc failed building libgemma_q8.so")
    tmp = LIBRARY + ".tmp"
    code, noise = _run([*base, *[o for _, o, _ in compiles], "-o", tmp, "-lpthread"], verbose)
    if code != 0:
        sys.stderr.write("\n".join(noise) + "\n")
        raise RuntimeError("linking libgemma_q8.so failed")
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build(verbose=True))
