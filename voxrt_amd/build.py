"""Build libvoxrt_hip.so (gfx950) in-tree with hipcc: every source to an object in parallel (voxrt_amd/_build/),
then one link.

Flags that the numerics depend on:
  -ffp-contract=off                 every a*b+c stays two rounded operations, as the Rust reference computes it
  -fno-gpu-flush-denormals-to-zero  fp32 denormals are kept (IEEE), as on the CPU
  -target-feature -packed-fp32-ops  no packed fp32 instructions are generated
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libvoxrt_hip.so")
SOURCES = ["vx_abi.hip", "vx_weights.hip", "vx_quant.hip", "vx_gemm.hip", "vx_gemm_stream.hip", "vx_gemm_stream_g.hip", "vx_gemm_small.hip", "vx_glue.hip", "vx_attn.hip",
           "vx_encoder.hip"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-ffp-contract=off", "-fno-gpu-flush-denormals-to-zero", "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"hipcc failed ({r.returncode}): {' '.join(cmd[-3:])}")


def build(verbose: bool = False) -> str:
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    os.makedirs(OBJ, exist_ok=True)
    objs = [os.path.join(OBJ, os.path.splitext(s)[0] + ".o") for s in SOURCES]
    jobs = max(1, min(len(SOURCES), os.cpu_count() or 1))
    with cf.ThreadPoolExecutor(jobs) as ex:
        futs = [ex.submit(_run, [hipcc, *HIPCC_FLAGS, "-c", os.path.join(CSRC, s), "-o", o], verbose)
                for s, o in zip(SOURCES, objs)]
        for f in futs:
            f.result()
    tmp = LIB + ".tmp"
    _run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp], verbose)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
