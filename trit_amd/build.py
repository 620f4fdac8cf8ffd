"""Builds libtrit_hip.so (the HIP kernels and the C ABI) for gfx950, in tree.

Run as `python -m trit_amd.build`. hipcc cross-compiles on a host without a
GPU; the built library sits next to this file and travels with the tree.
"""

from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "lib", "libtrit_hip.so")
# The measurement build: the persistent step's phase stamps compiled in.
OUT_STAMPS = os.path.join(HERE, "lib", "libtrit_hip_stamps.so")
SOURCES = ["layer.hip", "gemv.hip", "gemv_decode.hip", "gemv_stream.hip", "gemv_float.hip", "gemm.hip", "decoder.hip", "decode_step.hip", "attention_mfma.hip", "gguf.hip", "encoder.hip", "tokenizer.cpp"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Every fused multiply-add is explicit in the source; nothing else fuses.
    "-ffp-contract=off",
    # Packed FP32 instructions stay off.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]


def build(verbose: bool = False, jobs: int = 0, stamps: bool = False) -> str:
    """Compiles the sources in parallel (`jobs` at a time; 0: up to 8), then
    links. stamps: the measurement library with the step's phase stamps."""
    from concurrent.futures import ThreadPoolExecutor

    out = OUT_STAMPS if stamps else OUT
    os.makedirs(os.path.dirname(out), exist_ok=True)
    cmds, objs = [], []
    extra = ["-DTRIT_HIP_STEP_STAMPS"] if stamps else []
    for src in SOURCES:
        path = os.path.join(CSRC, src)
        if not os.path.exists(path):
            raise RuntimeError(f"build: source {path} is missing")
        obj = os.path.join(HERE, "lib", os.path.splitext(src)[0] + (".stamps.o" if stamps else ".o"))
        cmds.append([HIPCC, *FLAGS, *extra, "-c", path, "-o", obj])
        objs.append(obj)
    if verbose:
        for cmd in cmds:
            print(" ".join(cmd), flush=True)
    with ThreadPoolExecutor(jobs or min(8, os.cpu_count() or 1)) as pool:
        list(pool.map(run, cmds))
    tmp = out + ".tmp"
    run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, out)
    for obj in objs:
        os.remove(obj)
    return out


def run(cmd):
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = ("packed-fp32-ops", "not a recognized feature", "is not a recognized feature")
    err = "\n".join(line for line in res.stderr.splitlines() if not any(n in line for n in noise))
    if res.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{err}")
    if err.strip():
        print(err, file=sys.stderr)


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv, stamps="--stamps" in sys.argv))
