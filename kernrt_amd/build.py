"""Build libkernrt_hip.so in-tree for gfx950 with hipcc.

Flags:
  -ffp-contract=off   only explicit fma() fuses: the kernels reproduce the
                      reference's f32 rounding sequence bit for bit.
  -Xclang -target-feature -Xclang -packed-fp32-ops
                      no packed FP32 (v_pk_*_f32) code generation.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libkernrt_hip.so")

SOURCES = ["kernels.hip", "gemm.hip", "attn_mx.hip", "backend.hip", "llm.cpp"]
# per-source extra flags: the matrix-core attention and the Q8_0 GEMM keep
# MFMA results in ordinary vector registers (their vector epilogues read them
# directly)
EXTRA = {"attn_mx.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"], "gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}

FLAGS = [
    "-O3", "-std=c++17", "--offload-arch=gfx950", "-fPIC", "-shared",
    "-ffp-contract=off", "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-result",
    "-I", os.path.join(ROOT, "include"),
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build the HIP backend)")


def _run(cmd, verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build(verbose: bool = False) -> str:
    """Each source to an object (with its own extra flags), compiled in
    parallel, then one shared library."""
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    flags = [f for f in FLAGS if f != "-shared"]
    jobs = []
    for src in SOURCES:
        path = os.path.join(CSRC, src)
        obj = os.path.join(objdir, src + ".o")
        cmd = [hipcc(), *flags, *EXTRA.get(src, []), "-c", path, "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        jobs.append((cmd, obj, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)))
    noise = "'-packed-fp32-ops' is not a recognized feature"
    for cmd, obj, p in jobs:
        _, stderr = p.communicate()
        err = "\n".join(l for l in stderr.splitlines() if noise not in l)
        if p.returncode != 0:
            raise RuntimeError(f"hipcc failed ({p.returncode}) on {cmd[-3]}:\n{err}")
        if verbose and err.strip():
            print(err, file=sys.stderr)
    tmp = LIB + ".tmp"
    _run([hipcc(), "--offload-arch=gfx950", "-fPIC", "-shared", *[o for _, o, _ in jobs], "-o", tmp], verbose)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
