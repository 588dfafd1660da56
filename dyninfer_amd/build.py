"""Build the gfx950 kernel library in-tree: dyninfer_amd/libdyninfer_mi355x.so.

hipcc compiles every translation unit under csrc/ for gfx950 only (no other
targets, no CUDA path) and links one shared library exporting the C ABI of
include/dyninfer_mi355x.h.  Packed-FP32 instruction selection is disabled
(-packed-fp32-ops) for every device compile.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libdyninfer_mi355x.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

SOURCES = [
    "gemv_q6_k.hip", "gemv_q4_k.hip", "gemv_q5_k.hip", "gemv_iq4_xs.hip", "gemv_q4_0.hip", "gemv_q4_1.hip", "gemv_q8_0.hip", "gemv_mlx_u4.hip",
    "gemm_q6_k.hip", "gemm_q5_k.hip", "gemm_iq4_xs.hip", "gemm_q4_k.hip", "gemm_q8_0.hip", "gemm_mlx_u4.hip",
    "gemm_q4_0.hip", "gemm_q4_1.hip",
    "gemv.hip", "gemv_mfma.hip", "gemm.hip", "xprep.hip", "dequant.hip", "embedding.hip",
    "capi.cpp", "registry.cpp", "gguf.cpp", "safetensors.cpp",
]
COMMON = [
    "--offload-arch=gfx950",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, src + ".o")
    cmd = [HIPCC, *COMMON, "-c", os.path.join(CSRC, src), "-o", obj]
    if src.endswith(".cpp"):
        cmd[cmd.index("-c"):cmd.index("-c")] = ["-x", "hip"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature; drop that line only
    noise = "'-packed-fp32-ops' is not a recognized feature for this target (ignoring feature)"
    msgs = [ln for ln in (r.stdout + r.stderr).splitlines() if noise not in ln]
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n" + "\n".join(msgs))
    if msgs:
        print("\n".join(msgs), file=sys.stderr)
    return obj


def build(jobs: int | None = None) -> str:
    os.makedirs(BUILD, exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 4)
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stdout + r.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
