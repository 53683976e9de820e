"""Builds librusticide_hip.so in-tree with hipcc for gfx950.

Every HIP source is compiled with -ffp-contract=off (float expressions stay
unfused unless the source calls fmaf, as in the CPU path) and without packed
FP32 instructions, then linked into one shared library exporting the C ABI of
include/rusticide_hip.h.
"""

from __future__ import annotations

import concurrent.futures
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "librusticide_hip.so")
SOURCES = ["api.hip", "quantize.hip", "gemv.hip", "gemm.hip", "gemm_i2s.hip", "model.hip", "stream_read.hip", "gguf.hip"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-command-line-argument",
]


# The MFMA GEMMs keep their accumulators in ordinary VGPRs (gfx950 allows
# either file): their accumulators are shifted and read by vector code every
# K block, which the accumulation registers would force through copies, and
# the 128-token tiles fit in 256 registers, two waves per SIMD.
# The GEMV kernels' leading scalar arguments go into SGPRs before the first
# instruction (gfx950 kernel-argument preload): the _pl kernel forms put the
# activation's pointer and sizes first, so its loads wait on no argument load.
SOURCE_FLAGS = {
    "gemv.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=16"],
    "gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
    "gemm_i2s.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *FLAGS, *SOURCE_FLAGS.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build() -> str:
    os.makedirs(BUILD, exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=4) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
