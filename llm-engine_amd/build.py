"""Builds libllm_engine_amd.so for gfx950 in-tree (no JIT cache, no pip install).

    python llm-engine_amd/build.py            # the library

(The reference's own C++ test programs and bench are compiled against the
drop-in headers by oracle/Makefile's e2e target.)

Each csrc/*.hip compiles to an object under _build/ in parallel, then one
hipcc line links the shared library next to this file. Flags:
  --offload-arch=gfx950                 CDNA4 only
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                        no v_pk_*_f32 (packed fp32 ops have given
                                        wrong results on these boxes)
  -fhip-fp32-correctly-rounded-divide-sqrt
                                        IEEE division: quantize_q8's scale and
                                        reciprocal must round as the CPU's do
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libllm_engine_amd.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-I", os.path.join(ROOT, "include"),
    "-I", os.path.join(HERE, "csrc"),
]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{r.stdout}{r.stderr}")
    return r


# Per-file additions. attention.hip: the tile kernel rescales its MFMA
# accumulators with VALU ops after every key block; in the default AGPR form
# each rescale copies them out of and back into AGPRs (~300 moves per 128
# MFMAs), so its MFMAs write VGPRs instead. gemm_mfma.hip: in the AGPR form
# the one-workgroup-per-CU build of the fp32 GEMM loop moved accumulators
# between AGPRs and VGPRs (80 moves per 256 MFMAs). decode_mfma.hip: its
# accumulators are read by VALU reductions right after the loop.
FILE_FLAGS = {
    "attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "gemm_mfma.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "decode_mfma.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    _run([HIPCC, *HIP_FLAGS, *FILE_FLAGS.get(os.path.basename(src), []), "-c", src, "-o", obj])
    return obj


def build_library(jobs: int = 0) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(HERE, "csrc", "*.hip")))
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 2)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build_library())
    sys.exit(0)
