"""Builds libllm_engine_amd.so for gfx950 in-tree (no JIT cache, no pip install).

    python llm-engine_amd/build.py            # library + C++ drop-in test binary

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
# MFMAs), so its MFMAs write VGPRs instead.
FILE_FLAGS = {
    "attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
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


def build_cpp_tests() -> str:
    """The C++ drop-in tests, linked against the library: tests/cpp/
    test_drop_in.cpp (checker: oracle/liboracle.so) and
    tests/cpp/test_cuda_attention.cpp (its own double-precision checker)."""
    built = []
    inc = ["-I", os.path.join(ROOT, "include")]
    link = [f"-L{HERE}", "-lllm_engine_amd", f"-Wl,-rpath,{HERE}"]
    for name, extra in (("test_drop_in", [f"-L{os.path.join(ROOT, 'oracle')}", "-loracle",
                                           f"-Wl,-rpath,{os.path.join(ROOT, 'oracle')}"]),
                        ("test_cuda_attention", [])):
        src = os.path.join(ROOT, "tests", "cpp", name + ".cpp")
        out = os.path.join(ROOT, "tests", "cpp", name)
        if not os.path.exists(src):
            continue
        _run(["g++", "-O2", "-std=c++17", "-Wall", "-Wextra", *inc, "-o", out, src, *link,
              *extra, "-lm"])
        built.append(out)
    return " ".join(built)


if __name__ == "__main__":
    print(build_library())
    t = build_cpp_tests()
    if t:
        print(t)
    sys.exit(0)
