"""Runs the reference's own GPU test programs and CPU bench, compiled
unchanged from /root/reference against this build's drop-in headers by
oracle/Makefile's e2e target (the built binaries travel in oracle/_ref):
  oracle/_ref/test_cuda          tests/test_cuda.cpp: every GpuKernel, fusion,
                                 int8 B, split-K queue and error message, with
                                 the reference's CPU matmul.cpp as the checker
  oracle/_ref/test_cuda_model    tests/test_cuda_model.cpp: this build's
                                 CudaTransformer against the reference's CPU
                                 Transformer (model.cpp)
  oracle/_ref/bench_matmul_gpu   bench/bench_matmul.cpp on this build's
                                 matmul.h / quant.h (the GPU entry points)
  oracle/_ref/test_matmul_gpu    tests/test_matmul.cpp on the same headers:
                                 the known answer, 17 edge shapes at 1e-5 k,
                                 thread counts, the "2x3"/"4x2" message
  oracle/_ref/test_quant_gpu     tests/test_quant.cpp on the same headers:
                                 quantize_q8 / dequantize round trip and the
                                 int8 products against the dequantized ones
The reference's cuda_attention test and bench_cuda include the CUDA runtime
and cuBLAS directly, so they cannot be built here; tests/test_gpu_attention.py
covers attention. Exit 77 means no GPU (skip), as in the reference's CTest
setup (CMakeLists.txt:112)."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_BIN = os.path.join(ROOT, "oracle", "_ref")
SUITES = {
    "matmul": os.path.join(REF_BIN, "test_cuda"),
    "model": os.path.join(REF_BIN, "test_cuda_model"),
}
BENCH = os.path.join(REF_BIN, "bench_matmul_gpu")
# The reference's CPU-entry-point tests (no GPU check of their own: run on
# the GPU box only).
CPU_ENTRY = {
    "matmul": os.path.join(REF_BIN, "test_matmul_gpu"),
    "quant": os.path.join(REF_BIN, "test_quant_gpu"),
}


def run(path, *args, timeout=900):
    if not os.path.exists(path):
        pytest.fail(f"{path} is not built (__graft_entry__.build())")
    return subprocess.run([path, *args], capture_output=True, text=True, timeout=timeout)


@pytest.mark.parametrize("which", sorted(SUITES))
def test_reference_suite_links_and_skips_without_gpu(which):
    import torch
    if torch.cuda.is_available():
        pytest.skip("GPU present: the gpu-marked test runs the suite")
    r = run(SUITES[which])
    assert r.returncode == 77, r.stdout + r.stderr
    assert "skipping" in r.stdout


@pytest.mark.parametrize("path", [BENCH] + [CPU_ENTRY[k] for k in sorted(CPU_ENTRY)],
                         ids=["bench_matmul"] + sorted(CPU_ENTRY))
def test_reference_cpu_entry_programs_link(path):
    if not os.path.exists(path):
        pytest.fail(f"{path} is not built (__graft_entry__.build())")
    out = subprocess.run(["ldd", path], capture_output=True, text=True).stdout
    assert "libllm_engine_amd.so" in out, out


@pytest.mark.gpu
@pytest.mark.parametrize("which", sorted(CPU_ENTRY))
def test_reference_cpu_entry_tests_on_the_gpu(which):
    # matmul_naive / blocked / parallel and quantize_q8 / dequantize with the
    # reference's signatures, each call on the MI355X.
    r = run(CPU_ENTRY[which], timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all tests passed" in r.stdout


@pytest.mark.gpu
@pytest.mark.parametrize("which", sorted(SUITES))
def test_reference_gpu_suite_on_drop_in_headers(which):
    r = run(SUITES[which])
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all tests passed" in r.stdout


@pytest.mark.gpu
def test_reference_bench_matmul_on_the_gpu_entry_points():
    # bench_matmul.cpp's square table (sizes given: the decode table is
    # skipped, bench_matmul.cpp:95) through matmul_naive / blocked / parallel.
    r = run(BENCH, "128", "256", "512", timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    lines = [l for l in r.stdout.splitlines() if l.strip()[:3].strip().isdigit()]
    assert [int(l.split("|")[0]) for l in lines] == [128, 256, 512], r.stdout
    for l in lines:
        cells = [c.split() for c in l.split("|")[1:]]
        assert all(len(c) == 2 and float(c[1]) > 0 for c in cells), l
