"""Runs the reference's own GPU test programs, restated against this build's
C++ drop-in headers:
  tests/cpp/test_drop_in          test_cuda.cpp on cuda_matmul.h / matmul.h /
                                  quant.h (llm-engine_amd/build.py builds it)
  tests/cpp/test_cuda_attention   test_cuda_attention.cpp on cuda_attention.h
                                  (llm-engine_amd/build.py)
  oracle/_ref/test_cuda_model     test_cuda_model.cpp on cuda_model.h, with the
                                  reference's CPU Transformer compiled from
                                  source as the checker (oracle/Makefile e2e)
Exit 77 means no GPU (skip), as in the reference's CTest setup
(CMakeLists.txt:112)."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BINS = {
    "matmul": os.path.join(ROOT, "tests", "cpp", "test_drop_in"),
    "attention": os.path.join(ROOT, "tests", "cpp", "test_cuda_attention"),
    "model": os.path.join(ROOT, "oracle", "_ref", "test_cuda_model"),
}


def run(which):
    path = BINS[which]
    if not os.path.exists(path):
        pytest.fail(f"{path} is not built (__graft_entry__.build())")
    return subprocess.run([path], capture_output=True, text=True, timeout=900)


@pytest.mark.parametrize("which", sorted(BINS))
def test_binary_links_and_skips_without_gpu(which):
    import torch
    if torch.cuda.is_available():
        pytest.skip("GPU present: the gpu-marked test runs the suite")
    r = run(which)
    assert r.returncode in (0, 77), r.stdout + r.stderr
    if r.returncode == 77:
        assert "skipping" in r.stdout


@pytest.mark.gpu
@pytest.mark.parametrize("which", sorted(BINS))
def test_reference_gpu_suite_on_drop_in_headers(which):
    r = run(which)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all tests passed" in r.stdout
