"""Runs tests/cpp/test_drop_in (the reference's test_cuda.cpp against this
build's C++ drop-in headers). Built by __graft_entry__.build() /
llm-engine_amd/build.py; exit 77 means no GPU (skip), as in the reference's
CTest setup (CMakeLists.txt:112)."""
import os
import subprocess

import pytest

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "test_drop_in")


def run():
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} is not built (python llm-engine_amd/build.py)")
    return subprocess.run([BIN], capture_output=True, text=True, timeout=600)


def test_binary_links_and_skips_without_gpu():
    r = run()
    assert r.returncode in (0, 77), r.stdout + r.stderr
    if r.returncode == 77:
        assert "skipping" in r.stdout


@pytest.mark.gpu
def test_reference_gpu_suite_on_drop_in_headers():
    r = run()
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all tests passed" in r.stdout
