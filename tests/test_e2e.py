"""The stories15M-shaped Llama forward (the benchmark's end-to-end case) with every matmul
on this build's kernels gives the same greedy token stream as the CPU path.

Both sides run the reference's own model code (model.cpp, ops.cpp,
quant.cpp, thread_pool.cpp compiled from source by oracle/Makefile):
stories_cpu with the reference's matmul.cpp, stories_gpu with
tests/cpp/gpu_matmul_shim.cpp, which sends Transformer::project's 25
products per token (model.cpp:256-258) to em_matmul_f32 / em_matmul_q8.
The prompt (158 random tokens) is prefilled as one batch (m = 158 products),
then 98 greedy decode steps follow (m = 1 products): 99 tokens, as
generate.cpp:68-86 counts them.
"""
import json
import os
import subprocess

import pytest

from tests import e2e_model

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = os.path.join(ROOT, "oracle", "_ref")
CPU_BIN = os.path.join(REF, "stories_cpu")
GPU_BIN = os.path.join(REF, "stories_gpu")


def run(binary, ckpt, prompt, wtype, n_decode):
    if not os.path.exists(binary):
        pytest.fail(f"{binary} is not built (make -C oracle e2e)")
    r = subprocess.run([binary, ckpt, prompt, wtype, str(n_decode)], capture_output=True,
                       text=True, timeout=900)
    assert r.returncode == 0, r.stdout + r.stderr
    return json.loads(r.stdout)


@pytest.fixture(scope="module", params=[True, False], ids=["tied", "untied"])
def stories15m(request, tmp_path_factory):
    # The config fixes the shape and N(0, 0.02) weights, not whether the
    # classifier is tied to the embedding (stories15M's is): both are run.
    # With such small weights the stream settles on a few tokens, with
    # top-2 margins down to ~5e-4 -- still far above the ~1e-6 relative
    # difference between two fp32 summation orders.
    d = tmp_path_factory.mktemp("stories15m")
    ckpt, prompt = str(d / "model.bin"), str(d / "prompt.txt")
    e2e_model.write_checkpoint(ckpt, seed=15, shared=request.param, **e2e_model.STORIES15M)
    e2e_model.write_prompt(prompt, 158, e2e_model.STORIES15M["vocab"], seed=158)
    return ckpt, prompt


@pytest.fixture(scope="module")
def tiny(tmp_path_factory):
    d = tmp_path_factory.mktemp("tiny")
    ckpt, prompt = str(d / "model.bin"), str(d / "prompt.txt")
    e2e_model.write_checkpoint(ckpt, std=0.4, seed=3, shared=False, **e2e_model.TINY)
    e2e_model.write_prompt(prompt, 3, e2e_model.TINY["vocab"], seed=4)
    return ckpt, prompt


def test_checkpoint_size_matches_reference_loader(tmp_path):
    # expected_size(), model.cpp:74-83, for both classifier layouts.
    c = e2e_model.STORIES15M
    D, H, L, V, S = c["dim"], c["hidden"], c["layers"], c["vocab"], c["seq_len"]
    KV = c["kv_heads"] * (D // c["heads"])
    per_layer = 2 * D + 2 * D * D + 2 * D * KV + 3 * D * H
    floats = V * D + L * per_layer + D + S * (D // c["heads"])
    for shared in (True, False):
        path = str(tmp_path / f"m{shared}.bin")
        e2e_model.write_checkpoint(path, seed=1, shared=shared, **c)
        assert os.path.getsize(path) == 28 + 4 * (floats + (0 if shared else V * D))


def test_cpu_path_runs_and_is_deterministic(tiny):
    ckpt, prompt = tiny
    a = run(CPU_BIN, ckpt, prompt, "f32", 4)
    b = run(CPU_BIN, ckpt, prompt, "f32", 4)
    assert len(a["tokens"]) == 5 and a["tokens"] == b["tokens"]
    assert all(0 <= t < e2e_model.TINY["vocab"] for t in a["tokens"])


@pytest.mark.gpu
@pytest.mark.parametrize("wtype", ["f32", "q8"])
def test_tiny_model_stream(tiny, wtype):
    ckpt, prompt = tiny
    cpu = run(CPU_BIN, ckpt, prompt, wtype, 4)
    gpu = run(GPU_BIN, ckpt, prompt, wtype, 4)
    assert gpu["tokens"] == cpu["tokens"]


@pytest.mark.gpu
@pytest.mark.parametrize("wtype", ["f32", "q8"])
def test_config4_greedy_stream_identical(stories15m, wtype):
    ckpt, prompt = stories15m
    cpu = run(CPU_BIN, ckpt, prompt, wtype, 98)
    gpu = run(GPU_BIN, ckpt, prompt, wtype, 98)
    assert len(cpu["tokens"]) == 99
    first_diff = next((i for i, (a, b) in enumerate(zip(cpu["tokens"], gpu["tokens"])) if a != b),
                      None)
    print(f"{wtype}: min top-2 margin {min(cpu['margins']):.3g}; "
          f"cpu decode {cpu['decode_ms_per_token']:.3f} ms/tok, gpu {gpu['decode_ms_per_token']:.3f}")
    assert first_diff is None, (
        f"streams differ at step {first_diff} (cpu margin there "
        f"{cpu['margins'][first_diff]:.3g})")
