"""Random-init llama2.c checkpoints and prompts for the config-4 greedy-stream
test (tests/test_e2e.py).

The file layout is the llama2.c version-0 format that the reference's loader
reads (model.cpp:115-163, header checks :59-88): seven int32 header fields
(dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len; a
negative vocab_size means a separate classifier), then fp32 arrays in the
file's order, each projection stored (out x in): token embedding, rms_att,
wq, wk, wv, wo, rms_ffn, w1, w2, w3, rms_final, the legacy RoPE tables
(ignored by the loader; filled with 123.0 here, as the reference's own
fixture does, checkpoint_fixture.h:78-79), then wcls if not shared.

Weights are ~N(0, std) from tests/inputs.py; RMSNorm gains are 1.0, which
the config leaves open (standard init; it keeps logit margins wide).
"""
from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from tests import inputs  # noqa: E402

STORIES15M = dict(dim=288, hidden=768, layers=6, heads=6, kv_heads=6, vocab=32000, seq_len=256)
TINY = dict(dim=16, hidden=40, layers=2, heads=4, kv_heads=2, vocab=29, seq_len=8)


def write_checkpoint(path: str, dim: int, hidden: int, layers: int, heads: int, kv_heads: int,
                     vocab: int, seq_len: int, std: float = 0.02, seed: int = 0,
                     shared: bool = True) -> None:
    hs = dim // heads
    kv = kv_heads * hs
    counter = [seed * 1000]

    def normal(*shape):
        counter[0] += 1
        return inputs.normal(shape, std, counter[0])

    ones = lambda *shape: np.ones(shape, np.float32)  # noqa: E731
    parts = [
        np.array([dim, hidden, layers, heads, kv_heads, vocab if shared else -vocab, seq_len],
                 np.int32),
        normal(vocab, dim),
        ones(layers, dim),
        normal(layers, dim, dim),      # wq (out x in)
        normal(layers, kv, dim),       # wk
        normal(layers, kv, dim),       # wv
        normal(layers, dim, dim),      # wo
        ones(layers, dim),
        normal(layers, hidden, dim),   # w1
        normal(layers, dim, hidden),   # w2
        normal(layers, hidden, dim),   # w3
        ones(dim),
        np.full(seq_len * hs, 123.0, np.float32),
    ]
    if not shared:
        parts.append(normal(vocab, dim))
    with open(path, "wb") as f:
        for p in parts:
            f.write(np.ascontiguousarray(p).astype(p.dtype, copy=False).tobytes())


def write_prompt(path: str, n: int, vocab: int, seed: int) -> list:
    toks = (inputs._splitmix64(seed, n) % np.uint64(vocab)).astype(np.int64).tolist()
    with open(path, "w") as f:
        f.write(" ".join(map(str, toks)) + "\n")
    return toks
