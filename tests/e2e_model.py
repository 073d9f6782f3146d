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

# File order of the per-layer arrays after the embedding (model.cpp:138-149).
_LAYER_ORDER = ("rms_att", "wq", "wk", "wv", "wo", "rms_ffn", "w1", "w2", "w3")


def fixture_model(heads: int, kv_heads: int, shared: bool, seed: int, dim: int = 16,
                  hidden: int = 40, layers: int = 2, vocab: int = 29, seq_len: int = 8) -> dict:
    """Raw weights (file layout, projections out x in) drawn as the
    reference's model-test fixture draws them (checkpoint_fixture.h:30-52):
    uniform, embedding and classifier in +-1, wq/wk/wv +-0.4, wo/w1/w2/w3
    +-0.3, rms_att 1 +- 0.2, rms_ffn +-0.2, rms_final +-1. The bits come from
    tests/inputs.py, not mt19937."""
    hs = dim // heads
    kv = kv_heads * hs
    counter = [seed * 1000]

    def u(shape, scale, offset=0.0):
        counter[0] += 1
        return (inputs.uniform(shape, -scale, scale, counter[0]) + np.float32(offset)).astype(
            np.float32)

    m = dict(dim=dim, hidden=hidden, layers=layers, heads=heads, kv_heads=kv_heads, vocab=vocab,
             seq_len=seq_len, shared=shared, emb=u((vocab, dim), 1.0))
    per = {k: [] for k in _LAYER_ORDER}
    for _ in range(layers):
        per["rms_att"].append(u((dim,), 0.2, 1.0))
        per["rms_ffn"].append(u((dim,), 0.2))
        per["wq"].append(u((dim, dim), 0.4))
        per["wk"].append(u((kv, dim), 0.4))
        per["wv"].append(u((kv, dim), 0.4))
        per["wo"].append(u((dim, dim), 0.3))
        per["w1"].append(u((hidden, dim), 0.3))
        per["w2"].append(u((dim, hidden), 0.3))
        per["w3"].append(u((hidden, dim), 0.3))
    m.update(per)
    m["rms_final"] = u((dim,), 1.0)
    m["wcls"] = None if shared else u((vocab, dim), 1.0)
    return m


def write_raw(path: str, m: dict) -> None:
    """A llama2.c v0 file from fixture_model()'s arrays."""
    hs = m["dim"] // m["heads"]
    header = np.array([m["dim"], m["hidden"], m["layers"], m["heads"], m["kv_heads"],
                       m["vocab"] if m["shared"] else -m["vocab"], m["seq_len"]], np.int32)
    parts = [header, m["emb"]]
    for k in _LAYER_ORDER:
        parts.extend(m[k])
    parts.append(m["rms_final"])
    parts.append(np.full(m["seq_len"] * hs, 123.0, np.float32))
    if not m["shared"]:
        parts.append(m["wcls"])
    with open(path, "wb") as f:
        for p in parts:
            f.write(np.ascontiguousarray(p).tobytes())


def model_layout(m: dict) -> tuple:
    """(config, weights) in the CPU model's layout, restating the loader
    (model.cpp:127-163): projections transposed to in x out, q|k|v and w1|w3
    concatenated by columns, a tied classifier = the embedding transposed."""
    cfg = dict(dim=m["dim"], hidden_dim=m["hidden"], n_layers=m["layers"], n_heads=m["heads"],
               n_kv_heads=m["kv_heads"], vocab_size=m["vocab"], seq_len=m["seq_len"])
    layers = []
    for l in range(m["layers"]):
        layers.append(dict(
            rms_att=m["rms_att"][l],
            wqkv=np.concatenate([m["wq"][l].T, m["wk"][l].T, m["wv"][l].T], axis=1),
            wo=np.ascontiguousarray(m["wo"][l].T),
            rms_ffn=m["rms_ffn"][l],
            w13=np.concatenate([m["w1"][l].T, m["w3"][l].T], axis=1),
            w2=np.ascontiguousarray(m["w2"][l].T)))
    wcls = m["emb"].T if m["shared"] else m["wcls"].T
    return cfg, dict(token_embedding=m["emb"], rms_final=m["rms_final"],
                     wcls=np.ascontiguousarray(wcls, np.float32), layers=layers)


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
