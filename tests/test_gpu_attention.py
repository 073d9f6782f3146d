"""GPU attention (em_attention) against the double-precision oracle.

Mirrors /root/reference/tests/test_cuda_attention.cpp: multi-head,
grouped-query (every heads-per-workgroup case) and multi-query shapes, short
and long contexts, one and several rows (:155-172), every kernel, the
reference's tolerance 5e-5 (:33) against attention in double, and a second
identical call giving the same bits (:88-90, :128-129). Inputs are uniform in
[-1, 1] as the reference draws them (:35-40), from tests/inputs.py.
"""
import numpy as np
import pytest

import oracle
from tests import engine, inputs

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
em = engine.load()
orc = oracle.oracle()

TOL = 5e-5
KERNELS = ["single_block", "split", "automatic"]
# (heads, kv_heads, head_size, seq_len): test_cuda_attention.cpp:158-164.
CASES = [(6, 6, 48, 256), (8, 2, 64, 1000), (8, 1, 32, 600), (4, 2, 16, 300), (6, 2, 32, 300)]


def run_case(case, kernel, positions, rows, seed):
    heads, kv_heads, hs, T = case
    shape = em.attention_shape(heads, kv_heads, hs, T)
    em.attention_check(shape, kernel)
    q = inputs.uniform((rows, shape.q_stride), -1.0, 1.0, seed)
    kc = inputs.uniform((T, shape.kv_stride), -1.0, 1.0, seed + 1)
    vc = inputs.uniform((T, shape.kv_stride), -1.0, 1.0, seed + 2)
    dq, dk, dv = (torch.from_numpy(a).cuda() for a in (q, kc, vc))
    out = torch.empty((rows, shape.out_stride), device="cuda")
    n = em.attention_scratch_floats(shape, rows, kernel)
    scratch = torch.zeros((max(1, n),), device="cuda")
    pos_dev = torch.zeros((1,), dtype=torch.int32, device="cuda")
    worst = 0.0
    for pos in positions:
        if pos < 0 or pos + rows > T:
            continue
        print(f"attention {case} {kernel} rows={rows} pos={pos}", flush=True)
        pos_dev.fill_(pos)
        em.attention(shape, rows, pos_dev, dq, dk, dv, out, scratch, kernel)
        got = out.cpu().numpy()
        em.attention(shape, rows, pos_dev, dq, dk, dv, out, scratch, kernel)
        again = out.cpu().numpy()
        want = orc.attention(heads, kv_heads, hs, rows, pos, q, kc, vc)
        err = float(np.abs(got.astype(np.float64) - want).max())
        worst = max(worst, err)
        assert err <= TOL, f"{case} {kernel} pos {pos} rows {rows}: max diff {err}"
        assert np.array_equal(got, again), "second call gave different bits"
    return worst


@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c)))
@pytest.mark.parametrize("kernel", KERNELS)
def test_kernels_match_double_reference(case, kernel):
    # Positions cover one chunk, chunk edges, many chunks and the end
    # (test_cuda_attention.cpp:165-171).
    T = case[3]
    worst = 0.0
    for i, rows in enumerate((1, 3, 8, 12)):
        worst = max(worst, run_case(case, kernel, (0, 31, 32, 33, 63, 64, 65, 200, T - rows),
                                    rows, seed=7000 + 10 * i))
    print(f"{case} {kernel}: worst {worst:.2e}")


# Prefill rows (automatic, more than 12): the tile kernel for head sizes that
# are multiples of 16 up to 128 (every register layout it is built for, MHA,
# GQA, MQA), the one-chunk-per-row split kernel for the rest (20, 144). These
# grids have few heads, so the tile kernel also splits the context into
# chunks of 256 positions or more and merges them (at 3000 positions, up to
# 12 chunks); rows whose context fits the first chunk are written directly.
PREFILL_CASES = [(4, 4, 16, 200), (8, 2, 64, 700), (4, 1, 80, 300), (2, 1, 96, 300),
                 (3, 3, 112, 200), (8, 2, 128, 700), (6, 6, 48, 256), (4, 4, 32, 300),
                 (4, 2, 20, 200), (2, 2, 144, 300), (4, 2, 128, 3000)]


@pytest.mark.parametrize("case", PREFILL_CASES, ids=lambda c: "x".join(map(str, c)))
def test_prefill_rows_match_double_reference(case):
    # Row counts that fill 16-row tiles exactly and leave them ragged;
    # starting positions on and across 16-position block edges, rows on both
    # sides of a split tile's first chunk edge (position 256) in one tile,
    # and the end of the cache.
    T = case[3]
    worst = 0.0
    for i, rows in enumerate((13, 16, 17, 40, 100)):
        worst = max(worst, run_case(case, "automatic", (0, 15, 16, 31, 33, 250, T - rows),
                                    rows, seed=7400 + 10 * i))
    print(f"{case} prefill: worst {worst:.2e}")


def test_long_context_split_and_automatic():
    # Past single_block's LDS cap (test_cuda_attention.cpp:174-192).
    case = (4, 1, 128, 20000)
    shape = em.attention_shape(*case)
    with pytest.raises(em.InvalidArgument):
        em.attention_check(shape, "single_block")
    run_case(case, "split", (0, 5000, 19999), 1, seed=7100)
    run_case(case, "automatic", (12345, 19990), 10, seed=7200)


def test_graph_replay_reads_the_position_on_device():
    # One captured call serves every position: the grid never depends on it.
    heads, kv_heads, hs, T = 8, 2, 64, 1000
    shape = em.attention_shape(heads, kv_heads, hs, T)
    q = inputs.uniform((1, shape.q_stride), -1.0, 1.0, 7300)
    kc = inputs.uniform((T, shape.kv_stride), -1.0, 1.0, 7301)
    vc = inputs.uniform((T, shape.kv_stride), -1.0, 1.0, 7302)
    dq, dk, dv = (torch.from_numpy(a).cuda() for a in (q, kc, vc))
    out = torch.zeros((1, shape.out_stride), device="cuda")
    scratch = torch.zeros((em.attention_scratch_floats(shape, 1),), device="cuda")
    pos_dev = torch.zeros((1,), dtype=torch.int32, device="cuda")
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        em.attention(shape, 1, pos_dev, dq, dk, dv, out, scratch)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        em.attention(shape, 1, pos_dev, dq, dk, dv, out, scratch)
    for pos in (0, 63, 64, 500, 999, 5):
        pos_dev.fill_(pos)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        eager = em.attention(shape, 1, pos_dev, dq, dk, dv)
        torch.cuda.synchronize()
        assert np.array_equal(got, eager.cpu().numpy()), pos
        want = orc.attention(heads, kv_heads, hs, 1, pos, q, kc, vc)
        assert np.abs(got - want).max() <= TOL
