"""GPU parity of 9 .. 16-row int8 products over the strip layout
(strip_split.hip: one launch, its k slices added inside it), through
em_matmul_q8_packed and through em_matmul_q8 over registered weights, against
the CPU oracle; and of registered-weight batches of 9 .. 64 rows with every
fusion and the ranged magnitudes.

The reference runs these shapes as tiled_split plus sum_slices
(cuda_matmul.cu:333-363, 245-254); its tests hold them to 1e-5 * k (2k with
fusion, test_cuda.cpp:38-47,126-165) and bit-identical repeats
(test_cuda.cpp:272), and the north star to 1e-4 * sum_k |a||w| per element.
The exact split's only error is fp32 summation order, so it is also held to
1e-5 * sum|a||w| where the inputs are plain.
"""
import numpy as np
import pytest

import oracle
from tests import engine, inputs

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
em = engine.load()
orc = oracle.oracle()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def check(got, want, A, Bf, k, factor=1.0, C0=None):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    assert err.max() <= 1e-5 * max(k, 1) * factor, f"max err {err.max()} (k={k})"
    bound = orc.abs_bound(A, Bf)
    if C0 is not None:
        bound = bound + np.abs(C0)
    assert np.all(err <= 1e-4 * bound + 1e-30), "1e-4 * sum|a||w| bound exceeded"


def run_registered(A, q, s, C0=None, w=None, repeats=2):
    """em_matmul_q8 (automatic) over registered q, `repeats` times; the
    outputs as numpy arrays."""
    m, k = A.shape
    n = q.shape[1]
    qd, sd = dev(q), dev(s)
    wd = dev(w) if w is not None else None
    em.register_q8(qd)
    try:
        assert em.registered_q8(qd)
        outs = []
        for _ in range(repeats):
            C = dev(C0) if C0 is not None else torch.empty((m, n), device="cuda")
            em.matmul(dev(A), qd, C, scale=sd, accumulate=C0 is not None, rms_weight=wd)
            outs.append(host(C).copy())
    finally:
        em.unregister_q8(qd)
    return outs


def run_packed(A, q, s, C0=None, w=None, repeats=2):
    """em_matmul_q8_packed over q's strip layout, `repeats` times."""
    m, k = A.shape
    n = q.shape[1]
    P, sd = em.pack_q8(dev(q)), dev(s)
    wd = dev(w) if w is not None else None
    outs = []
    for _ in range(repeats):
        C = dev(C0) if C0 is not None else torch.empty((m, n), device="cuda")
        em.matmul_packed(dev(A), P, n, sd, C, accumulate=C0 is not None, rms_weight=wd)
        outs.append(host(C).copy())
    return outs


@pytest.mark.parametrize("fusion", ["plain", "acc", "rms", "rms_acc"])
@pytest.mark.parametrize("m", [9, 12, 16])
def test_strip_4096_against_oracle(m, fusion):
    # Config 2's m = 16 row and its neighbours: 4096^2 split into 64 tiles x
    # 4 slices. automatic over registered weights takes the same kernel here,
    # so it must give the same bits.
    k = n = 4096
    A = inputs.normal((m, k), 1.0, 900 + m)
    q, s = orc.quantize_q8(inputs.normal((k, n), 0.02, 901))
    acc = "acc" in fusion
    rms = "rms" in fusion
    C0 = inputs.uniform((m, n), -1.0, 1.0, 902) if acc else None
    w = inputs.uniform((k,), 0.5, 1.5, 903) if rms else None
    outs = run_packed(A, q, s, C0, w)
    assert np.array_equal(outs[0], outs[1]), "repeat not bit-identical"
    assert np.array_equal(outs[0], run_registered(A, q, s, C0, w, repeats=1)[0])
    want = orc.matmul_fused(A, Bq=q, scale=s, w=w, C0=C0)
    An = orc.rmsnorm(A, w) if rms else A
    Bf = orc.dequantize(q, s)
    check(outs[0], want, An, Bf, k, 2.0 if (acc or rms) else 1.0, C0)
    if fusion == "plain":
        exact = orc.matmul_f64(A, Bf)
        ratio = np.abs(outs[0] - exact) / np.maximum(orc.abs_bound(A, Bf), 1e-300)
        assert ratio.max() <= 1e-5, ratio.max()


@pytest.mark.parametrize("fusion", ["plain", "acc", "rms", "rms_acc"])
@pytest.mark.parametrize("m", [24, 32, 48, 64])
def test_registered_batches_above_16_rows(m, fusion):
    # automatic over registered weights above 16 rows: the row-major exact
    # split, unchanged by registration (the same bits as unregistered).
    k = n = 4096
    A = inputs.normal((m, k), 1.0, 905 + m)
    q, s = orc.quantize_q8(inputs.normal((k, n), 0.02, 906))
    acc = "acc" in fusion
    rms = "rms" in fusion
    C0 = inputs.uniform((m, n), -1.0, 1.0, 907) if acc else None
    w = inputs.uniform((k,), 0.5, 1.5, 908) if rms else None
    outs = run_registered(A, q, s, C0, w)
    assert np.array_equal(outs[0], outs[1])
    C = dev(C0) if acc else torch.empty((m, n), device="cuda")
    em.matmul(dev(A), dev(q), C, scale=dev(s), accumulate=acc, rms_weight=dev(w) if rms else None)
    assert np.array_equal(outs[0], host(C))
    want = orc.matmul_fused(A, Bq=q, scale=s, w=w, C0=C0)
    An = orc.rmsnorm(A, w) if rms else A
    check(outs[0], want, An, orc.dequantize(q, s), k, 2.0 if (acc or rms) else 1.0, C0)


# n not a multiple of 64 (a tile of 2 strips: 288; 54 strips: 864), k not a
# multiple of 32 (300, 1028: masked chunks), the Llama-7B shapes (k = 11008
# deep; n = 11008 and 32000 wide, one slice), a tiny k (one chunk, most waves
# idle) and 16 columns.
SHAPES = [(288, 864), (768, 288), (300, 1536), (1028, 272), (4096, 11008), (11008, 4096),
          (4096, 32000), (32, 64), (4, 16), (2048, 16)]


@pytest.mark.parametrize("fusion", ["plain", "rms_acc"])
@pytest.mark.parametrize("m", [9, 16])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_strip_shapes_against_oracle(shape, m, fusion):
    k, n = shape
    A = inputs.uniform((m, k), -1.0, 1.0, 910)
    q, s = orc.quantize_q8(inputs.normal((k, n), 0.02, 911))
    acc = rms = fusion == "rms_acc"
    C0 = inputs.uniform((m, n), -1.0, 1.0, 912) if acc else None
    w = inputs.uniform((k,), 0.5, 1.5, 913) if rms else None
    outs = run_packed(A, q, s, C0, w)
    assert np.array_equal(outs[0], outs[1]), "repeat not bit-identical"
    want = orc.matmul_fused(A, Bq=q, scale=s, w=w, C0=C0)
    An = orc.rmsnorm(A, w) if rms else A
    check(outs[0], want, An, orc.dequantize(q, s), k, 2.0 if (acc or rms) else 1.0, C0)


@pytest.mark.parametrize("case", [(16, 4096, 4096, True), (9, 288, 864, True), (12, 768, 288, True),
                                  (16, 4096, 12288, True), (16, 11008, 4096, False),
                                  (16, 4096, 32000, False), (12, 1024, 2048, False)],
                         ids=lambda c: "x".join(map(str, c[:3])))
def test_automatic_routing_over_registered_weights(case):
    # Where the strip kernel is preferred, automatic over registered weights
    # gives em_matmul_q8_packed's bits; elsewhere the row-major exact split's
    # (the same bits as unregistered weights).
    m, k, n, strip = case
    A = inputs.normal((m, k), 1.0, 915)
    q, s = orc.quantize_q8(inputs.normal((k, n), 0.02, 916))
    got = run_registered(A, q, s, repeats=1)[0]
    if strip:
        assert np.array_equal(got, run_packed(A, q, s, repeats=1)[0])
    else:
        assert np.array_equal(got, host(em.matmul(dev(A), dev(q), scale=dev(s))))
    check(got, orc.matmul_fused(A, Bq=q, scale=s), A, orc.dequantize(q, s), k)


def test_strip_shapes_in_turn_and_back():
    # Calls of different tile and slice counts in a row (the counters and
    # partials grow, and each call must leave its counters at zero), then
    # the first shape again: the same bits as its first call.
    cases = []
    for i, (m, k, n) in enumerate([(16, 4096, 4096), (9, 11008, 4096), (12, 288, 864),
                                   (16, 4096, 11008), (10, 1028, 272)]):
        A = inputs.normal((m, k), 1.0, 920 + i)
        q, s = orc.quantize_q8(inputs.normal((k, n), 0.02, 930 + i))
        cases.append((A, q, s, dev(A), em.pack_q8(dev(q)), dev(s)))
    first = [host(em.matmul_packed(Ad, P, q.shape[1], sd)).copy() for _, q, _, Ad, P, sd in cases]
    again = [host(em.matmul_packed(Ad, P, q.shape[1], sd)).copy()
             for _, q, _, Ad, P, sd in reversed(cases)]
    for (A, q, s, *_), f, a in zip(cases, first, reversed(again)):
        assert np.array_equal(f, a)
        check(f, orc.matmul_fused(A, Bq=q, scale=s), A, orc.dequantize(q, s), A.shape[1])


def ranged_rows(m, k, seed):
    """Rows that stress the three-term split, one class per row (as in
    test_gpu_matmul.py): log-uniform over 1e-38 .. 1e-30, one magnitude near
    1e-37, fp32's smallest normals, subnormals, and 1e-38 .. 1e20 mixed."""
    ln_ranges = [(np.log(1e-38), np.log(1e-30)), (-85.2, -85.2 + 0.7),
                 (np.log(2.0 ** -126), np.log(2.0 ** -126) + 0.05),
                 (np.log(1.5e-45), np.log(1e-38)), (np.log(1e-38), np.log(1e20))]
    rows = []
    for r in range(m):
        a, b = ln_ranges[r % len(ln_ranges)]
        mag = np.exp(inputs.uniform((k,), a, b, seed + r).astype(np.float64)).astype(np.float32)
        sign = np.where(inputs.uniform((k,), -1.0, 1.0, seed + 7919 + r) < 0, -1.0, 1.0)
        rows.append((mag * sign).astype(np.float32))
    return np.stack(rows).astype(np.float32)


@pytest.mark.parametrize("shape", [(16, 4096, 512), (16, 4096, 4096), (13, 300, 272),
                                   (9, 8192, 64)], ids=lambda s: "x".join(map(str, s)))
def test_strip_tiny_magnitudes(shape):
    # Blocks whose lo terms drop bits are computed again by fp32
    # multiply-adds: every row within 1e-4 * sum|a||w| of the f64 product
    # (plus fp32's subnormal spacing). With the norm, a row whose sum of
    # squares passes fp32's range gets a zero row, as the fp32 norm does.
    m, k, n = shape
    A = ranged_rows(m, k, 941)
    q, s = orc.quantize_q8(inputs.normal((k, n), 0.02, 942))
    Bf = orc.dequantize(q, s)
    w = inputs.uniform((k,), 0.5, 1.5, 943)
    floor = 2.0 ** -149
    ss = (A.astype(np.float64) ** 2).sum(axis=1)
    fits = ss < float(np.finfo(np.float32).max)
    for norm in (False, True):
        outs = run_packed(A, q, s, w=w if norm else None)
        assert np.array_equal(outs[0], outs[1])
        got = outs[0].astype(np.float64)
        rows = fits if norm else np.ones(m, bool)
        Ause = orc.rmsnorm(A[rows], w) if norm else A
        err = np.abs(got[rows] - orc.matmul_f64(Ause, Bf))
        bound = orc.abs_bound(Ause, Bf)
        assert np.all(err <= 1e-4 * bound + floor), (norm, float((err / np.maximum(bound, 1e-300)).max()))
        if norm:
            assert np.all(got[~rows] == 0.0)


@pytest.mark.parametrize("m", [9, 12, 16, 24, 32, 48, 64])
def test_registered_ranged_magnitudes(m):
    # The ranged rows through em_matmul_q8 over registered weights, at every
    # batch size the decode batches use (the strip kernel up to 16 rows, the
    # row-major exact split above): within 1e-4 * sum|a||w| of the f64
    # product plus fp32's subnormal spacing, bit-identical on repeat, with
    # and without the norm.
    k = n = 4096
    A = ranged_rows(m, k, 971 + m)
    q, s = orc.quantize_q8(inputs.normal((k, n), 0.02, 972))
    Bf = orc.dequantize(q, s)
    w = inputs.uniform((k,), 0.5, 1.5, 973)
    floor = 2.0 ** -149
    fits = (A.astype(np.float64) ** 2).sum(axis=1) < float(np.finfo(np.float32).max)
    for norm in (False, True):
        outs = run_registered(A, q, s, w=w if norm else None)
        assert np.array_equal(outs[0], outs[1]), "repeat not bit-identical"
        got = outs[0].astype(np.float64)
        rows = fits if norm else np.ones(m, bool)
        Ause = orc.rmsnorm(A[rows], w) if norm else A
        err = np.abs(got[rows] - orc.matmul_f64(Ause, Bf))
        bound = orc.abs_bound(Ause, Bf)
        assert np.all(err <= 1e-4 * bound + floor), (norm, float((err / np.maximum(bound, 1e-300)).max()))
        if norm:
            assert np.all(got[~rows] == 0.0)


def test_strip_infinities_pass_through():
    # An infinite activation gives +-inf where its weight is non-zero and NaN
    # where it is zero; a NaN activation makes its row NaN; other rows stay
    # within the bound.
    m, k, n = 16, 4096, 512
    A = inputs.normal((m, k), 1.0, 951)
    A[1, 5] = np.inf
    A[3, 7] = -np.inf
    A[5, 3] = np.inf
    A[5, k - 1] = -np.inf
    A[7, 100] = np.nan
    q, s = orc.quantize_q8(inputs.normal((k, n), 0.02, 952))
    q[5, :n // 4] = 0
    Bf = orc.dequantize(q, s)
    with np.errstate(invalid="ignore", over="ignore"):
        want = A.astype(np.float64) @ Bf.astype(np.float64)
    got = run_packed(A, q, s)[0].astype(np.float64)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(np.isposinf(got), np.isposinf(want))
    assert np.array_equal(np.isneginf(got), np.isneginf(want))
    finite_rows = [r for r in range(m) if np.all(np.isfinite(A[r]))]
    err = np.abs(got[finite_rows] - want[finite_rows])
    assert np.all(err <= 1e-4 * orc.abs_bound(A[finite_rows], Bf))


def test_registered_batch_graph_replay_matches_eager():
    # Captured once, replayed five times with eager products of another
    # shape in between (they use the same counters and partials): every
    # replay equals the eager result bit for bit.
    m, k, n = 16, 4096, 4096
    q, s = em.quantize_q8(dev(inputs.normal((k, n), 0.02, 961)))
    A = dev(inputs.normal((m, k), 1.0, 962))
    q2, s2 = em.quantize_q8(dev(inputs.normal((288, 864), 0.02, 963)))
    A2 = dev(inputs.normal((12, 288), 1.0, 964))
    em.register_q8(q)
    em.register_q8(q2)
    try:
        eager = host(em.matmul(A, q, scale=s)).copy()
        other = host(em.matmul(A2, q2, scale=s2)).copy()
        C = torch.empty((m, n), device="cuda")
        stream = torch.cuda.Stream()
        with torch.cuda.stream(stream):
            em.matmul(A, q, C, scale=s)  # any growth before capture
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                em.matmul(A, q, C, scale=s)
        for _ in range(5):
            C.zero_()
            graph.replay()
            assert np.array_equal(host(C), eager)
            assert np.array_equal(host(em.matmul(A2, q2, scale=s2)), other)
    finally:
        em.unregister_q8(q)
        em.unregister_q8(q2)
