"""GPU parity of every kernel against the CPU oracle.

Mirrors /root/reference/tests/test_cuda.cpp: the same shapes (:63-72), every
GpuKernel (:55-61), every MatmulFusion (:123-165), int8 B (:167-213), the
split-K queue with bit-identical repeats (:215-275) and output reuse
(:91-105). Two tolerances are checked: the reference tests' own
|got - want| <= 1e-5 * k (2k with fusion), and the north star's
|got - want| <= 1e-4 * sum_k |a||w| per element.
"""
import numpy as np
import pytest

import oracle
from tests import engine, inputs

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
em = engine.load()
orc = oracle.oracle()

KERNELS = ["naive", "tiled", "tiled_split", "skinny", "automatic"]
MAX_M = {"skinny": 8}

# (m, k, n): test_cuda.cpp:66-72.
SHAPES = [
    (1, 1, 1), (1, 17, 1), (3, 5, 7), (8, 8, 128), (9, 9, 129),
    (127, 300, 129), (128, 256, 128), (200, 513, 33), (130, 70, 1030),
    (1, 4096, 288), (1, 288, 4096), (2, 1000, 70), (4, 4097, 33), (7, 64, 4111),
    (8, 513, 2049), (16, 4096, 300), (33, 1029, 257), (64, 2000, 4096),
    (1, 0, 5), (12, 0, 3),
]
# Extra int8 shapes for 4 | n and 16 | n lanes (test_cuda.cpp:172-175) and the
# MFMA tiles' edges.
Q8_EXTRA = [(3, 100, 1028), (8, 1000, 4100), (6, 20, 36), (1, 4096, 4), (24, 300, 512),
            (40, 777, 272), (65, 64, 96)]


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def check(got, want, A, Bf, k, factor=1.0, C0=None):
    """Both bounds; Bf is the fp32 (or dequantised) B, A the (normed) A."""
    assert got.shape == want.shape
    if got.size == 0:
        return
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    assert err.max() <= 1e-5 * max(k, 1) * factor, f"max err {err.max()} (k={k})"
    bound = orc.abs_bound(A, Bf) if k else np.zeros(got.shape)
    if C0 is not None:
        bound = bound + np.abs(C0)
    assert np.all(err <= 1e-4 * bound + 1e-30), "1e-4 * sum|a||w| bound exceeded"


def seeded(m, k, n, seed):
    A = inputs.uniform((m, k), -1.0, 1.0, seed)
    B = inputs.uniform((k, n), -1.0, 1.0, seed + 1)
    return A, B


@pytest.mark.parametrize("kernel", KERNELS)
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_fp32_against_oracle(kernel, shape):
    m, k, n = shape
    if m > MAX_M.get(kernel, 1 << 30):
        pytest.skip("skinny takes m <= 8")
    A, B = seeded(m, k, n, 42)
    want = orc.matmul_naive(A, B)
    got = host(em.matmul(dev(A), dev(B), kernel=kernel))
    check(got, want, A, B, k)


@pytest.mark.parametrize("kernel", KERNELS)
@pytest.mark.parametrize("shape", SHAPES + Q8_EXTRA, ids=lambda s: "x".join(map(str, s)))
def test_q8_against_oracle(kernel, shape):
    m, k, n = shape
    if m > MAX_M.get(kernel, 1 << 30):
        pytest.skip("skinny takes m <= 8")
    A = inputs.uniform((m, k), -1.0, 1.0, 11)
    q, s = orc.quantize_q8(inputs.uniform((k, n), -1.0, 1.0, 12))
    want = orc.matmul_fused(A, Bq=q, scale=s)
    got = host(em.matmul(dev(A), dev(q), scale=dev(s), kernel=kernel))
    check(got, want, A, orc.dequantize(q, s), k)


FUSION_SHAPES = [(1, 288, 300), (3, 100, 70), (8, 513, 129), (9, 64, 33), (70, 40, 130),
                 (16, 288, 864), (5, 768, 288), (2, 20, 64), (3, 288, 30)]


@pytest.mark.parametrize("q8", [False, True], ids=["f32", "q8"])
@pytest.mark.parametrize("kernel", KERNELS)
@pytest.mark.parametrize("shape", FUSION_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_fusion(kernel, shape, q8):
    # test_cuda.cpp:126-165,190-212: accumulate, rms, rms + accumulate.
    m, k, n = shape
    if m > MAX_M.get(kernel, 1 << 30):
        pytest.skip("skinny takes m <= 8")
    A = inputs.uniform((m, k), -1.0, 1.0, 9)
    Bsrc = inputs.uniform((k, n), -1.0, 1.0, 10)
    C0 = inputs.uniform((m, n), -1.0, 1.0, 13)
    w = inputs.uniform((k,), -1.0, 1.0, 14)
    if q8:
        q, s = orc.quantize_q8(Bsrc)
        Bf = orc.dequantize(q, s)
        kw = dict(Bq=q, scale=s)
        dB, dS = dev(q), dev(s)
    else:
        Bf = Bsrc
        kw = dict(B=Bsrc)
        dB, dS = dev(Bsrc), None
    normed = orc.rmsnorm(A, w)
    for acc, use_w in [(True, False), (False, True), (True, True)]:
        want = orc.matmul_fused(A, w=w if use_w else None, C0=C0 if acc else None, **kw)
        C = dev(C0.copy())
        em.matmul(dev(A), dB, C, scale=dS, kernel=kernel, accumulate=acc,
                  rms_weight=dev(w) if use_w else None)
        check(host(C), want, normed if use_w else A, Bf, k, factor=2.0,
              C0=C0 if acc else None)


def test_split_k_queue_is_deterministic():
    # test_cuda.cpp:221-275: products queued back to back with no host sync,
    # over 1..many k slices and both lane widths; repeats must match bit for bit.
    cases = [((1, 4096, 4096), False, False), ((8, 4096, 4100), True, True),
             ((1, 288, 32000), True, False), ((3, 768, 288), False, True),
             ((1, 288, 864), True, True), ((5, 1000, 70), True, False),
             ((16, 4096, 4096), True, False), ((64, 4096, 4096), True, True),
             ((48, 2000, 1000), False, True), ((200, 2048, 256), False, False)]
    for rnd in range(2):
        outs, wants = [], []
        keep = []
        for idx, ((m, k, n), q8, acc) in enumerate(cases):
            A = inputs.uniform((m, k), -1, 1, 100 + 10 * idx + rnd)
            Bsrc = inputs.uniform((k, n), -1, 1, 101 + 10 * idx + rnd)
            C0 = inputs.uniform((m, n), -1, 1, 102 + 10 * idx + rnd)
            if q8:
                q, s = orc.quantize_q8(Bsrc)
                dB, dS = dev(q), dev(s)
                want = orc.matmul_fused(A, Bq=q, scale=s, C0=C0 if acc else None)
            else:
                dB, dS = dev(Bsrc), None
                want = orc.matmul_fused(A, B=Bsrc, C0=C0 if acc else None)
            dA = dev(A)
            keep.append((dA, dB, dS))
            kernel = "skinny" if m <= 8 else "automatic"
            for _ in range(3):
                C = dev(C0.copy())
                em.matmul(dA, dB, C, scale=dS, kernel=kernel, accumulate=acc)
                outs.append((C, k))
                wants.append(want)
        torch.cuda.synchronize()
        got = [c.cpu().numpy() for c, _ in outs]
        for i, (g, want) in enumerate(zip(got, wants)):
            k = outs[i][1]
            assert np.abs(g - want).max() <= 2e-5 * k, f"case {i // 3}"
            if i % 3:
                assert np.array_equal(g.view(np.uint32), got[i - 1].view(np.uint32)), \
                    f"case {i // 3}: repeat differs"


def test_reuse_across_growing_scratch():
    # test_cuda.cpp:93-105: shapes of growing split-K scratch, one after another.
    for i, (m, k, n) in enumerate([(1, 2000, 300), (4, 100, 5000), (64, 3000, 64), (200, 64, 64),
                                   (2, 8192, 8192)]):
        A, B = seeded(m, k, n, 5 + 2 * i)
        got = host(em.matmul(dev(A), dev(B)))
        check(got, orc.matmul_naive(A, B), A, B, k)


def big_skinny(seed, k=65536):
    """An int8 skinny product whose split-K partials (8 rows x 16384 columns
    x k / 256 slices: 128 MiB at k = 65536) outgrow every other test's;
    B stays under the 2^31 elements the entry points accept."""
    m, n = 8, 16384
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    B = torch.randint(-127, 128, (k, n), generator=g, device="cuda", dtype=torch.int8)
    s = torch.rand((n,), generator=g, device="cuda") * 1e-3
    A = torch.randn((m, k), generator=g, device="cuda")
    return A, B, s


def test_scratch_generation_bumps_on_growth_only():
    # cuda_scratch_generation (src/cuda_matmul.h:112, cuda_matmul.cu:268-281,567):
    # growing the scratch bumps it; a shape that fits what is there does not.
    A, B, s = big_skinny(1)
    gen0 = em.scratch_generation()
    C1 = em.matmul(A, B, scale=s, kernel="skinny")
    torch.cuda.synchronize()
    gen1 = em.scratch_generation()
    assert gen1 > gen0
    C2 = em.matmul(A, B, scale=s, kernel="skinny")
    torch.cuda.synchronize()
    assert em.scratch_generation() == gen1  # same shape: no growth
    assert torch.equal(C1, C2)
    A2, B2 = seeded(4, 3000, 2000, 17)
    got = host(em.matmul(dev(A2), dev(B2), kernel="skinny"))  # smaller: fits
    assert em.scratch_generation() == gen1
    check(got, orc.matmul_naive(A2, B2), A2, B2, 3000)
    del A, B, s, C1, C2
    torch.cuda.synchronize()


def test_graph_recaptured_after_generation_bump():
    # The graph user's rule (cuda_model.cu:175-177,196): a graph captured
    # before a bump points at freed scratch, so it is captured again; the new
    # graph's replays equal eager results. (The old graph is not replayed.)
    m, k, n = 2, 8192, 4096
    A, B = seeded(m, k, n, 23)
    dA, dB = dev(A), dev(B)
    C = torch.empty((m, n), device="cuda")

    def capture():
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            em.matmul(dA, dB, C, kernel="skinny")
        return g

    em.matmul(dA, dB, C, kernel="skinny")  # scratch for this shape exists
    eager = host(C).copy()
    g = capture()
    gen = em.scratch_generation()
    g.replay()
    assert np.array_equal(host(C), eager)
    Ab, Bb, sb = big_skinny(2, k=98304)  # 384 slices: past the generation test's 256
    em.matmul(Ab, Bb, scale=sb, kernel="skinny")  # grows the scratch
    torch.cuda.synchronize()
    assert em.scratch_generation() > gen
    del g, Ab, Bb, sb
    g = capture()
    for _ in range(3):
        C.zero_()
        torch.cuda.synchronize()
        g.replay()
        assert np.array_equal(host(C), eager)
    del g
    torch.cuda.synchronize()


def test_bad_shapes_on_device():
    with pytest.raises(em.InvalidArgument) as e:
        em.matmul(dev(np.zeros((2, 3), np.float32)), dev(np.zeros((4, 2), np.float32)))
    assert "2x3" in str(e.value) and "4x2" in str(e.value)
    with pytest.raises(em.InvalidArgument):
        em.matmul(dev(np.zeros((9, 2), np.float32)), dev(np.zeros((2, 2), np.float32)),
                  kernel="skinny")


def test_k_zero_zeroes_or_keeps_C():
    C0 = inputs.uniform((12, 3), -1, 1, 3)
    for kernel in KERNELS:
        if kernel == "skinny":
            continue
        C = dev(C0.copy())
        em.matmul(dev(np.zeros((12, 0), np.float32)), dev(np.zeros((0, 3), np.float32)), C,
                  kernel=kernel)
        assert not host(C).any()
        C = dev(C0.copy())
        em.matmul(dev(np.zeros((12, 0), np.float32)), dev(np.zeros((0, 3), np.float32)), C,
                  kernel=kernel, accumulate=True)
        assert np.array_equal(host(C), C0)


def test_graph_replay_matches_eager():
    # The reference replays its decode step as a graph (cuda_model.cu:189-230).
    # Capture fused split-K GEMVs (whose last workgroup re-arms its tile
    # counter), a tiled_split product and a GEMM with residual adds; replay
    # several times with eager work in between; every replay must equal the
    # eager result bit for bit.
    specs = [((1, 4096, 4096), True, False, "skinny"), ((4, 2048, 1000), False, True, "skinny"),
             ((16, 4096, 1024), True, False, "tiled_split"), ((130, 512, 256), False, True, "tiled")]
    tensors = []
    for i, ((m, k, n), q8, acc, kernel) in enumerate(specs):
        A = inputs.uniform((m, k), -1, 1, 500 + i)
        Bsrc = inputs.uniform((k, n), -1, 1, 600 + i)
        C0 = inputs.uniform((m, n), -1, 1, 700 + i)
        if q8:
            q, s = orc.quantize_q8(Bsrc)
            dB, dS = dev(q), dev(s)
        else:
            dB, dS = dev(Bsrc), None
        tensors.append((dev(A), dB, dS, dev(C0), C0, acc, kernel))

    def run_all(outs):
        for (dA, dB, dS, _, C0h, acc, kernel), C in zip(tensors, outs):
            em.matmul(dA, dB, C, scale=dS, kernel=kernel, accumulate=acc)

    eager = [t[3].clone() for t in tensors]
    run_all(eager)
    torch.cuda.synchronize()
    eager = [e.cpu().numpy() for e in eager]

    outs = [t[3].clone() for t in tensors]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run_all([t[3].clone() for t in tensors])  # grow scratch outside capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run_all(outs)
    for rep in range(3):
        for o, t in zip(outs, tensors):
            o.copy_(t[3])
        g.replay()
        torch.cuda.synchronize()
        for i, (o, e) in enumerate(zip(outs, eager)):
            assert np.array_equal(o.cpu().numpy().view(np.uint32), e.view(np.uint32)), \
                f"replay {rep}, product {i}"
        extra = em.matmul(tensors[0][0], tensors[0][1], scale=tensors[0][2])  # eager in between
        torch.cuda.synchronize()
        del extra


# ---- The benchmark configurations' shapes at full size --------------------

@pytest.mark.parametrize("m", [1, 4, 16, 64])
def test_config2_int8_gemv_4096(m):
    # Config 2: W ~ N(0, 0.02) 4096^2 quantised on the GPU, A ~ N(0, 1).
    W = inputs.normal((4096, 4096), 0.02, 1001)
    A = inputs.normal((m, 4096), 1.0, 2000 + m)
    q, s = em.quantize_q8(dev(W))
    qh, sh = host(q), host(s)
    want = orc.matmul_fused(A, Bq=qh, scale=sh)
    got = host(em.matmul(dev(A), q, scale=s))
    check(got, want, A, orc.dequantize(qh, sh), 4096)


def test_config1_fp32_gemv_4096():
    W = inputs.normal((4096, 4096), 0.02, 1001)
    A = inputs.normal((1, 4096), 1.0, 2001)
    got = host(em.matmul(dev(A), dev(W)))
    check(got, orc.matmul_naive(A, W), A, W, 4096)


# Config 5: Llama-7B layer projections, int8 (quantised on the GPU), decode
# m = 1 (every element checked) and prefill m = 512 (rows sampled against
# the f64 product and the 1e-4 * sum|a||w| bound). (k, n) = (in, out).
LLAMA7B = {"wq": (4096, 4096), "w1": (4096, 11008), "w2": (11008, 4096), "cls": (4096, 32000)}


@pytest.mark.parametrize("name", sorted(LLAMA7B))
def test_config5_llama7b_projections(name):
    k, n = LLAMA7B[name]
    W = inputs.normal((k, n), 0.02, 5000 + k + n)
    q, s = em.quantize_q8(dev(W))
    qh, sh = host(q), host(s)
    Wd = orc.dequantize(qh, sh)
    A1 = inputs.normal((1, k), 1.0, 6000 + n)
    got1 = host(em.matmul(dev(A1), q, scale=s))
    check(got1, orc.matmul_fused(A1, Bq=qh, scale=sh), A1, Wd, k)
    A = inputs.normal((512, k), 1.0, 7000 + n)
    got = host(em.matmul(dev(A), q, scale=s))
    rows = np.array([0, 1, 77, 255, 256, 400, 510, 511])
    exact = orc.matmul_f64(A[rows], Wd)
    assert np.all(np.abs(got[rows] - exact) <= 1e-4 * orc.abs_bound(A[rows], Wd))
    # The whole C against the reference's matmul_parallel(A, QTensor) at the
    # reference tests' 1e-5 * k, as config 3 does (oracle/_ref present).
    ref = oracle.ref()
    if ref is not None:
        want = ref.matmul_q8(A, qh, sh)
        assert np.abs(got - want).max() <= 1e-5 * k


@pytest.mark.parametrize("N", [1024, 2048, 4096])
def test_config3_square_gemm(N):
    # Config 3: A, B ~ U(-1, 1) N x N on the MFMA GEMM. Full C against the
    # reference's matmul_parallel where oracle/_ref is present; rows sampled
    # against the f64 oracle and its sum|a||b| bound always.
    A = inputs.uniform((N, N), -1.0, 1.0, 3000 + N)
    B = inputs.uniform((N, N), -1.0, 1.0, 4000 + N)
    got = host(em.matmul(dev(A), dev(B), kernel="tiled"))
    rows = np.linspace(0, N - 1, 16).astype(int)
    exact = orc.matmul_f64(A[rows], B)
    bound = orc.abs_bound(A[rows], B)
    assert np.all(np.abs(got[rows] - exact) <= 1e-4 * bound)
    ref = oracle.ref()
    if ref is not None:
        want = ref.matmul(A, B, "parallel")
        assert np.abs(got - want).max() <= 1e-5 * N


# The streamlined fp32 tiled kernel (k % 32 == 0, n % 4 == 0): rows and
# columns ending inside a 64 x 64 tile (out-of-range buffer loads must read
# zeros and stores must stop), one row, k split over slices when the tile
# grid is small (1 tile, k = 8192: 32 slices), accumulate into a non-zero C,
# and a grid whose tile count is not a multiple of 8 (no XCD reordering).
FAST_SHAPES = [(100, 96, 68), (1, 4096, 1028), (64, 8192, 64), (65, 32, 4),
               (300, 1024, 700), (129, 2048, 1924), (7 * 64, 256, 5 * 64)]


@pytest.mark.parametrize("shape", FAST_SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("accumulate", [False, True])
def test_tiled_fast_kernel_edges(shape, accumulate):
    m, k, n = shape
    A, B = seeded(m, k, n, 77)
    C0 = inputs.uniform((m, n), -1.0, 1.0, 79) if accumulate else np.zeros((m, n), np.float32)
    C = dev(C0)
    got = host(em.matmul(dev(A), dev(B), C, kernel="tiled", accumulate=accumulate))
    want = orc.matmul_naive(A, B) + C0
    check(got, want, A, B, k, C0=C0 if accumulate else None)


# ------------------------------------------------- exact-split bf16 products

# Covers one, two and four 16-row blocks per workgroup (m <= 256, < 1024,
# >= 1024), k whole chunks of 32 or ragged, k not a multiple of 8 (pre-split
# planes), and m and n that end inside a tile.
SPLIT_SHAPES = [(9, 300, 32), (12, 4096, 4096), (24, 4096, 4096), (64, 4096, 4096), (100, 777, 272),
                (512, 4096, 512), (33, 1029, 256), (64, 31, 48), (300, 4096, 256), (1024, 1024, 512),
                (1040, 520, 272), (1100, 301, 160),
                # wide products, with k whole chunks or ragged, A split in
                # registers or pre-split, m ending inside a tile
                (512, 4096, 12288), (300, 520, 12288), (200, 301, 32768), (2048, 1024, 4096)]


# automatic's cuts below 9 rows, on both sides: int8 B goes to the exact-split
# kernel from 5 rows, from 3 at 2^25 weights and from 2 at 2^26; fp32 B to
# tiled_split from 4 rows at 2^25. (m, k, n, int8)
ROUTING_CASES = [(2, 4096, 8176, True), (2, 4096, 8192, True), (3, 4096, 8192, True),
                 (4, 4096, 4096, True), (5, 4096, 4096, True), (8, 2048, 4112, True),
                 (2, 4096, 16384, True), (3, 4096, 8176, True),
                 (3, 4096, 8192, False), (4, 4096, 8192, False), (8, 4096, 8192, False),
                 (4, 4096, 8176, False)]


@pytest.mark.parametrize("case", ROUTING_CASES, ids=lambda c: "x".join(map(str, c[:3])) +
                         ("_q8" if c[3] else "_f32"))
def test_automatic_small_m_routing_matches_oracle(case):
    # Whichever kernel automatic picks at these sizes, with and without the
    # fused norm and accumulation, every element within the north star's
    # 1e-4 * sum_k |a||w|.
    m, k, n, q8 = case
    A = inputs.normal((m, k), 1.0, 521 + m)
    C0 = inputs.normal((m, n), 1.0, 522)
    w = inputs.uniform((k,), 0.5, 1.5, 523)
    if q8:
        q, s = orc.quantize_q8(inputs.normal((k, n), 0.02, 524))
        Bf = orc.dequantize(q, s)
        B, scale = dev(q), dev(s)
    else:
        Bf = inputs.normal((k, n), 0.02, 524)
        B, scale = dev(Bf), None
    An = orc.rmsnorm(A, w)
    for norm in (False, True):
        Ause = An if norm else A
        want = orc.matmul_f64(Ause, Bf) + C0.astype(np.float64)
        bound = orc.abs_bound(Ause, Bf)
        C = dev(C0)
        em.matmul(dev(A), B, C, scale=scale, accumulate=True,
                  rms_weight=dev(w) if norm else None)
        got = host(C).astype(np.float64)
        ratio = float((np.abs(got - want) / np.maximum(bound, 1e-30)).max())
        print(f"{case} norm={norm}: max |err| / sum|a||w| = {ratio:.2e}")
        assert ratio <= 1e-4, (case, norm, ratio)


@pytest.mark.parametrize("shape", SPLIT_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_exact_split_tighter_than_fp32_tolerance(shape):
    # automatic sends int8 B above 8 rows to the exact-split bf16 kernel: with A
    # split exactly into three bf16 terms, its only error is fp32 summation
    # order, so it must sit far inside the north star's 1e-4 * sum|a||w|.
    # A spans 1e-20 .. 1e20 within each row, which block-scaled (shared
    # exponent) formats could not hold; per-element bf16 exponents do.
    m, k, n = shape
    mag = np.exp(inputs.uniform((m, k), -46.0, 46.0, 501)).astype(np.float32)
    sign = np.where(inputs.uniform((m, k), -1.0, 1.0, 502) < 0, -1.0, 1.0).astype(np.float32)
    A = (mag * sign).astype(np.float32)
    q, s = orc.quantize_q8(inputs.normal((k, n), 0.02, 503))
    Bf = orc.dequantize(q, s)
    exact = orc.matmul_f64(A, Bf)
    bound = orc.abs_bound(A, Bf)
    for kernel in ("automatic", "tiled_split"):
        got = host(em.matmul(dev(A), dev(q), scale=dev(s), kernel=kernel)).astype(np.float64)
        ratio = float((np.abs(got - exact) / np.maximum(bound, 1e-300)).max())
        print(f"{shape} {kernel}: max |err| / sum|a||w| = {ratio:.2e}")
        assert ratio <= 1e-5, (kernel, ratio)


def ranged_rows(m, k, seed):
    """Rows of A that stress the three-term split, each row one class:
    log-uniform over 1e-38 .. 1e-30 (remainders far below fp32's normal
    range), one magnitude near 1e-37 (every value's low bits subnormal),
    fp32's smallest normals (2^-126 and just above), subnormals (1.5e-45 ..
    1e-38), and mixed over 1e-38 .. 1e20; signs random."""
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


# k a multiple of 8 (A split in registers), ragged k (pre-split planes), one
# 16-row block and several, a split k.
RANGE_SHAPES = [(16, 4096, 512), (12, 1029, 256), (64, 4096, 4096), (40, 300, 272),
                (512, 4096, 512), (9, 8192, 64)]


@pytest.mark.parametrize("shape", RANGE_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_exact_split_tiny_magnitudes(shape):
    # Each row's sum against the f64 product within 1e-4 * sum|a||w|, with
    # and without the fused norm (the pre-pass path). A C element may round
    # into fp32's subnormal range, where its spacing is 2^-149: that much
    # absolute slack is allowed, the reference's fp32 sum has no less.
    # The fused norm sums squares in fp32, as the reference's CUDA norm does
    # (cuda_matmul.cu:162-170,256-266; its CPU rmsnorm sums in double): a
    # row whose sum of squares passes fp32's range (values past ~1.8e19)
    # gets scale 1 / sqrt(inf) = 0 and a zero row of C there, which is what
    # is checked for it.
    m, k, n = shape
    A = ranged_rows(m, k, 531)
    q, s = orc.quantize_q8(inputs.normal((k, n), 0.02, 532))
    Bf = orc.dequantize(q, s)
    w = inputs.uniform((k,), 0.5, 1.5, 533)
    floor = 2.0 ** -149
    ss = (A.astype(np.float64) ** 2).sum(axis=1)
    fits = ss < float(np.finfo(np.float32).max)
    assert fits.sum() >= m // 2 and (~fits).any()
    for kernel in ("automatic", "tiled_split"):
        for norm in (False, True):
            rows = fits if norm else np.ones(m, bool)
            Ause = orc.rmsnorm(A[rows], w) if norm else A
            exact = orc.matmul_f64(Ause, Bf)
            bound = orc.abs_bound(Ause, Bf)
            got = host(em.matmul(dev(A), dev(q), scale=dev(s), kernel=kernel,
                                 rms_weight=dev(w) if norm else None)).astype(np.float64)
            err = np.abs(got[rows] - exact)
            ratio = float((err / np.maximum(bound, 1e-300)).max())
            print(f"{shape} {kernel} norm={norm}: max |err| / sum|a||w| = {ratio:.2e}")
            assert np.all(err <= 1e-4 * bound + floor), (kernel, norm, ratio)
            if norm:
                assert np.all(got[~rows] == 0.0), kernel


@pytest.mark.parametrize("shape", [(16, 4096, 512), (12, 1029, 256)],
                         ids=lambda s: "x".join(map(str, s)))
def test_exact_split_infinities_pass_through(shape):
    # An infinite activation gives +-inf in every column where its weight is
    # non-zero and NaN where it is zero (inf * 0), as fp32 arithmetic and the
    # reference's CPU product do; rows without one stay finite and within
    # the bound. A NaN activation makes its row NaN.
    m, k, n = shape
    A = inputs.normal((m, k), 1.0, 541)
    A[1, 5] = np.inf
    A[3, 7] = -np.inf
    A[5, 3] = np.inf
    A[5, k - 1] = -np.inf  # both signs in one row: NaN where both weights are non-zero
    A[7, 100] = np.nan
    q, s = orc.quantize_q8(inputs.normal((k, n), 0.02, 542))
    q[5, :n // 4] = 0  # inf * 0 columns
    Bf = orc.dequantize(q, s)
    with np.errstate(invalid="ignore", over="ignore"):
        want = A.astype(np.float64) @ Bf.astype(np.float64)
    finite_rows = [r for r in range(m) if np.all(np.isfinite(A[r]))]
    bound = orc.abs_bound(A[finite_rows], Bf)
    for kernel in ("automatic", "tiled_split"):
        got = host(em.matmul(dev(A), dev(q), scale=dev(s), kernel=kernel)).astype(np.float64)
        assert np.array_equal(np.isnan(got), np.isnan(want)), kernel
        assert np.array_equal(np.isposinf(got), np.isposinf(want)), kernel
        assert np.array_equal(np.isneginf(got), np.isneginf(want)), kernel
        err = np.abs(got[finite_rows] - want[finite_rows])
        assert np.all(err <= 1e-4 * bound), kernel


@pytest.mark.parametrize("shape", [(40, 1000, 304), (256, 1000, 16384), (300, 4096, 512),
                                   (100, 6001, 272), (64, 8192, 256), (40, 12000, 64)],
                         ids=lambda s: "x".join(map(str, s)))
def test_exact_split_fused_norm_and_accumulate(shape):
    # A narrow product split across k, and a wide one; then rows the norm
    # pre-pass holds in registers in one, two and four steps of 2048 values
    # (6001: rows that are not 16-byte groups, loaded by scalars), and one
    # past that (12000), which it reads twice.
    m, k, n = shape
    A = inputs.normal((m, k), 1.0, 511)
    w = inputs.uniform((k,), 0.5, 1.5, 512)
    C0 = inputs.normal((m, n), 1.0, 513)
    q, s = orc.quantize_q8(inputs.normal((k, n), 0.02, 514))
    want = orc.matmul_fused(A, Bq=q, scale=s, w=w, C0=C0)
    C = dev(C0)
    em.matmul(dev(A), dev(q), C, scale=dev(s), accumulate=True, rms_weight=dev(w))
    An = orc.rmsnorm(A, w)
    check(host(C), want, An, orc.dequantize(q, s), k, factor=2.0, C0=C0)


@pytest.mark.parametrize("norm", [True, False], ids=["norm", "plain"])
def test_exact_split_last_round_as_two_block_tiles(norm):
    # 512 x 4096 x 12288 with the norm: 384 four-block tiles, whose last
    # round (128 tiles) runs as 256 two-block tiles in a second launch. Each
    # element is summed in the same order either way, so the product equals,
    # bit for bit, its column ranges computed as products of their own
    # (8192 columns: four-block tiles; 4096: two-block), and the f64 product
    # within 1e-4 * sum|a||w|. Without the norm the whole product takes
    # two-block tiles (the same comparison, no second launch).
    m, k, n = 512, 4096, 12288
    A = dev(inputs.normal((m, k), 1.0, 551))
    q, s = em.quantize_q8(dev(inputs.normal((k, n), 0.02, 552)))
    w = dev(inputs.uniform((k,), 0.5, 1.5, 553)) if norm else None
    whole = host(em.matmul(A, q, scale=s, rms_weight=w))
    assert np.array_equal(whole, host(em.matmul(A, q, scale=s, rms_weight=w)))
    for c0, c1 in ((0, 8192), (8192, 12288)):
        part = host(em.matmul(A, q[:, c0:c1].contiguous(), scale=s[c0:c1].contiguous(),
                              rms_weight=w))
        assert np.array_equal(whole[:, c0:c1], part), (c0, c1)
    rows = np.array([0, 63, 64, 255, 300, 511])
    Ah = host(A)[rows]
    An = orc.rmsnorm(Ah, host(w)) if norm else Ah
    Wd = orc.dequantize(host(q), host(s))
    exact = orc.matmul_f64(An, Wd)
    assert np.all(np.abs(whole[rows] - exact) <= 1e-4 * orc.abs_bound(An, Wd))


def test_stream_read_runs_and_checks_alignment():
    # The bench's read-only ceiling: one pass over a buffer, nothing written
    # but (almost never) the sink.
    buf = torch.ones(1 << 20, device="cuda")
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    em.stream_read(buf, sink)
    torch.cuda.synchronize()
    with pytest.raises(em.InvalidArgument):
        em.stream_read(buf[1:5], sink)  # 4-byte offset
