"""em_matmul_q8_noalloc against em_matmul_q8 with the skinny kernel, through
the C ABI: the same bits (integer work on int8 weights summed in the same
fixed order: the two run the same kernels), nothing allocated, and shapes
whose split-K partials pass the static scratch rejected before any launch.
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


def case(m, k, n, seed, acc=False, rms=False):
    A = dev(inputs.normal((m, k), 1.0, seed))
    q, s = em.quantize_q8(dev(inputs.normal((k, n), 0.02, seed + 1)))
    C0 = dev(inputs.normal((m, n), 1.0, seed + 2))
    w = dev(inputs.uniform((k,), 0.5, 1.5, seed + 3)) if rms else None
    return A, q, s, C0, w


def noalloc(A, q, s, C0, w, acc):
    C = C0.clone() if acc else torch.full_like(C0, 7.0)
    em.matmul_q8_noalloc(A, q, C, s, accumulate=acc, rms_weight=w)
    return C


def skinny(A, q, s, C0, w, acc):
    C = C0.clone() if acc else torch.full_like(C0, 7.0)
    em.matmul(A, q, C, scale=s, kernel="skinny", accumulate=acc, rms_weight=w)
    return C


# (m, k, n, accumulate, rms): two calls in a row, the second smaller, each
# with a split k: the Llama-7B classifier at 8 rows (31.25 MiB of
# partials, the most the scratch holds for these shapes), then 4096^2 and
# 11008 x 4096 shapes, and widths that take 4- and 1-column lanes.
PAIRS = [((8, 4096, 32000, False, False), (1, 2048, 1024, False, False)),
         ((8, 4096, 11008, True, True), (2, 1000, 336, True, False)),
         ((3, 11008, 4096, False, True), (1, 4096, 4096, True, True)),
         ((5, 1030, 36, True, False), (1, 300, 7, False, True)),
         ((4, 4096, 4096, False, False), (4, 2048, 4096, True, False))]


@pytest.mark.parametrize("pair", PAIRS, ids=lambda p: "_".join("x".join(map(str, c[:3]))
                                                              for c in p))
def test_same_bits_as_skinny_on_two_calls(pair):
    cases = [case(m, k, n, 900 + 10 * i + m, acc, rms)
             for i, (m, k, n, acc, rms) in enumerate(pair)]
    torch.cuda.synchronize()
    gen = em.scratch_generation()
    got = [host(noalloc(*c[:5], spec[3])) for c, spec in zip(cases, pair)]
    assert em.scratch_generation() == gen  # no library scratch touched
    for (A, q, s, C0, w), spec, g in zip(cases, pair, got):
        want = host(skinny(A, q, s, C0, w, spec[3]))
        assert np.array_equal(g, want), spec
        # and the oracle's bound, as every int8 product here is held to
        m, k, n = spec[:3]
        Ah = host(A)
        An = orc.rmsnorm(Ah, host(w)) if w is not None else Ah
        Bf = orc.dequantize(host(q), host(s))
        exact = orc.matmul_f64(An, Bf) + (host(C0).astype(np.float64) if spec[3] else 0.0)
        bound = orc.abs_bound(An, Bf) + (np.abs(host(C0)) if spec[3] else 0.0)
        assert np.all(np.abs(g - exact) <= 1e-4 * bound), spec


def test_allocates_nothing():
    # Device memory free before and after a run of calls (the library and
    # its kernels loaded and warm first), and the scratch generation still.
    A, q, s, C0, w = case(8, 4096, 11008, 950, rms=True)
    C = torch.empty_like(C0)
    em.matmul(A, q, C, scale=s, kernel="skinny", rms_weight=w)
    em.matmul_q8_noalloc(A, q, C, s, rms_weight=w)
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    gen = em.scratch_generation()
    for _ in range(3):
        em.matmul_q8_noalloc(A, q, C, s, rms_weight=w)
        em.matmul_q8_noalloc(A[:1], q, C[:1], s)
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    assert free1 == free0 and em.scratch_generation() == gen


def test_registered_weights_take_the_strip_path_too():
    A, q, s, C0, w = case(1, 4096, 2048, 960)
    em.register_q8(q)
    try:
        got = host(noalloc(A, q, s, C0, None, False))
        want = host(skinny(A, q, s, C0, None, False))
    finally:
        em.unregister_q8(q)
    assert np.array_equal(got, want)


def test_partials_past_the_static_scratch_are_rejected():
    # m = 8, k = 65536, n = 16384: 512 slices of 8 x 16384 partials (256
    # MiB) against 32 MiB. Real buffers of the full shape, so nothing would
    # read out of bounds even if a kernel ran; C must be left as it was.
    m, k, n = 8, 65536, 16384
    A = torch.zeros((m, k), device="cuda")
    B = torch.zeros((k, n), dtype=torch.int8, device="cuda")
    s = torch.ones((n,), device="cuda")
    C = torch.full((m, n), 3.0, device="cuda")
    with pytest.raises(em.EngineError) as e:
        em.matmul_q8_noalloc(A, B, C, s)
    assert e.value.code == em.EM_EINVAL and "static scratch" in str(e.value)
    assert bool((C == 3.0).all())
    del A, B
    torch.cuda.synchronize()


def test_rejects_what_em_matmul_q8_rejects():
    A = torch.zeros((9, 64), device="cuda")
    B = torch.zeros((64, 32), dtype=torch.int8, device="cuda")
    s = torch.ones((32,), device="cuda")
    C = torch.empty((9, 32), device="cuda")
    with pytest.raises(em.EngineError) as e:
        em.matmul_q8_noalloc(A, B, C, s)
    assert e.value.code == em.EM_EINVAL and "at most 8 rows" in str(e.value)
