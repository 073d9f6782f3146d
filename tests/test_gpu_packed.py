"""GPU parity of the strip layout of int8 weights (em_pack_q8 /
em_matmul_q8_packed) against the CPU oracle.

The layout is an explicit opt-in copy behind the boundary (the reference keeps
QTensor row-major, tensor.h:23-28), so its products are held to the same
contract as em_matmul_q8's skinny path: the reference tests' 1e-5 * k (2k
with fusion, test_cuda.cpp:38-47,126-165) and the north star's
1e-4 * sum_k |a||w| per element, accumulate and rms fusions, k == 0, and
bit-identical repeats (test_cuda.cpp:272).
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


def strips(q):
    """The layout by its definition, written as loops over its indices:
    packed[(j * k + 4 qd) * 16 + 16 c + 4 t + u] = B[4 qd + t, 16 j + 4 c + u]."""
    k, n = q.shape
    out = np.empty(k * n, dtype=q.dtype)
    j, qd, c, t, u = np.meshgrid(np.arange(n // 16), np.arange(k // 4), np.arange(4), np.arange(4),
                                 np.arange(4), indexing="ij")
    out[(j * k + 4 * qd) * 16 + 16 * c + 4 * t + u] = q[4 * qd + t, 16 * j + 4 * c + u]
    return out


def test_strips_reference_is_a_permutation():
    # The definition above, checked on a matrix of distinct values: every
    # byte lands once, and a quad's unit c holds rows 4q..4q+3 of columns
    # 4c..4c+3, row by row.
    k, n = 8, 32
    q = np.arange(k * n, dtype=np.int32).reshape(k, n)
    got = strips(q)
    assert np.array_equal(np.sort(got), np.arange(k * n))
    # strip 1, quad 1, unit 2: rows 4..7 of columns 16 + 8 .. 16 + 11.
    unit = got[(1 * k + 4) * 16 + 32:(1 * k + 4) * 16 + 48].reshape(4, 4)
    assert np.array_equal(unit, q[4:8, 24:28])


@pytest.mark.parametrize("shape", [(4, 16), (12, 32), (288, 864), (20, 4096), (4096, 4096),
                                   (11008, 64)], ids=lambda s: "x".join(map(str, s)))
def test_pack_layout_and_round_trip(shape):
    k, n = shape
    q, _ = orc.quantize_q8(inputs.uniform((k, n), -1.0, 1.0, 5))
    packed = em.pack_q8(dev(q))
    got = host(packed)
    assert np.array_equal(got, strips(q))
    assert np.array_equal(host(em.unpack_q8(packed, k, n)), q)


def test_pack_rejects_k_not_a_multiple_of_4():
    q = torch.zeros((17, 32), dtype=torch.int8, device="cuda")
    with pytest.raises(em.EngineError, match="multiple of 16 and k of 4"):
        em.pack_q8(q)
    A = torch.zeros((1, 17), device="cuda")
    with pytest.raises(em.EngineError, match="multiple of 16 and k of 4"):
        em.matmul_packed(A, torch.zeros((17 * 32,), dtype=torch.int8, device="cuda"), 32,
                         torch.ones((32,), device="cuda"))


# (m, k, n): decode rows 1..8 against the stories15M and Llama-7B-shaped
# projections, a k that needs several 4096-row batches (11008, 8196), k
# below one batch or not a multiple of 256, the deepest one-row pass
# without a norm (12288) and one quad past it, and k past the MFMA
# kernel's 4096 at 2 .. 8 rows (4100, 11008: the VALU kernel).
SHAPES = [(1, 288, 864), (1, 288, 32000), (1, 768, 288), (1, 4096, 4096), (1, 11008, 4096),
          (1, 8196, 64), (1, 12288, 48), (1, 12292, 32), (1, 4, 16), (1, 20, 48),
          (2, 300, 1536), (3, 4096, 272),
          (4, 4100, 32), (5, 516, 2048), (8, 1000, 4096), (8, 11008, 64), (6, 20, 16),
          (7, 4, 160), (2, 4096, 4096), (4, 4096, 11008), (8, 4096, 4096), (5, 288, 32000)]


def check(got, want, A, Bf, k, factor=1.0, C0=None):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    assert err.max() <= 1e-5 * max(k, 1) * factor, f"max err {err.max()} (k={k})"
    bound = orc.abs_bound(A, Bf)
    if C0 is not None:
        bound = bound + np.abs(C0)
    assert np.all(err <= 1e-4 * bound + 1e-30), "1e-4 * sum|a||w| bound exceeded"


@pytest.mark.parametrize("fusion", ["plain", "acc", "rms", "rms_acc"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_packed_against_oracle(shape, fusion):
    m, k, n = shape
    A = inputs.uniform((m, k), -1.0, 1.0, 21)
    q, s = orc.quantize_q8(inputs.normal((k, n), 0.02, 22))
    acc = "acc" in fusion
    rms = "rms" in fusion
    C0 = inputs.uniform((m, n), -1.0, 1.0, 23) if acc else None
    w = inputs.uniform((k,), 0.5, 1.5, 24) if rms else None
    want = orc.matmul_fused(A, Bq=q, scale=s, w=w, C0=C0)
    C = dev(C0) if acc else torch.empty((m, n), device="cuda")
    em.matmul_packed(dev(A), em.pack_q8(dev(q)), n, dev(s), C, accumulate=acc,
                     rms_weight=dev(w) if rms else None)
    An = orc.rmsnorm(A, w) if rms else A
    check(host(C), want, An, orc.dequantize(q, s), k, 2.0 if (acc or rms) else 1.0, C0)


def test_packed_matches_rowmajor_path_and_repeats():
    # Same weights through em_matmul_q8 (row-major, split-K) and the strip
    # layout: within the tolerance of each other, each bit-identical on repeat.
    m, k, n = 1, 4096, 4096
    A = dev(inputs.normal((m, k), 1.0, 31))
    q, s = em.quantize_q8(dev(inputs.normal((k, n), 0.02, 32)))
    packed = em.pack_q8(q)
    outs = []
    for _ in range(3):
        outs.append(host(em.matmul_packed(A, packed, n, s)))
    assert all(np.array_equal(outs[0], o) for o in outs[1:])
    row = host(em.matmul(A, q, scale=s))
    bound = orc.abs_bound(host(A), orc.dequantize(host(q), host(s)))
    assert np.all(np.abs(outs[0].astype(np.float64) - row) <= 1e-4 * bound)


def test_packed_k_zero():
    n = 32
    C = torch.full((2, n), 3.0, device="cuda")
    A = torch.empty((2, 0), device="cuda")
    packed = torch.empty((0,), dtype=torch.int8, device="cuda")
    s = torch.ones((n,), device="cuda")
    em.matmul_packed(A, packed, n, s, C, accumulate=True)
    assert np.all(host(C) == 3.0)
    em.matmul_packed(A, packed, n, s, C)
    assert np.all(host(C) == 0.0)


def test_packed_graph_replay_matches_eager():
    m, k, n = 1, 4096, 1024
    A = dev(inputs.normal((m, k), 1.0, 41))
    q, s = em.quantize_q8(dev(inputs.normal((k, n), 0.02, 42)))
    packed = em.pack_q8(q)
    C = torch.empty((m, n), device="cuda")
    em.matmul_packed(A, packed, n, s, C)
    eager = host(C).copy()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        em.matmul_packed(A, packed, n, s, C)
    for _ in range(3):
        C.zero_()
        torch.cuda.synchronize()
        g.replay()
        assert np.array_equal(host(C), eager)


# ---- registered weights: em_matmul_q8 over the strip copy -------------------

REG_SHAPES = [(288, 864), (4096, 4096), (8192, 64), (11008, 64), (11008, 4096), (768, 288),
              (288, 32000), (20, 48), (4096, 12288), (3000, 8192), (4096, 32000)]


@pytest.mark.parametrize("fusion", ["plain", "rms"])
@pytest.mark.parametrize("shape", [(4096, 4096), (288, 864), (11008, 4096)],
                         ids=lambda s: "x".join(map(str, s)))
def test_registered_one_row_misaligned_a(shape, fusion):
    # A one float past a 16-byte boundary: the one-pass kernel needs 16-byte
    # A, so the call takes the kernel that stages A in LDS (or, past its
    # depth, the row-major path); either way within the oracle's bound, and
    # the same bits on a second call.
    k, n = shape
    A = inputs.uniform((1, k), -1.0, 1.0, 61)
    q, s = orc.quantize_q8(inputs.normal((k, n), 0.02, 62))
    rms = fusion == "rms"
    w = inputs.uniform((k,), 0.5, 1.5, 63) if rms else None
    qd, sd = dev(q), dev(s)
    buf = torch.zeros((k + 1,), device="cuda")
    buf[1:] = dev(A)[0]
    Am = buf[1:].view(1, k)
    assert Am.data_ptr() % 16 == 4
    em.register_q8(qd)
    try:
        wd = dev(w) if rms else None
        C = torch.empty((1, n), device="cuda")
        em.matmul(Am, qd, C, scale=sd, rms_weight=wd)
        got = host(C)
        em.matmul(Am, qd, C, scale=sd, rms_weight=wd)
        assert np.array_equal(got, host(C))
    finally:
        em.unregister_q8(qd)
    want = orc.matmul_fused(A, Bq=q, scale=s, w=w)
    An = orc.rmsnorm(A, w) if rms else A
    check(got, want, An, orc.dequantize(q, s), k, 2.0 if rms else 1.0)


@pytest.mark.parametrize("kernel", ["automatic", "skinny"])
@pytest.mark.parametrize("fusion", ["plain", "acc", "rms", "rms_acc"])
@pytest.mark.parametrize("shape", REG_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_registered_one_row_against_oracle(shape, fusion, kernel):
    k, n = shape
    A = inputs.uniform((1, k), -1.0, 1.0, 51)
    q, s = orc.quantize_q8(inputs.normal((k, n), 0.02, 52))
    acc = "acc" in fusion
    rms = "rms" in fusion
    C0 = inputs.uniform((1, n), -1.0, 1.0, 53) if acc else None
    w = inputs.uniform((k,), 0.5, 1.5, 54) if rms else None
    qd, sd = dev(q), dev(s)
    em.register_q8(qd)
    try:
        assert em.registered_q8(qd)
        C = dev(C0) if acc else torch.empty((1, n), device="cuda")
        wd = dev(w) if rms else None
        em.matmul(dev(A), qd, C, scale=sd, kernel=kernel, accumulate=acc, rms_weight=wd)
        got = host(C)
        # Where the registered call takes the strip copy (k <= 8192, or
        # 12288 without a norm and with n >= 4096), it is the strip-layout
        # product, bit for bit; otherwise it is the row-major call.
        if k <= 8192 or (not rms and k <= 12288 and n >= 4096):
            P = em.pack_q8(qd)
            C2 = dev(C0) if acc else torch.empty((1, n), device="cuda")
            em.matmul_packed(dev(A), P, n, sd, C2, accumulate=acc, rms_weight=wd)
            assert np.array_equal(got, host(C2))
    finally:
        em.unregister_q8(qd)
    assert not em.registered_q8(qd)
    want = orc.matmul_fused(A, Bq=q, scale=s, w=w, C0=C0)
    An = orc.rmsnorm(A, w) if rms else A
    check(got, want, An, orc.dequantize(q, s), k, 2.0 if (acc or rms) else 1.0, C0)


@pytest.mark.parametrize("fusion", ["plain", "acc", "rms", "rms_acc"])
@pytest.mark.parametrize("shape", [(2, 288, 864), (4, 4096, 4096), (8, 4096, 11008), (3, 768, 288),
                                   (6, 4096, 32000), (7, 20, 48), (5, 11008, 64), (8, 4096, 4096),
                                   (4, 4096, 32000), (2, 1000, 2048)],
                         ids=lambda s: "x".join(map(str, s)))
def test_registered_decode_rows_against_oracle(shape, fusion):
    # 2 .. 8 rows with automatic over registered weights: the MFMA kernel
    # over the strip copy where it takes the shape (k <= 4096; 3 .. 4 rows up
    # to n = 24576, 5 .. 8 up to 4096), the row-major kernels otherwise;
    # bit-identical on repeat, and the same bits as em_matmul_q8_packed where
    # both run the MFMA kernel.
    m, k, n = shape
    A = inputs.uniform((m, k), -1.0, 1.0, 56)
    q, s = orc.quantize_q8(inputs.normal((k, n), 0.02, 57))
    acc = "acc" in fusion
    rms = "rms" in fusion
    C0 = inputs.uniform((m, n), -1.0, 1.0, 58) if acc else None
    w = inputs.uniform((k,), 0.5, 1.5, 59) if rms else None
    qd, sd = dev(q), dev(s)
    wd = dev(w) if rms else None
    em.register_q8(qd)
    try:
        outs = []
        for _ in range(2):
            C = dev(C0) if acc else torch.empty((m, n), device="cuda")
            em.matmul(dev(A), qd, C, scale=sd, accumulate=acc, rms_weight=wd)
            outs.append(host(C))
        assert np.array_equal(outs[0], outs[1])
        if k <= 4096 and (m <= 2 or (m <= 4 and n <= 24576) or n <= 4096):
            # Both entry points run the MFMA kernel here.
            C2 = dev(C0) if acc else torch.empty((m, n), device="cuda")
            em.matmul_packed(dev(A), em.pack_q8(qd), n, sd, C2, accumulate=acc, rms_weight=wd)
            assert np.array_equal(outs[0], host(C2))
    finally:
        em.unregister_q8(qd)
    want = orc.matmul_fused(A, Bq=q, scale=s, w=w, C0=C0)
    An = orc.rmsnorm(A, w) if rms else A
    check(outs[0], want, An, orc.dequantize(q, s), k, 2.0 if (acc or rms) else 1.0, C0)


def test_registered_weights_leave_other_calls_row_major():
    # Explicit kernels (12 rows through tiled_split among them), k past the
    # strip cut and an unregistered B all run the row-major kernels: the same
    # bits as before registering. One row and (automatic) 2 .. 8 rows run
    # over the strip copy: the same bits as em_matmul_q8_packed, within the
    # tolerance of the row-major path (automatic 9 .. 64 rows over the copy:
    # test_gpu_strip_split.py).
    k, n = 4096, 512
    q, s = em.quantize_q8(dev(inputs.normal((k, n), 0.02, 61)))
    A1 = dev(inputs.normal((1, k), 1.0, 62))
    A4 = dev(inputs.normal((4, k), 1.0, 63))
    A12 = dev(inputs.normal((12, k), 1.0, 66))
    same = (("m4 skinny", A4, "skinny"), ("m12 tiled_split", A12, "tiled_split"), ("tiled", A1, "tiled"),
            ("naive", A1, "naive"))
    before = {name: host(em.matmul(A, q, scale=s, kernel=kern)).copy() for name, A, kern in same}
    row = {m: host(em.matmul(A, q, scale=s)).copy() for m, A in ((1, A1), (4, A4))}
    em.register_q8(q)
    try:
        for name, A, kern in same:
            assert np.array_equal(host(em.matmul(A, q, scale=s, kernel=kern)), before[name])
        reg = {m: host(em.matmul(A, q, scale=s)).copy() for m, A in ((1, A1), (4, A4))}
        P = em.pack_q8(q)
        for m, A in ((1, A1), (4, A4)):
            assert np.array_equal(reg[m], host(em.matmul_packed(A, P, n, s)))
    finally:
        em.unregister_q8(q)
    for m, A in ((1, A1), (4, A4)):
        assert np.array_equal(host(em.matmul(A, q, scale=s)), row[m])
        bound = orc.abs_bound(host(A), orc.dequantize(host(q), host(s)))
        assert np.all(np.abs(reg[m].astype(np.float64) - row[m]) <= 1e-4 * bound)
    # k = 8193: past the strip cut, registered or not the row-major path.
    q2, s2 = em.quantize_q8(dev(inputs.normal((8193, 64), 0.02, 64)))
    A2 = dev(inputs.normal((1, 8193), 1.0, 65))
    want = host(em.matmul(A2, q2, scale=s2)).copy()
    em.register_q8(q2)
    try:
        assert np.array_equal(host(em.matmul(A2, q2, scale=s2)), want)
    finally:
        em.unregister_q8(q2)


def test_register_again_after_the_bytes_change():
    k, n = 1024, 256
    qa, s = em.quantize_q8(dev(inputs.normal((k, n), 0.02, 71)))
    qb, _ = em.quantize_q8(dev(inputs.normal((k, n), 0.02, 72)))
    A = dev(inputs.normal((1, k), 1.0, 73))
    q = qa.clone()
    em.register_q8(q)
    try:
        first = host(em.matmul(A, q, scale=s)).copy()
        q.copy_(qb)
        em.register_q8(q)  # repacks from the new bytes
        second = host(em.matmul(A, q, scale=s)).copy()
    finally:
        em.unregister_q8(q)
    assert np.array_equal(first, host(em.matmul_packed(A, em.pack_q8(qa), n, s)))
    assert np.array_equal(second, host(em.matmul_packed(A, em.pack_q8(qb), n, s)))


def test_registered_graph_replay_matches_eager():
    k, n = 4096, 2048
    q, s = em.quantize_q8(dev(inputs.normal((k, n), 0.02, 81)))
    A = dev(inputs.normal((1, k), 1.0, 82))
    em.register_q8(q)
    try:
        C = torch.empty((1, n), device="cuda")
        em.matmul(A, q, C, scale=s)
        eager = host(C).copy()
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            em.matmul(A, q, C, scale=s)
        for _ in range(3):
            C.zero_()
            torch.cuda.synchronize()
            g.replay()
            assert np.array_equal(host(C), eager)
        del g
        torch.cuda.synchronize()
    finally:
        em.unregister_q8(q)


def _q8_product_raw(B_ptr, A, s, k, n):
    C = torch.empty((A.shape[0], n), device="cuda")
    em.matmul_q8_raw(A.shape[0], n, k, A.data_ptr(), B_ptr, s.data_ptr(), C.data_ptr())
    return host(C)


def test_em_free_drops_the_registration():
    # A registered buffer freed with em_free takes its strip copy with it:
    # a new allocation at the same address, holding other bytes, must not be
    # multiplied by the stale copy (the reference's DeviceQTensor owns and
    # frees its bytes, cuda_matmul.cu:488-513, so it has no copy to go stale).
    import ctypes
    L = em.lib()
    k, n = 1024, 256
    qa, s = orc.quantize_q8(inputs.normal((k, n), 0.02, 301))
    qb, _ = orc.quantize_q8(inputs.normal((k, n), 0.02, 302))
    A = dev(inputs.normal((1, k), 1.0, 303))
    sd = dev(s)
    p1 = ctypes.c_void_p()
    assert L.em_malloc(ctypes.byref(p1), k * n) == em.EM_OK
    assert L.em_memcpy_h2d(p1, qa.ctypes.data, k * n) == em.EM_OK
    assert L.em_q8_register(p1, k, n, None) == em.EM_OK
    assert L.em_q8_registered(p1, k, n) == 1
    first = _q8_product_raw(p1.value, A, sd, k, n)
    assert L.em_free(p1) == em.EM_OK
    assert L.em_q8_registered(p1, k, n) == 0
    # Allocate until one buffer lands on the freed address (the allocator
    # need not hand it back at once); multiply by the first that does.
    held = []
    try:
        for _ in range(16):
            p2 = ctypes.c_void_p()
            assert L.em_malloc(ctypes.byref(p2), k * n) == em.EM_OK
            held.append(p2)
            if p2.value == p1.value:
                break
        p2 = held[-1]
        assert L.em_memcpy_h2d(p2, qb.ctypes.data, k * n) == em.EM_OK
        got = _q8_product_raw(p2.value, A, sd, k, n)
        check(got, orc.matmul_fused(host(A), Bq=qb, scale=s), host(A), orc.dequantize(qb, s), k)
        check(first, orc.matmul_fused(host(A), Bq=qa, scale=s), host(A), orc.dequantize(qa, s), k)
        if p2.value != p1.value:
            pytest.skip("no allocation got the freed address back; the copy was dropped anyway")
    finally:
        for p in held:
            L.em_free(p)


def test_python_registration_ends_with_its_tensor():
    # register_q8 ties the registration to the tensor: once it is collected,
    # torch's caching allocator may hand the same address to new bytes, which
    # must be multiplied as they are.
    import gc
    k, n = 2048, 512
    qa, s = orc.quantize_q8(inputs.normal((k, n), 0.02, 311))
    qb, _ = orc.quantize_q8(inputs.normal((k, n), 0.02, 312))
    A = dev(inputs.normal((1, k), 1.0, 313))
    sd = dev(s)
    q = dev(qa)
    addr = q.data_ptr()
    em.register_q8(q)
    assert em.registered_q8(q)
    del q
    gc.collect()
    torch.cuda.synchronize()
    q2 = dev(qb)
    assert not em.registered_q8(q2)
    got = host(em.matmul(A, q2, scale=sd))
    check(got, orc.matmul_fused(host(A), Bq=qb, scale=s), host(A), orc.dequantize(qb, s), k)
    if q2.data_ptr() != addr:
        pytest.skip("the caching allocator gave another address; the registration ended anyway")


@pytest.mark.parametrize("m", [1, 12, 64, 200])
@pytest.mark.parametrize("shape", [(4096, 4096), (288, 864)], ids=lambda s: "x".join(map(str, s)))
def test_registered_misaligned_norm_weight(shape, m):
    # The norm weight one float past a 16-byte boundary (the reference's
    # MatmulFusion.rms_weight may be any device float pointer,
    # cuda_matmul.h:85-92): the kernels that load it four floats at a time
    # are passed over for ones that load it per value (the one-row strip
    # kernel; at 64 and 200 rows the exact split's pre-pass); within the
    # oracle's bound, the same bits on a second call.
    k, n = shape
    A = inputs.uniform((m, k), -1.0, 1.0, 321)
    q, s = orc.quantize_q8(inputs.normal((k, n), 0.02, 322))
    w = inputs.uniform((k,), 0.5, 1.5, 323)
    qd, sd = dev(q), dev(s)
    wbuf = torch.zeros((k + 1,), device="cuda")
    wbuf[1:] = dev(w)
    wm = wbuf[1:]
    assert wm.data_ptr() % 16 == 4
    em.register_q8(qd)
    try:
        C = torch.empty((m, n), device="cuda")
        em.matmul(dev(A), qd, C, scale=sd, rms_weight=wm)
        got = host(C).copy()
        em.matmul(dev(A), qd, C, scale=sd, rms_weight=wm)
        assert np.array_equal(got, host(C))
    finally:
        em.unregister_q8(qd)
    want = orc.matmul_fused(A, Bq=q, scale=s, w=w)
    check(got, want, orc.rmsnorm(A, w), orc.dequantize(q, s), k, 2.0)


@pytest.mark.parametrize("fusion", ["plain", "acc", "rms", "rms_acc"])
@pytest.mark.parametrize("shape", [(4096, 12288), (3000, 8192), (288, 32000), (4096, 4112),
                                   (1024, 16384)], ids=lambda s: "x".join(map(str, s)))
def test_registered_wide_rows_match_narrow_bit_for_bit(shape, fusion):
    # Past one strip per CU the strip kernel's grid runs in rounds; a
    # strip's sums do not depend on its round or on the other strips. So
    # columns [c0, c0 + 4096) of the wide product equal, bit for bit, the
    # product of those 4096 columns registered on their own (256 strips, one
    # round): checked at the first, a middle and the last block of columns,
    # and against the oracle.
    k, n = shape
    A = inputs.uniform((1, k), -1.0, 1.0, 61)
    q, s = orc.quantize_q8(inputs.normal((k, n), 0.02, 62))
    acc = "acc" in fusion
    rms = "rms" in fusion
    C0 = inputs.uniform((1, n), -1.0, 1.0, 63) if acc else None
    w = inputs.uniform((k,), 0.5, 1.5, 64) if rms else None
    dA, wd = dev(A), (dev(w) if rms else None)
    qd, sd = dev(q), dev(s)
    em.register_q8(qd)
    try:
        C = dev(C0) if acc else torch.empty((1, n), device="cuda")
        em.matmul(dA, qd, C, scale=sd, accumulate=acc, rms_weight=wd)
        wide = host(C)
        C2 = dev(C0) if acc else torch.empty((1, n), device="cuda")
        em.matmul(dA, qd, C2, scale=sd, accumulate=acc, rms_weight=wd)
        assert np.array_equal(wide, host(C2)), "repeat not bit-identical"
    finally:
        em.unregister_q8(qd)
    for c0 in sorted({0, (n // 2 - 2048) // 16 * 16, n - 4096}):
        qn = dev(np.ascontiguousarray(q[:, c0:c0 + 4096]))
        sn = dev(np.ascontiguousarray(s[c0:c0 + 4096]))
        em.register_q8(qn)
        try:
            Cn = dev(np.ascontiguousarray(C0[:, c0:c0 + 4096])) if acc else \
                torch.empty((1, 4096), device="cuda")
            em.matmul(dA, qn, Cn, scale=sn, accumulate=acc, rms_weight=wd)
            narrow = host(Cn)
        finally:
            em.unregister_q8(qn)
        assert np.array_equal(wide[:, c0:c0 + 4096], narrow), f"columns from {c0}"
    want = orc.matmul_fused(A, Bq=q, scale=s, w=w, C0=C0)
    An = orc.rmsnorm(A, w) if rms else A
    check(wide, want, An, orc.dequantize(q, s), k, 2.0 if (acc or rms) else 1.0, C0)
