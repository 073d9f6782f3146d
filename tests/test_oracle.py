"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

Each oracle function is checked against (a) the reference's own outputs
(golden fixtures written by tests/golden/make_golden.py from oracle/_ref, and
the live oracle/_ref where it is built), (b) the known-answer tests of the
reference's test files, and (c) what the mathematics fixes. The "planted"
tests put a plausible mistake into a copy of the oracle's result, on the
CPU, and show that the same check rejects it.
"""
import hashlib
import json
import os

import numpy as np
import pytest

import oracle
from tests import inputs

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def orc():
    return oracle.oracle()


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def golden_quant_small():
    z = np.load(os.path.join(GOLDEN, "quant_small.npz"))
    names = sorted({k.split("__")[0] for k in z.files})
    out = {}
    for name in names:
        if f"{name}__B" in z.files:
            B = z[f"{name}__B"]
        else:
            seed = int(z[f"{name}__seed"])
            shape = z[f"{name}__q"].shape
            B = (inputs.uniform(shape, -1.0, 1.0, seed) if name.startswith("u_")
                 else inputs.normal(shape, 0.02, seed))
            assert sha(B) == z[f"{name}__shaB"].item().decode(), f"{name}: input drifted"
        out[name] = (B, z[f"{name}__q"], z[f"{name}__scale"])
    return out


# ---------------------------------------------------------------- quantize_q8

def test_quant_matches_reference_fixtures_bit_exact(orc):
    for name, (B, q_ref, s_ref) in golden_quant_small().items():
        q, s = orc.quantize_q8(B)
        assert np.array_equal(q, q_ref), name
        assert np.array_equal(s.view(np.uint32), s_ref.view(np.uint32)), name


def test_quant_ties_round_half_away_from_zero(orc):
    # scale 1 (absmax 127) so q = lround(B): 0.5 -> 1, -0.5 -> -1, 2.5 -> 3, 126.5 -> 127.
    col = np.array([127.0, 0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 126.5, -126.5, 63.5], np.float32)
    q, s = orc.quantize_q8(col[:, None])
    assert s[0] == np.float32(1.0)
    assert q[:, 0].tolist() == [127, 1, -1, 2, -2, 3, -3, 127, -127, 64]


def test_quant_invariants_of_reference_test(orc):
    # tests/test_quant.cpp:33-51: zero column -> scale 0 and q 0, max|q| = 127
    # elsewhere, |dequantize - B| <= scale / 2 * (1 + 1e-5).
    B = golden_quant_small()["round_trip_37x21"][0]
    q, s = orc.quantize_q8(B)
    d = orc.dequantize(q, s)
    assert s[4] == 0.0 and not q[:, 4].any()
    for c in range(B.shape[1]):
        assert np.abs(q[:, c].astype(int)).max() == (0 if c == 4 else 127)
        assert np.all(np.abs(d[:, c] - B[:, c]) <= s[c] * 0.5 * (1 + 1e-5))


def test_quant_closed_form_float32(orc):
    # The closed form in float32 arithmetic, with a half-away-from-zero round
    # written independently of the C code.
    B = inputs.normal((300, 77), 0.02, 5)
    B[:, 3] = 0.0
    q, s = orc.quantize_q8(B)
    absmax = np.abs(B).max(axis=0)
    scale = (absmax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(scale > 0, np.float32(1.0) / scale, np.float32(0.0)).astype(np.float32)
    x = (B * inv).astype(np.float32)
    r = np.trunc(x) + np.where(np.abs(x - np.trunc(x)) >= 0.5, np.sign(x), 0)
    want = np.clip(r, -127, 127).astype(np.int8)
    assert np.array_equal(s, scale)
    assert np.array_equal(q, want)


def test_quant_digest_small_config_shape(orc):
    # The config-4 wqkv shape (288 x 864) against the reference's digest.
    d = json.load(open(os.path.join(GOLDEN, "quant_digests.json")))["s15m_wqkv_288x864"]
    B = inputs.normal(tuple(d["shape"]), d["std"], d["seed"])
    assert sha(B) == d["B"]
    q, s = orc.quantize_q8(B)
    assert sha(q) == d["q"] and sha(s) == d["scale"]


@pytest.mark.parametrize("name", ["w_4096x4096", "s15m_cls_288x32000"])
def test_quant_digest_config_shapes(orc, name):
    d = json.load(open(os.path.join(GOLDEN, "quant_digests.json")))[name]
    B = inputs.normal(tuple(d["shape"]), d["std"], d["seed"])
    assert sha(B) == d["B"], "input generator drifted"
    q, s = orc.quantize_q8(B)
    assert sha(q) == d["q"]
    assert sha(s) == d["scale"]


def test_planted_round_half_even_is_caught():
    # numpy's rint rounds half to even: the ties fixture must reject it.
    B, q_ref, _ = golden_quant_small()["ties_10x4"]
    absmax = np.abs(B).max(axis=0)
    scale = (absmax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(scale > 0, np.float32(1.0) / scale, 0).astype(np.float32)
    wrong = np.clip(np.rint(B * inv), -127, 127).astype(np.int8)
    assert not np.array_equal(wrong, q_ref)


# ---------------------------------------------------------------- matmul_naive

def test_known_answer(orc):
    # tests/test_matmul.cpp:40-52.
    A = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    B = np.array([[7, 8], [9, 10], [11, 12]], np.float32)
    assert orc.matmul_naive(A, B).tolist() == [[58, 64], [139, 154]]


def test_planted_transpose_fails_known_answer(orc):
    A = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    B = np.array([[7, 8], [9, 10], [11, 12]], np.float32)
    wrong = orc.matmul_naive(A, B).T  # a transposed result
    assert wrong.tolist() != [[58, 64], [139, 154]]


def test_naive_exact_on_small_integers(orc):
    # Products and sums of small integers are exact in fp32: every summation
    # order gives the same bits, so the oracle must equal the f64 product.
    rng = np.random.default_rng(0)
    A = rng.integers(-8, 9, (13, 37)).astype(np.float32)
    B = rng.integers(-8, 9, (37, 29)).astype(np.float32)
    assert np.array_equal(orc.matmul_naive(A, B).astype(np.float64), orc.matmul_f64(A, B))


def test_naive_linearity(orc):
    A1 = inputs.uniform((5, 40), -1, 1, 1)
    A2 = inputs.uniform((5, 40), -1, 1, 2)
    B = inputs.uniform((40, 9), -1, 1, 3)
    lhs = orc.matmul_naive(A1 + A2, B)
    rhs = orc.matmul_naive(A1, B) + orc.matmul_naive(A2, B)
    assert np.abs(lhs - rhs).max() <= 1e-5 * 40


def test_naive_matches_reference_fixtures(orc):
    z = np.load(os.path.join(GOLDEN, "matmul_small.npz"))
    keys = sorted({k.split("__")[0] for k in z.files})
    assert len(keys) == 17
    for key in keys:
        m, k, n = map(int, key.split("x"))
        A = inputs.uniform((m, k), -1.0, 1.0, int(z[f"{key}__seedA"]))
        B = inputs.uniform((k, n), -1.0, 1.0, int(z[f"{key}__seedB"]))
        assert sha(A) == z[f"{key}__shaA"].item().decode()
        assert sha(B) == z[f"{key}__shaB"].item().decode()
        got = orc.matmul_naive(A, B)
        tol = 1e-5 * max(k, 1)  # tests/test_matmul.cpp:77-84
        assert np.abs(got - z[f"{key}__naive"]).max(initial=0) <= tol, key
        assert np.abs(got - z[f"{key}__parallel"]).max(initial=0) <= tol, key
        if k == 0:
            assert not got.any()


def test_q8_product_matches_reference_parallel(orc):
    # int8 path: matmul_parallel(A, Bq) == naive(A, dequantize(Bq)) within
    # 1e-5 k (tests/test_quant.cpp:57-79), on the fixture shapes.
    z = np.load(os.path.join(GOLDEN, "matmul_small.npz"))
    keys = sorted({k.split("__")[0] for k in z.files})
    for key in keys:
        m, k, n = map(int, key.split("x"))
        A = inputs.uniform((m, k), -1.0, 1.0, int(z[f"{key}__seedA"]))
        src = inputs.uniform((k, n), -0.5, 0.5, int(z[f"{key}__seedQ"]))
        q, s = orc.quantize_q8(src)
        got = orc.matmul_fused(A, Bq=q, scale=s)
        assert np.abs(got - z[f"{key}__parallel_q8"]).max(initial=0) <= 1e-5 * max(k, 1), key


def test_planted_missing_scale_is_caught(orc):
    z = np.load(os.path.join(GOLDEN, "matmul_small.npz"))
    key = "5x200x300"
    A = inputs.uniform((5, 200), -1.0, 1.0, int(z[f"{key}__seedA"]))
    src = inputs.uniform((200, 300), -0.5, 0.5, int(z[f"{key}__seedQ"]))
    q, s = orc.quantize_q8(src)
    wrong = orc.matmul_naive(A, q.astype(np.float32))  # scale dropped
    assert np.abs(wrong - z[f"{key}__parallel_q8"]).max() > 1e-5 * 200


# ---------------------------------------------------------------- rmsnorm

def test_rmsnorm_known_values(orc):
    # tests/test_ops.cpp:30-50.
    x = np.array([[3, 4], [0, 0]], np.float32)
    y = orc.rmsnorm(x, np.array([1, 2], np.float32), 0.0)
    s = np.float32(1) / np.sqrt(np.float32(12.5))
    assert abs(y[0, 0] - 3 * s) <= 1e-5 and abs(y[0, 1] - 4 * s * 2) <= 1e-5
    z = orc.rmsnorm(x, np.array([1, 1], np.float32))
    assert z[1, 0] == 0 and z[1, 1] == 0
    u = orc.rmsnorm(np.array([[-2, 0.5, 7, 1, -3]], np.float32), np.ones(5, np.float32), 0.0)
    assert abs(float((u.astype(np.float64) ** 2).mean()) - 1.0) <= 1e-5


def test_rmsnorm_matches_reference_fixture(orc):
    z = np.load(os.path.join(GOLDEN, "rmsnorm.npz"))
    y = orc.rmsnorm(z["x"], z["w"])
    assert np.abs(y - z["y"]).max() <= 1e-6
    assert np.abs(orc.rmsnorm(z["x"][:3], z["w"], 0.0) - z["y_eps0"]).max() <= 1e-6


def test_fused_composition(orc):
    # C0 + rmsnorm(A, w) x B from parts (test_cuda.cpp:145-151).
    A = inputs.uniform((3, 100), -1, 1, 31)
    B = inputs.uniform((100, 70), -1, 1, 32)
    C0 = inputs.uniform((3, 70), -1, 1, 33)
    w = inputs.uniform((100,), -1, 1, 34)
    want = C0 + orc.matmul_naive(orc.rmsnorm(A, w), B)
    got = orc.matmul_fused(A, B=B, w=w, C0=C0)
    assert np.abs(got - want).max() <= 1e-6


# ---------------------------------------------------------------- tolerance helpers

def test_abs_bound_and_f64_product(orc):
    # For non-negative operands sum|a||b| is the product itself; flipping signs
    # leaves the bound unchanged and never lets |A B| exceed it.
    P = inputs.uniform((6, 50), 0.0, 1.0, 61)
    Q = inputs.uniform((50, 9), 0.0, 1.0, 62)
    exact = orc.matmul_f64(P, Q)
    assert np.allclose(orc.abs_bound(P, Q), exact, rtol=1e-12, atol=0)
    signs = np.where(inputs.uniform((6, 50), -1, 1, 63) < 0, -1, 1).astype(np.float32)
    Ps = P * signs
    assert np.array_equal(orc.abs_bound(Ps, Q), orc.abs_bound(P, Q))
    assert np.all(np.abs(orc.matmul_f64(Ps, Q)) <= orc.abs_bound(Ps, Q) * (1 + 1e-12))
    # the f64 product against a closed form: a rank-one product of ramps.
    a = np.arange(1, 8, dtype=np.float32)[:, None]
    b = np.arange(1, 5, dtype=np.float32)[None, :]
    assert np.array_equal(orc.matmul_f64(a, b), (a.astype(np.float64) @ b.astype(np.float64)))


def test_argmax_first_max_wins(orc):
    # sampler.cpp:28-29: std::max_element returns the first maximum.
    assert orc.argmax(np.array([1, 5, 3, 5, 2], np.float32)) == 1
    assert orc.argmax(np.array([7], np.float32)) == 0
    assert orc.argmax(np.array([-3, -1, -1, -2], np.float32)) == 1


# ---------------------------------------------------------------- live reference

ref = oracle.ref()
needs_ref = pytest.mark.skipif(ref is None, reason="oracle/_ref not built on this machine")


@needs_ref
def test_live_reference_quant_agrees(orc):
    for seed, shape in [(91, (17, 5)), (92, (128, 300)), (93, (1, 64))]:
        B = inputs.normal(shape, 0.02, seed)
        q, s = orc.quantize_q8(B)
        q2, s2 = ref.quantize_q8(B)
        assert np.array_equal(q, q2) and np.array_equal(s, s2)


@needs_ref
def test_live_reference_shape_error_names_both_shapes():
    msg = ref.shape_error(2, 3, 4, 2)
    assert "2x3" in msg and "4x2" in msg


# ---------------------------------------------------------------- attention

def test_attention_known_answer(orc):
    # head_size 4: scores 0 and (q . k1) / sqrt(4) = 2 / 2 = 1, so the
    # weights are 1 / (1 + e) and e / (1 + e) (cuda_attention.h:28-31).
    q = np.array([[1, 0, 0, 0]], np.float32)
    kc = np.array([[0, 0, 0, 0], [2, 0, 0, 0]], np.float32)
    vc = np.array([[1, 0, 0, 0], [0, 1, 0, 0]], np.float32)
    e = np.e
    got = orc.attention(1, 1, 4, rows=1, pos=1, q=q, kc=kc, vc=vc)
    assert np.allclose(got, [[1 / (1 + e), e / (1 + e), 0, 0]], rtol=0, atol=1e-15)


def test_attention_one_position_returns_its_value(orc):
    heads, kv_heads, hs = 4, 2, 8
    q = inputs.normal((1, heads * hs), 3.0, 301)
    kc = inputs.normal((5, kv_heads * hs), 3.0, 302)
    vc = inputs.normal((5, kv_heads * hs), 1.0, 303)
    got = orc.attention(heads, kv_heads, hs, rows=1, pos=0, q=q, kc=kc, vc=vc)
    for h in range(heads):
        kvh = h // (heads // kv_heads)
        assert np.array_equal(got[0, h * hs:(h + 1) * hs],
                              vc[0, kvh * hs:(kvh + 1) * hs].astype(np.float64))


def test_attention_equal_keys_give_the_mean(orc):
    hs, n = 16, 7
    q = inputs.normal((1, hs), 1.0, 311)
    kc = np.tile(inputs.normal((1, hs), 1.0, 312), (n, 1))
    vc = inputs.normal((n, hs), 1.0, 313)
    got = orc.attention(1, 1, hs, rows=1, pos=n - 1, q=q, kc=kc, vc=vc)
    assert np.allclose(got[0], vc.astype(np.float64).mean(axis=0), rtol=0, atol=1e-12)


def test_attention_head_mapping_and_causal_rows(orc):
    # kv head j holds the constant value j + 1 and zero keys, so query head h
    # must return h // (heads / kv_heads) + 1; reading kv head h % kv_heads
    # (a plausible mistake) gives other constants. Row i of a 3-row call at
    # pos 2 attends to positions [0, 2 + i]: giving position t the value t in
    # kv head 0 makes the row's output the mean 0..2+i.
    heads, kv_heads, hs, T = 8, 2, 4, 6
    vc = np.zeros((T, kv_heads * hs), np.float32)
    for j in range(kv_heads):
        vc[:, j * hs:(j + 1) * hs] = j + 1
    kc = np.zeros_like(vc)
    q = inputs.normal((1, heads * hs), 1.0, 321)
    got = orc.attention(heads, kv_heads, hs, rows=1, pos=T - 1, q=q, kc=kc, vc=vc)
    for h in range(heads):
        assert np.all(got[0, h * hs:(h + 1) * hs] == h // (heads // kv_heads) + 1)
    vc2 = np.repeat(np.arange(T, dtype=np.float32)[:, None], kv_heads * hs, axis=1)
    q3 = inputs.normal((3, heads * hs), 1.0, 322)
    got = orc.attention(heads, kv_heads, hs, rows=3, pos=2, q=q3, kc=kc, vc=vc2)
    for i in range(3):
        assert np.allclose(got[i], np.mean(np.arange(3 + i)), rtol=0, atol=1e-12)


# ------------------------------------------------ forward pass: loader layout

needs_ref_model = pytest.mark.skipif(oracle.ref_model_lib() is None,
                                     reason="oracle/_ref/libref_model.so not built")


@needs_ref_model
@pytest.mark.parametrize("heads,kv_heads,shared", [(4, 4, True), (4, 2, False), (4, 1, True)])
def test_model_layout_matches_reference_loader(heads, kv_heads, shared, tmp_path):
    # tests/e2e_model.model_layout restates load_checkpoint's transposes and
    # concatenations (model.cpp:127-163); the reference's own loader must give
    # the same arrays bit for bit.
    from tests import e2e_model
    m = e2e_model.fixture_model(heads, kv_heads, shared, seed=heads * 10 + kv_heads)
    path = str(tmp_path / "m.bin")
    e2e_model.write_raw(path, m)
    ck = oracle.RefCheckpoint(oracle.ref_model_lib(), path)
    cfg, w = e2e_model.model_layout(m)
    assert ck.config == cfg
    rw = ck.weights()
    for k in ("token_embedding", "rms_final", "wcls"):
        assert np.array_equal(rw[k], w[k]), k
    for l in range(cfg["n_layers"]):
        for k, v in w["layers"][l].items():
            assert np.array_equal(rw["layers"][l][k], v), (l, k)
