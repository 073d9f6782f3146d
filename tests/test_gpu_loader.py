"""em_model_load on the GPU against the reference's own loader
(load_checkpoint, model.cpp:115-163, compiled from source in oracle/_ref):
every array the model holds equals the reference's array bit for bit (fp32),
or quantize_q8 of it bit for bit (int8 bytes and scales); and a loaded model
gives the same logits, bit for bit, as one created from the reference's
arrays (em_model_create), through prefill and decode."""
import numpy as np
import pytest

import oracle
from tests import e2e_model, engine

pytestmark = pytest.mark.gpu

em = engine.load()
orc = oracle.oracle()
lib = oracle.ref_model_lib()
if lib is None:
    pytest.skip("oracle/_ref/libref_model.so not built (make -C oracle ref)",
                allow_module_level=True)

PROJ = ("wqkv", "wo", "w13", "w2")


def write(tmp_path, heads, kv_heads, shared, **kw):
    m = e2e_model.fixture_model(heads, kv_heads, shared, seed=heads * 10 + kv_heads, **kw)
    path = str(tmp_path / "model.bin")
    e2e_model.write_raw(path, m)
    return path


def check_arrays(model, ck, q8):
    w = ck.weights()
    exact = lambda a, b, what: (a.shape == b.shape and np.array_equal(a, b)) or \
        pytest.fail(f"{what} differs")  # noqa: E731
    exact(model.weight("token_embedding"), w["token_embedding"], "token_embedding")
    exact(model.weight("rms_final"), w["rms_final"], "rms_final")
    layers = [("wcls", None, w["wcls"])] + [(k, l, lw[k]) for l, lw in enumerate(w["layers"])
                                             for k in ("rms_att", "rms_ffn") + PROJ]
    for name, layer, want in layers:
        got = model.weight(name, layer or 0)
        if q8 and name in PROJ + ("wcls",):
            q, s = orc.quantize_q8(want)
            exact(got, q, f"{name}[{layer}] int8")
            exact(model.weight(name + ".scale", layer or 0), s, f"{name}[{layer}] scale")
        else:
            exact(got, want, f"{name}[{layer}]")


@pytest.mark.parametrize("wtype", ["f32", "q8"])
@pytest.mark.parametrize("heads,kv_heads,shared", [(4, 4, True), (4, 2, False), (4, 1, True)],
                         ids=["mha_tied", "gqa_untied", "mqa_tied"])
def test_load_matches_reference_loader(tmp_path, heads, kv_heads, shared, wtype):
    path = write(tmp_path, heads, kv_heads, shared)
    q8 = wtype == "q8"
    ck = oracle.RefCheckpoint(lib, path)
    loaded = em.Model.load(path, q8=q8)
    assert loaded.config == ck.config
    check_arrays(loaded, ck, q8)
    created = em.Model(ck.config, ck.weights(), q8=q8)
    T, V = ck.config["seq_len"], ck.config["vocab_size"]
    tokens = [(p * 5 + 1) % V for p in range(T)]
    assert np.array_equal(loaded.forward(tokens[:3], 0), created.forward(tokens[:3], 0))
    for pos in range(3, T):
        assert np.array_equal(loaded.forward(tokens[pos], pos), created.forward(tokens[pos], pos))
    loaded.close()
    created.close()


@pytest.mark.parametrize("shared", [True, False], ids=["tied", "untied"])
def test_stories15m_shape(tmp_path, shared):
    # The stories15M shape (dim 288, 6 layers, hidden 768, vocab 32000):
    # the 32000 x 288 sections span several 64 MiB staging chunks' worth of
    # rows only for the classifier; arrays and logits as above.
    c = e2e_model.STORIES15M
    path = str(tmp_path / "stories.bin")
    e2e_model.write_checkpoint(path, c["dim"], c["hidden"], c["layers"], c["heads"],
                               c["kv_heads"], c["vocab"], c["seq_len"], seed=3, shared=shared)
    ck = oracle.RefCheckpoint(lib, path)
    for q8 in (False, True):
        loaded = em.Model.load(path, q8=q8)
        check_arrays(loaded, ck, q8)
        created = em.Model(ck.config, ck.weights(), q8=q8)
        prompt = list(range(1, 20))
        assert np.array_equal(loaded.forward(prompt, 0), created.forward(prompt, 0))
        assert np.array_equal(loaded.forward(7, 19), created.forward(7, 19))
        loaded.close()
        created.close()


def test_large_sections_cross_staging_chunks(tmp_path):
    # A projection larger than one 64 MiB staging chunk (dim 4096: wq is
    # 64 MiB, w1 / w2 86 MiB) goes through the chunked transpose; two layers,
    # GQA 8 kv heads, untied classifier.
    path = str(tmp_path / "big.bin")
    e2e_model.write_checkpoint(path, 4096, 5504, 2, 32, 8, 3000, 16, seed=5, shared=False)
    ck = oracle.RefCheckpoint(lib, path)
    loaded = em.Model.load(path, q8=True)
    check_arrays(loaded, ck, True)
    loaded.close()


def test_load_rows_longer_than_a_staging_chunk(tmp_path):
    # w2 is stored dim rows of hidden_dim floats; with hidden_dim past 2^24
    # one row is longer than the loader's 64 MiB staging chunk, so rows go in
    # segments. A sparse file (zeros but for planted values at the segment
    # edges) must land transposed, every planted value in its place and
    # nothing else non-zero (the reference's read_transposed,
    # model.cpp:43-53, reads a row at a time into a buffer of its size).
    dim, heads, vocab, seq_len = 16, 4, 8, 8
    per = (64 << 20) // 4
    H = per + 48
    header = np.array([dim, H, 1, heads, heads, vocab, seq_len], np.int32)
    path = str(tmp_path / "wide.bin")
    off = header.nbytes
    sizes = [("emb", vocab * dim), ("rms_att", dim), ("wq", dim * dim), ("wk", dim * dim),
             ("wv", dim * dim), ("wo", dim * dim), ("rms_ffn", dim), ("w1", H * dim),
             ("w2", dim * H), ("w3", H * dim), ("rms_final", dim), ("freq", seq_len * dim // heads)]
    at = {}
    for name, count in sizes:
        at[name] = off
        off += 4 * count
    plants = {}  # (row of w2 in the file, column) -> value
    for r in (0, 7, dim - 1):
        for c in (0, per - 1, per, per + 1, H - 1):
            plants[(r, c)] = np.float32(1.0 + r + c * 1e-7)
    with open(path, "wb") as f:
        f.write(header.tobytes())
        f.seek(off - 4)
        f.write(np.zeros(1, np.float32).tobytes())
        for (r, c), v in plants.items():
            f.seek(at["w2"] + 4 * (r * H + c))
            f.write(np.array([v], np.float32).tobytes())
    model = em.Model.load(path, q8=False)
    try:
        w2 = model.weight("w2")  # H x dim: the file's w2 transposed
        assert w2.shape == (H, dim)
        for (r, c), v in plants.items():
            assert w2[c, r] == v, (r, c)
        assert int(np.count_nonzero(w2)) == len(plants)
    finally:
        model.close()
