"""The device-resident forward pass (em_model) against the reference's CPU
Transformer, compiled from its own sources (oracle/_ref/libref_model.so).

Mirrors /root/reference/tests/test_cuda_model.cpp: multi-head with a tied
classifier, grouped-query with a separate one, multi-query (:119-123), fp32
and int8 weights; decode over the whole context, prefill in chunks of 1, 1
and 5 rows, a decode step on that cache and a whole-context prefill that
rewinds over it (:57-79), every logit within the reference's 1e-4 (:31); and
the same rejections as the CPU model, after which the cache still works
(:91-106). Then the stories15M end-to-end case through this
build's own forward pass: 158-token prefill and 98 greedy decodes, token
stream identical to the CPU Transformer's.
"""
import time

import numpy as np
import pytest

import oracle
from tests import e2e_model, engine, inputs

pytestmark = pytest.mark.gpu

em = engine.load()
lib = oracle.ref_model_lib()
if lib is None:
    pytest.skip("oracle/_ref/libref_model.so not built (make -C oracle ref)",
                allow_module_level=True)

TOL = 1e-4


def load(tmp_path, heads, kv_heads, shared):
    m = e2e_model.fixture_model(heads, kv_heads, shared, seed=heads * 10 + kv_heads)
    path = str(tmp_path / "model.bin")
    e2e_model.write_raw(path, m)
    ck = oracle.RefCheckpoint(lib, path)
    return ck, ck.weights()


def close(gpu, cpu, what):
    d = float(np.abs(gpu - cpu).max())
    assert d <= TOL, f"{what}: max diff {d}"
    return d


@pytest.mark.parametrize("wtype", ["f32", "q8"])
@pytest.mark.parametrize("heads,kv_heads,shared", [(4, 4, True), (4, 2, False), (4, 1, True)],
                         ids=["mha_tied", "gqa_untied", "mqa_tied"])
def test_matches_cpu(tmp_path, heads, kv_heads, shared, wtype):
    ck, w = load(tmp_path, heads, kv_heads, shared)
    q8 = wtype == "q8"
    cpu = oracle.RefTransformer(lib, ck, q8)
    gpu = em.Model(ck.config, w, q8=q8)
    T, V = ck.config["seq_len"], ck.config["vocab_size"]
    tokens = [(p * 7 + 3) % V for p in range(T)]
    worst = 0.0
    for pos in range(T):
        print(f"model {heads}/{kv_heads} {wtype} forward pos {pos}", flush=True)
        worst = max(worst, close(gpu.forward(tokens[pos], pos), cpu.run([tokens[pos]], pos, True),
                                 f"forward at {pos}"))
    pos = 0
    for chunk in (1, 1, 5):
        part = tokens[pos:pos + chunk]
        worst = max(worst, close(gpu.forward(part, pos), cpu.run(part, pos), f"prefill at {pos}"))
        pos += chunk
    worst = max(worst, close(gpu.forward(tokens[pos], pos), cpu.run([tokens[pos]], pos, True),
                             "forward after prefill"))
    worst = max(worst, close(gpu.forward(tokens, 0), cpu.run(tokens, 0), "full prefill"))
    print(f"{heads}/{kv_heads} {wtype}: worst logit diff {worst:.2e}")
    gpu.close()


@pytest.mark.parametrize("dim,hidden,heads,kv_heads,wtype",
                         [(256, 688, 4, 2, "q8"), (256, 688, 4, 4, "f32"), (320, 864, 5, 5, "q8"),
                          (192, 512, 6, 2, "q8")],
                         ids=["d256_gqa_q8", "d256_mha_f32", "d320_q8", "d192_group3_q8"])
def test_norm_from_producer_sums_of_squares(tmp_path, dim, hidden, heads, kv_heads, wtype):
    # A width that is a multiple of 64: one-token steps take each norm GEMV's
    # scale from the sums of squares that embed and the residual reduces
    # leave (the wo and w2 GEMVs split k here, so those reduces run), and
    # rotate q and k inside the attention launch. Every decode over the
    # context, then chunked and whole prefills (which take neither path),
    # against the CPU Transformer.
    #
    # d192_group3: three query heads per kv head, one per split workgroup,
    # so only the first of them writes the current key and value.
    #
    # Tolerance: these logits reach ~20 (the reference fixture's, which its
    # absolute 1e-4 is set for, are of order 1). fp32 results that differ
    # only in summation order measured up to 1.0e-5 of the largest logit here
    # on every GPU path, with or without the fused steps; the bound is 3e-5
    # of it, and every decode's greedy token must equal the CPU's.
    m = e2e_model.fixture_model(heads, kv_heads, False, seed=dim + heads, dim=dim,
                                hidden=hidden, vocab=300, seq_len=24)
    path = str(tmp_path / "model.bin")
    e2e_model.write_raw(path, m)
    ck = oracle.RefCheckpoint(lib, path)
    q8 = wtype == "q8"
    cpu = oracle.RefTransformer(lib, ck, q8)
    gpu = em.Model(ck.config, ck.weights(), q8=q8)
    T, V = ck.config["seq_len"], ck.config["vocab_size"]
    tokens = [(p * 11 + 5) % V for p in range(T)]

    def near(g, c, what):
        tol = 3e-5 * float(np.abs(c).max())
        d = float(np.abs(g - c).max())
        assert d <= tol, f"{what}: max diff {d} > {tol}"
        return d / tol

    worst = 0.0
    for pos in range(T):
        print(f"dim {dim} {wtype} forward pos {pos}", flush=True)
        g, c = gpu.forward(tokens[pos], pos), cpu.run([tokens[pos]], pos, True)
        worst = max(worst, near(g, c, f"forward at {pos}"))
        assert int(np.argmax(g)) == int(np.argmax(c)), f"greedy token at {pos}"
    worst = max(worst, near(gpu.forward(tokens[:7], 0), cpu.run(tokens[:7], 0), "prefill 7"))
    worst = max(worst, near(gpu.forward(tokens[7], 7), cpu.run([tokens[7]], 7, True),
                            "forward after prefill"))
    worst = max(worst, near(gpu.forward(tokens, 0), cpu.run(tokens, 0), "full prefill"))
    print(f"dim {dim} {wtype}: worst logit diff {worst:.2f} of the bound")
    gpu.close()


@pytest.mark.parametrize("seq_len", [1024, 2048])
@pytest.mark.parametrize("dim,hidden,heads,kv_heads,wtype",
                         [(256, 688, 4, 2, "q8"), (256, 688, 2, 2, "f32")],
                         ids=["hs64_gqa_q8", "hs128_f32"])
def test_decode_merge_inside_wo_gemv(tmp_path, monkeypatch, dim, hidden, heads, kv_heads,
                                     wtype, seq_len):
    # One-token steps leave the split attention's chunks unmerged, and the wo
    # GEMV merges them as it stages its A when a row has 2 to 16 chunks; a
    # row of more is merged by the merge kernel, and the GEMV reads its
    # output. A second model created with EM_DECODE_MERGE_KERNEL=1 merges
    # every row with the merge kernel first. Both merge in the same slots and
    # order, so every decode's logits must be the same bits. With one head
    # per split workgroup (hs128) chunks are at least 64 positions: the
    # decodes cover one chunk (the split kernel writes the row itself), a
    # second chunk from position 64, one slot up to 8 chunks, two from 9
    # (position 512), 16 from 960 and, at seq_len 2048, 17 from 1024. With
    # two heads per workgroup (hs64_gqa) they are at least 32: 2-3 chunks
    # at 40-80, 16 then 17 at 500-540 (the wo GEMV, then the merge kernel),
    # 32 from 1000. Each decode is checked against the CPU Transformer too,
    # greedy token equal, within the reference's 1e-4 taken relative to the
    # largest logit (~18 here; the reference's fixture logits are of order
    # 1). The 3e-5 of the short-context test above is too tight over
    # hundreds of positions: at position 55, where both models run the
    # one-chunk path, fp32 summation order alone measured 3.7e-5.
    m = e2e_model.fixture_model(heads, kv_heads, False, seed=dim + 7 * heads, dim=dim,
                                hidden=hidden, vocab=300, seq_len=seq_len)
    path = str(tmp_path / "model.bin")
    e2e_model.write_raw(path, m)
    ck = oracle.RefCheckpoint(lib, path)
    q8 = wtype == "q8"
    w = ck.weights()
    cpu = oracle.RefTransformer(lib, ck, q8)
    fused = em.Model(ck.config, w, q8=q8)
    monkeypatch.setenv("EM_DECODE_MERGE_KERNEL", "1")
    merged_first = em.Model(ck.config, w, q8=q8)
    monkeypatch.delenv("EM_DECODE_MERGE_KERNEL")
    V = ck.config["vocab_size"]
    tokens = [(p * 13 + 7) % V for p in range(seq_len)]
    pos, worst = 0, 0.0
    for prefill_to, decode_to in ((40, 80), (500, 540), (1000, min(1040, seq_len))):
        part = tokens[pos:prefill_to]
        print(f"merge {wtype} heads {heads} seq_len {seq_len}: prefill {pos}..{prefill_to}",
              flush=True)
        a, b = fused.forward(part, pos), merged_first.forward(part, pos)
        assert np.array_equal(a, b), f"prefill to {prefill_to}"
        cpu.run(part, pos)
        for pos in range(prefill_to, decode_to):
            print(f"merge {wtype} heads {heads} seq_len {seq_len}: decode {pos}", flush=True)
            a, b = fused.forward(tokens[pos], pos), merged_first.forward(tokens[pos], pos)
            assert np.array_equal(a, b), f"decode at {pos}: max diff {np.abs(a - b).max()}"
            c = cpu.run([tokens[pos]], pos, True)
            tol = 1e-4 * float(np.abs(c).max())
            d = float(np.abs(a - c).max())
            assert d <= tol, f"decode at {pos}: max diff {d} > {tol}"
            assert int(np.argmax(a)) == int(np.argmax(c)), f"greedy token at {pos}"
            worst = max(worst, d / tol)
        pos = decode_to
    print(f"merge {wtype} heads {heads}: worst logit diff {worst:.2f} of the bound")
    fused.close()
    merged_first.close()


@pytest.mark.parametrize("dim,hidden,heads,kv_heads",
                         [(256, 688, 4, 2), (320, 864, 5, 5), (192, 512, 6, 2),
                          (256, 4608, 4, 2)],
                         ids=["d256_gqa", "d320_mha", "d192_group3", "d256_wide_ffn"])
def test_strip_copy_decode_matches_cpu(tmp_path, monkeypatch, dim, hidden, heads, kv_heads):
    # int8 with a vocabulary of 320 (a multiple of 16): every projection
    # takes a strip-layout copy, so one-token steps run each product as one
    # em_matmul_q8 call over it (norm and residual inside, the attention
    # merging its own chunks, w13 and the SwiGLU one launch). A second model
    # created with EM_MODEL_STRIPS=0 runs the row-major decode path, a third
    # with EM_MODEL_SWIGLU_FUSION=0 the strips with swiglu_kernel after the
    # w13 product, which must give the fused model's logits bit for bit.
    # Every decode over the context, then a chunked and a whole prefill
    # (row-major either way), each model against the CPU Transformer within
    # the 3e-5 of the largest logit used above, greedy token equal. With
    # hidden 4608 the w13 product has 576 strips (288 gate | up pairs), more
    # workgroups than the 256 CUs in both w13 paths.
    m = e2e_model.fixture_model(heads, kv_heads, False, seed=dim + 3 * heads, dim=dim,
                                hidden=hidden, vocab=320, seq_len=24)
    path = str(tmp_path / "model.bin")
    e2e_model.write_raw(path, m)
    ck = oracle.RefCheckpoint(lib, path)
    w = ck.weights()
    cpu = oracle.RefTransformer(lib, ck, True)
    strips = em.Model(ck.config, w, q8=True)
    monkeypatch.setenv("EM_MODEL_STRIPS", "0")
    rowmajor = em.Model(ck.config, w, q8=True)
    monkeypatch.delenv("EM_MODEL_STRIPS")
    monkeypatch.setenv("EM_MODEL_SWIGLU_FUSION", "0")
    unfused = em.Model(ck.config, w, q8=True)
    monkeypatch.delenv("EM_MODEL_SWIGLU_FUSION")
    T, V = ck.config["seq_len"], ck.config["vocab_size"]
    tokens = [(p * 7 + 3) % V for p in range(T)]

    def near(g, c, what):
        tol = 3e-5 * float(np.abs(c).max())
        d = float(np.abs(g - c).max())
        assert d <= tol, f"{what}: max diff {d} > {tol}"
        assert int(np.argmax(g)) == int(np.argmax(c)), f"{what}: greedy token"

    for pos in range(T):
        print(f"strip decode dim {dim} pos {pos}", flush=True)
        c = cpu.run([tokens[pos]], pos, True)
        g = strips.forward(tokens[pos], pos)
        near(g, c, f"strips at {pos}")
        near(rowmajor.forward(tokens[pos], pos), c, f"row-major at {pos}")
        u = unfused.forward(tokens[pos], pos)
        assert np.array_equal(g, u), f"SwiGLU fused against not at {pos}: {np.abs(g - u).max()}"
    c = cpu.run(tokens[:7], 0)
    near(strips.forward(tokens[:7], 0), c, "prefill 7")
    c = cpu.run([tokens[7]], 7, True)
    near(strips.forward(tokens[7], 7), c, "decode after prefill")
    c = cpu.run(tokens, 0)
    near(strips.forward(tokens, 0), c, "full prefill")
    strips.close()
    rowmajor.close()
    unfused.close()


@pytest.mark.parametrize("dim,hidden,heads,kv_heads",
                         [(256, 688, 4, 2), (320, 864, 5, 5), (256, 4608, 4, 2)],
                         ids=["h688_partial_tile", "h864_mha", "h4608_wide"])
def test_prefill_swiglu_pair_same_bits(tmp_path, monkeypatch, dim, hidden, heads, kv_heads):
    # Int8 prefill rows past 16 form silu(gate) * up in the exact-split w13
    # product's epilogue (each 256-column tile holds 128 gates and their 128
    # ups); a second model created with EM_MODEL_SWIGLU_FUSION=0 writes the
    # product and runs swiglu_kernel. Every logit must be the same bits: a
    # 40-row prefill, a 100-row chunk from position 40, then decode steps
    # over the caches both wrote; each against the CPU Transformer too.
    # hidden 688 = 5 x 128 + 48 leaves a last tile of 48 gates; 864 = 6 x 128
    # + 96; 4608 = 36 x 128.
    m = e2e_model.fixture_model(heads, kv_heads, False, seed=500 + dim + hidden, dim=dim,
                                hidden=hidden, vocab=300, seq_len=160)
    path = str(tmp_path / "model.bin")
    e2e_model.write_raw(path, m)
    ck = oracle.RefCheckpoint(lib, path)
    w = ck.weights()
    cpu = oracle.RefTransformer(lib, ck, True)
    monkeypatch.delenv("EM_MODEL_SWIGLU_FUSION", raising=False)
    paired = em.Model(ck.config, w, q8=True)
    monkeypatch.setenv("EM_MODEL_SWIGLU_FUSION", "0")
    unpaired = em.Model(ck.config, w, q8=True)
    monkeypatch.delenv("EM_MODEL_SWIGLU_FUSION")
    V = ck.config["vocab_size"]
    tokens = [(p * 17 + 9) % V for p in range(160)]

    def check(a, b, c, what):
        assert np.array_equal(a, b), f"{what}: max diff {np.abs(a - b).max()}"
        tol = 1e-4 * float(np.abs(c).max())
        assert float(np.abs(a - c).max()) <= tol, what
        assert int(np.argmax(a)) == int(np.argmax(c)), f"{what}: greedy token"

    print(f"swiglu pair hidden {hidden}: prefill 0..40", flush=True)
    check(paired.forward(tokens[:40], 0), unpaired.forward(tokens[:40], 0),
          cpu.run(tokens[:40], 0), "prefill 40")
    print(f"swiglu pair hidden {hidden}: prefill 40..140", flush=True)
    check(paired.forward(tokens[40:140], 40), unpaired.forward(tokens[40:140], 40),
          cpu.run(tokens[40:140], 40), "prefill 40..140")
    for pos in range(140, 146):
        print(f"swiglu pair hidden {hidden}: decode {pos}", flush=True)
        check(paired.forward(tokens[pos], pos), unpaired.forward(tokens[pos], pos),
              cpu.run([tokens[pos]], pos, True), f"decode at {pos}")
    paired.close()
    unpaired.close()


@pytest.mark.parametrize("dim", [256, 240])
@pytest.mark.parametrize("heads,kv_heads", [(4, 4), (4, 2)], ids=["mha", "gqa"])
def test_prefill_rope_epilogue_same_bits_as_rope_kernel(tmp_path, monkeypatch, heads, kv_heads, dim):
    # Int8 prefill rows send the fused qkv product to the exact-split kernel;
    # with no k split (k = dim here) it rotates q and k and writes the
    # caches in its epilogue (dim 240: k not a whole number of 32-row chunks,
    # head size 60). A second model created with
    # EM_PREFILL_ROPE_FUSION=0 writes qkv and runs rope_cache_kernel
    # instead. Every logit must be the same bits: prefill from 0, a second
    # prefill chunk from position 40 (angles taken at pos + row) and decode
    # steps that read the caches both wrote. Against the CPU Transformer too.
    m = e2e_model.fixture_model(heads, kv_heads, False, seed=300 + heads + kv_heads, dim=dim,
                                hidden=688, vocab=300, seq_len=128)
    path = str(tmp_path / "model.bin")
    e2e_model.write_raw(path, m)
    ck = oracle.RefCheckpoint(lib, path)
    w = ck.weights()
    cpu = oracle.RefTransformer(lib, ck, True)
    fused = em.Model(ck.config, w, q8=True)
    monkeypatch.setenv("EM_PREFILL_ROPE_FUSION", "0")
    plain = em.Model(ck.config, w, q8=True)
    monkeypatch.delenv("EM_PREFILL_ROPE_FUSION")
    V = ck.config["vocab_size"]
    tokens = [(p * 17 + 3) % V for p in range(100)]
    steps = [(tokens[:40], 0), (tokens[40:72], 40)] + [([tokens[p]], p) for p in range(72, 80)]
    for part, pos in steps:
        a, b = fused.forward(part, pos), plain.forward(part, pos)
        assert np.array_equal(a, b), f"{len(part)} rows at {pos}: max diff {np.abs(a - b).max()}"
        c = cpu.run(part, pos, len(part) == 1)
        assert float(np.abs(a - c).max()) <= 1e-4 * float(np.abs(c).max()), f"at {pos}"
    fused.close()
    plain.close()


def test_bad_inputs_then_cache_still_works(tmp_path):
    ck, w = load(tmp_path, 4, 2, True)
    gpu = em.Model(ck.config, w)
    cpu = oracle.RefTransformer(lib, ck, False)
    V, T = ck.config["vocab_size"], ck.config["seq_len"]
    with pytest.raises(em.OutOfRange):
        gpu.forward(V, 0)
    with pytest.raises(em.OutOfRange):
        gpu.forward(-1, 0)
    with pytest.raises(em.OutOfRange):
        gpu.forward(0, 1)  # skips position 0
    with pytest.raises(em.InvalidArgument):
        gpu.forward(np.array([], np.int32), 0)
    with pytest.raises(em.OutOfRange):
        gpu.forward([0] * (T + 1), 0)
    close(gpu.forward([1, 2, 3], 0), cpu.run([1, 2, 3], 0), "after errors")
    gpu.close()


def test_repeat_gives_identical_bits(tmp_path):
    # Rewinding and feeding the same tokens again replays the captured graph;
    # its logits must equal the first pass's bit for bit.
    ck, w = load(tmp_path, 4, 1, True)
    gpu = em.Model(ck.config, w, q8=True)
    T = ck.config["seq_len"]
    first = [gpu.forward(t % 29, p) for p, t in enumerate(range(3, 3 + T))]
    second = [gpu.forward(t % 29, p) for p, t in enumerate(range(3, 3 + T))]
    for a, b in zip(first, second):
        assert np.array_equal(a, b)
    gpu.close()


@pytest.fixture(scope="module")
def stories15m(tmp_path_factory):
    d = tmp_path_factory.mktemp("s15m_model")
    path = str(d / "model.bin")
    e2e_model.write_checkpoint(path, seed=15, shared=False, **e2e_model.STORIES15M)
    ck = oracle.RefCheckpoint(lib, path)
    prompt = e2e_model.write_prompt(str(d / "prompt.txt"), 158, e2e_model.STORIES15M["vocab"],
                                    seed=158)
    return ck, ck.weights(), prompt


@pytest.mark.parametrize("wtype", ["f32", "q8"])
def test_config4_stream_through_device_forward_pass(stories15m, wtype):
    ck, w, prompt = stories15m
    q8 = wtype == "q8"
    cpu = oracle.RefTransformer(lib, ck, q8)
    gpu = em.Model(ck.config, w, q8=q8)
    lc, lg = cpu.run(prompt, 0), gpu.forward(prompt, 0)
    worst = close(lg, lc, "prefill logits")
    toks_c, toks_g = [int(np.argmax(lc))], [int(np.argmax(lg))]
    pos = len(prompt)
    t_gpu = 0.0
    for step in range(98):
        lc = cpu.run([toks_c[-1]], pos, True)
        t0 = time.perf_counter()
        lg = gpu.forward(toks_g[-1], pos)
        t_gpu += time.perf_counter() - t0
        worst = max(worst, float(np.abs(lg - lc).max()))
        toks_c.append(int(np.argmax(lc)))
        toks_g.append(int(np.argmax(lg)))
        pos += 1
    print(f"config4 {wtype}: worst logit diff {worst:.2e}; gpu decode "
          f"{t_gpu / 98 * 1e3:.3f} ms/token (host call, graph replay)")
    assert len(toks_c) == 99
    assert toks_g == toks_c
    gpu.close()


def llama7b_shaped(torch, n_layers, n_kv_heads, seq_len, seed):
    """Config and CPU-layout weights at Llama-2-7B dimensions (dim 4096,
    hidden 11008, 32 heads, vocab 32000), n_layers deep: projections and
    classifier ~N(0, 0.02), embedding ~N(0, 1), RMSNorm gains 1. Drawn on the
    GPU from a seeded generator (host numpy would take minutes at this size)."""
    D, H, V, heads = 4096, 11008, 32000, 32
    KV = n_kv_heads * (D // heads)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)

    def rnd(*shape, std=0.02):
        return (torch.randn(shape, generator=g, device="cuda") * std).cpu().numpy()

    layers = [dict(rms_att=np.ones(D, np.float32), wqkv=rnd(D, D + 2 * KV), wo=rnd(D, D),
                   rms_ffn=np.ones(D, np.float32), w13=rnd(D, 2 * H), w2=rnd(H, D))
              for _ in range(n_layers)]
    cfg = dict(dim=D, hidden_dim=H, n_layers=n_layers, n_heads=heads, n_kv_heads=n_kv_heads,
               vocab_size=V, seq_len=seq_len)
    w = dict(token_embedding=rnd(V, D, std=1.0), rms_final=np.ones(D, np.float32),
             wcls=rnd(D, V), layers=layers)
    return cfg, w


@pytest.mark.parametrize("n_kv_heads", [32, 8], ids=["mha", "gqa8"])
def test_llama7b_shaped_model_matches_cpu(n_kv_heads):
    # The forward pass at Llama-7B layer shapes (and an
    # 8-kv-head GQA variant), int8 weights, two layers deep: a 48-token
    # prefill and 8 greedy decode steps against the reference's CPU
    # Transformer on the same weights.
    torch = pytest.importorskip("torch")
    cfg, w = llama7b_shaped(torch, 2, n_kv_heads, 256, seed=70 + n_kv_heads)
    ck = oracle.RefCheckpoint(lib, config=cfg, weights=w)
    cpu = oracle.RefTransformer(lib, ck, True)
    gpu = em.Model(cfg, w, q8=True)
    del w
    prompt = [int(t) for t in inputs._splitmix64(7000 + n_kv_heads, 48) % np.uint64(32000)]
    lc, lg = cpu.run(prompt, 0), gpu.forward(prompt, 0)
    scale = float(np.abs(lc).max())
    worst = float(np.abs(lg - lc).max())
    toks_c, toks_g = [int(np.argmax(lc))], [int(np.argmax(lg))]
    pos = len(prompt)
    for _ in range(8):
        print(f"llama7b-shaped kv={n_kv_heads} decode pos {pos}", flush=True)
        lc, lg = cpu.run([toks_c[-1]], pos, True), gpu.forward(toks_g[-1], pos)
        worst = max(worst, float(np.abs(lg - lc).max()))
        toks_c.append(int(np.argmax(lc)))
        toks_g.append(int(np.argmax(lg)))
        pos += 1
    print(f"llama7b-shaped kv={n_kv_heads}: worst logit diff {worst:.2e} (max |logit| {scale:.2f})")
    assert worst <= 1e-4 * max(1.0, scale) * 10, worst
    assert toks_g == toks_c
    gpu.close()


@pytest.mark.parametrize("dim,hidden,heads,kv_heads",
                         [(256, 688, 2, 2), (256, 688, 4, 2)], ids=["hs128_mha", "hs64_gqa"])
def test_strip_decode_merges_chunks_inside_attention(tmp_path, monkeypatch, dim, hidden, heads,
                                                     kv_heads):
    # One-token steps over strip copies merge the split attention's chunks
    # inside the attention launch: the last of a row's chunk workgroups to
    # finish merges them, in the merge kernel's slots and order. The model
    # created with EM_DECODE_MERGE_KERNEL=0 does so for every shape (by
    # default only where a workgroup serves one head); a second model
    # created with EM_DECODE_MERGE_KERNEL=1 launches the merge kernel
    # instead, so every decode's logits must be the same bits; both against
    # the CPU Transformer (greedy token equal, 1e-4 of the largest logit).
    # Decodes from one chunk up to 16 and 32 chunks (hs128: 64-position
    # chunks; hs64 with two heads per workgroup: 32-position chunks).
    seq_len = 1024
    m = e2e_model.fixture_model(heads, kv_heads, False, seed=dim + 11 * heads, dim=dim,
                                hidden=hidden, vocab=320, seq_len=seq_len)
    path = str(tmp_path / "model.bin")
    e2e_model.write_raw(path, m)
    ck = oracle.RefCheckpoint(lib, path)
    w = ck.weights()
    cpu = oracle.RefTransformer(lib, ck, True)
    monkeypatch.setenv("EM_DECODE_MERGE_KERNEL", "0")
    inside = em.Model(ck.config, w, q8=True)
    monkeypatch.setenv("EM_DECODE_MERGE_KERNEL", "1")
    launched = em.Model(ck.config, w, q8=True)
    monkeypatch.delenv("EM_DECODE_MERGE_KERNEL")
    V = ck.config["vocab_size"]
    tokens = [(p * 11 + 5) % V for p in range(seq_len)]
    pos = 0
    for prefill_to, decode_to in ((40, 80), (500, 520), (990, 1024)):
        part = tokens[pos:prefill_to]
        a, b = inside.forward(part, pos), launched.forward(part, pos)
        assert np.array_equal(a, b), f"prefill to {prefill_to}"
        cpu.run(part, pos)
        for pos in range(prefill_to, decode_to):
            print(f"strip merge heads {heads}: decode {pos}", flush=True)
            a, b = inside.forward(tokens[pos], pos), launched.forward(tokens[pos], pos)
            assert np.array_equal(a, b), f"decode at {pos}: max diff {np.abs(a - b).max()}"
            c = cpu.run([tokens[pos]], pos, True)
            tol = 1e-4 * float(np.abs(c).max())
            assert float(np.abs(a - c).max()) <= tol, f"decode at {pos}"
            assert int(np.argmax(a)) == int(np.argmax(c)), f"greedy token at {pos}"
        pos = decode_to
    inside.close()
    launched.close()
