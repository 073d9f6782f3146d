#!/usr/bin/env python3
"""Benchmark of the MI355X matmul hot path (BASELINE.json metric).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-extra]
    python bench.py --profile-pass      (eager launches for rocprofv3 --pmc)

Workload (the metric's headline): int8-weight GEMV,
m = 1, A[1, 4096] fp32 ~ N(0, 1) times W[4096, 4096] ~ N(0, 0.02) quantised
by this library's quantize_q8 (bit-exact with quant.cpp). POOL copies of
(W_q, scale) -- over 512 MiB -- are visited in turn so each product reads its
weights from HBM, not from the 256 MB Infinity Cache. One step is one sweep
over the pool (POOL products, each on its own weights). The timed region
replays a HIP graph of one step K times: products are launched back to back
as a decode loop would launch them (the reference also replays its decode
step as a graph, cuda_model.cu:189-230), so the host's launch cost does not
hide the kernel.

value = algorithmic bytes (W + scales + A + C) x products / seconds, in GB/s.
The JSON line also carries:
  roofline     the product's algorithmic bytes per call / its average call
               time from HIP events over the timed region, against 8 TB/s
               HBM; traffic = HBM bytes per call measured with FETCH_SIZE and
               WRITE_SIZE (profiles/gemv_int8_m1_4096_traffic.json)
  cpu_baseline the reference's own matmul_parallel (oracle/_ref, built from
               /root/reference/src with amdclang++ -O3) on the box's host
               cores, same inputs, median as bench_matmul.cpp:49-63
  extra        the metric's second half (fp32 GEMM N = 4096 on MFMA, TFLOPS
               and % of the 157.3 TFLOPS fp32 MFMA peak), int8 GEMV at
               m = 4/16/64, fp32 GEMV m = 1, and the reference's own timing
               convention (host launch -> synchronize, median)
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, 8 TB/s
FP32_MFMA_PEAK_TFLOPS = 157.3
BF16_MFMA_PEAK_TFLOPS = 2516.6   # MI355X dense bf16 (no sparsity)
# int8 B above 8 rows (and at 2-8 rows by a shape rule) runs on bf16 MFMA
# with A split exactly into three bf16 terms: three MFMA products per fp32
# multiply-add, so its compute roof in fp32-equivalent flops is a third of
# the bf16 peak.
EXACT_SPLIT_PEAK_TFLOPS = BF16_MFMA_PEAK_TFLOPS / 3


def q8_kernel(m: int, k: int = 4096, n: int = 4096, registered: bool = False) -> tuple:
    """(kernel name, compute peak in TFLOP/s) that automatic uses for int8 B.
    Registered weights (em_q8_register, as DeviceQTensor does): one row runs
    the strip-copy GEMV (k <= 8192, or 12288 with n >= 4096: no norm here), 2 - 4 rows (k <= 4096) and 5 - 8 rows (k, n <= 4096)
    the strip-copy MFMA kernel (decode_mfma_supported). Otherwise (and
    unregistered): the GEMV up to 4 rows of small weights, the exact-split
    kernel from 5 rows (split_bf16_preferred)."""
    if registered and m == 1 and (k <= 8192 or (k <= 12288 and n >= 4096)):
        return "strip-copy GEMV (fp32 VALU)", FP32_MFMA_PEAK_TFLOPS / 2
    if registered and 2 <= m <= 8 and k <= 4096 and k % 4 == 0 and (
            m <= 2 or (m <= 4 and n <= 24576) or n <= 4096):
        return "strip-copy fp32 MFMA (v_mfma_f32_4x4x1_16b_f32)", FP32_MFMA_PEAK_TFLOPS
    w = k * n
    if m < 5 and not (m >= 3 and w >= 1 << 25) and not (m >= 2 and w >= 1 << 26):
        return "skinny GEMV (fp32 VALU)", FP32_MFMA_PEAK_TFLOPS / 2
    return "exact-split bf16 MFMA (3 terms)", EXACT_SPLIT_PEAK_TFLOPS
METRIC = "int8 GEMV HBM GB/s (m=1, 4096²) + fp32 GEMM TFLOPS (N=4096), % of peak"
DIM = 4096
POOL_MIN_BYTES = 600 << 20   # > 512 MiB


def load_engine():
    spec = importlib.util.spec_from_file_location(
        "llm_engine_amd", os.path.join(ROOT, "llm-engine_amd", "__init__.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules["llm_engine_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def gemv_bytes(m: int, k: int, n: int, q8: bool) -> int:
    """Algorithmic bytes: W + (int8) scales + A + C."""
    return k * n * (1 if q8 else 4) + (4 * n if q8 else 0) + 4 * m * k + 4 * m * n


class Pool:
    """POOL copies of a K x N weight matrix (int8 + scales, or fp32) on the GPU.
    With packed, int8 copies are kept in the strip layout (em_pack_q8) only;
    with register, each row-major int8 copy is registered with the library
    (em_q8_register, what the C++ DeviceQTensor does when it is built), so
    em_matmul_q8 runs one-row products over its strip copy."""

    def __init__(self, em, torch, q8: bool, k: int, n: int, copies: int, seed: int,
                 packed: bool = False, register: bool = False):
        self.q8 = q8
        self.packed = packed
        self.em = em
        self.registered = []
        self.ws, self.scales = [], []
        g = torch.Generator(device="cuda")
        for i in range(copies):
            g.manual_seed(seed + i)
            W = torch.randn((k, n), generator=g, device="cuda", dtype=torch.float32) * 0.02
            if q8:
                q, s = em.quantize_q8(W)
                if packed:
                    pq = em.pack_q8(q)
                    del q
                    q = pq
                elif register:
                    em.register_q8(q)
                    self.registered.append(q)
                self.ws.append(q)
                self.scales.append(s)
                del W
            else:
                self.ws.append(W)
                self.scales.append(None)
        torch.cuda.synchronize()

    def close(self):
        for q in self.registered:
            self.em.unregister_q8(q)
        self.registered = []
        self.ws, self.scales = [], []

    def __del__(self):
        self.close()


def pool_product(em, A, C, pool, w, s):
    if pool.packed:
        em.matmul_packed(A, w, C.shape[1], s, C)
    else:
        em.matmul(A, w, C, scale=s)


def capture_step(em, torch, A, C, pool: Pool):
    """A HIP graph of one sweep over the pool."""
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):  # warm the library's scratch outside capture
        for w, s in zip(pool.ws, pool.scales):
            pool_product(em, A, C, pool, w, s)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for w, s in zip(pool.ws, pool.scales):
            pool_product(em, A, C, pool, w, s)
    torch.cuda.synchronize()
    return graph


def time_graph(torch, graph, steps: int, warmup: int):
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return start.elapsed_time(end) / 1e3, wall


def gemv_case(em, torch, m, q8, steps, warmup, copies=None, seed=1000, k=DIM, n=DIM,
              packed=False, register=False):
    per_copy = k * n * (1 if q8 else 4)
    copies = copies or max(2, -(-POOL_MIN_BYTES // per_copy))
    pool = Pool(em, torch, q8, k, n, copies, seed, packed=packed, register=register)
    g = torch.Generator(device="cuda")
    g.manual_seed(7 + m)
    A = torch.randn((m, k), generator=g, device="cuda", dtype=torch.float32)
    C = torch.empty((m, n), device="cuda", dtype=torch.float32)
    graph = capture_step(em, torch, A, C, pool)
    secs, wall = time_graph(torch, graph, steps, warmup)
    calls = steps * copies
    nbytes = gemv_bytes(m, k, n, q8)
    out = {"m": m, "q8": q8, "copies": copies, "pool_MiB": round(copies * per_copy / 2**20, 1),
           "calls": calls, "us_per_call": secs / calls * 1e6,
           "GBps": nbytes * calls / secs / 1e9, "bytes_per_call": nbytes,
           "wall_s": wall, "secs": secs, "flops_per_call": 2 * m * k * n}
    del graph
    pool.close()
    del pool
    torch.cuda.synchronize()
    return out, (A, C)


# Config 5: Llama-7B layer projections (in x out), int8 weights.
LLAMA7B_LAYER = [("wq", 4096, 4096), ("wk", 4096, 4096), ("wv", 4096, 4096), ("wo", 4096, 4096),
                 ("w1", 4096, 11008), ("w3", 4096, 11008), ("w2", 11008, 4096)]


# The reference's attention benchmark shapes (bench_attention.cpp:93-97):
# (name, heads, kv_heads, head_size) and its contexts.
ATTENTION_MODELS = [("stories15M (6 x 48)", 6, 6, 48), ("7B MHA (32 x 128)", 32, 32, 128),
                    ("8B GQA (32 x 128, 8 kv)", 32, 8, 128)]
ATTENTION_CONTEXTS = (32, 256, 1024, 4096, 16384)


def attention_case(em, torch, reps: int = 20):
    """Decode attention, one row, per call in a HIP graph, at the last
    position of each context; K and V rotate over enough copies to exceed
    512 MiB so they come from HBM. GB/s counts K and V (the reference's
    bench_attention convention)."""
    out = {}
    for name, heads, kv_heads, hs in ATTENTION_MODELS:
        for n_ctx in ATTENTION_CONTEXTS:
            if heads == 6 and n_ctx > 256:
                continue  # stories15M's seq_len is 256
            dim, kv = heads * hs, kv_heads * hs
            shape = em.attention_shape(heads, kv_heads, hs, n_ctx, q_stride=dim)
            kv_bytes = 2 * n_ctx * kv * 4
            copies = max(1, -(-POOL_MIN_BYTES // kv_bytes))
            q = torch.randn((1, dim), device="cuda")
            caches = [(torch.randn((n_ctx, kv), device="cuda"), torch.randn((n_ctx, kv), device="cuda"))
                      for _ in range(copies)]
            res = {}
            for kernel in ("split", "automatic"):
                scratch = torch.zeros((max(1, em.attention_scratch_floats(shape, 1, kernel)),),
                                      device="cuda")
                o = torch.empty((1, dim), device="cuda")
                pos = torch.full((1,), n_ctx - 1, dtype=torch.int32, device="cuda")
                stream = torch.cuda.Stream()
                stream.wait_stream(torch.cuda.current_stream())
                with torch.cuda.stream(stream):
                    for kc, vc in caches:
                        em.attention(shape, 1, pos, q, kc, vc, o, scratch, kernel)
                torch.cuda.current_stream().wait_stream(stream)
                torch.cuda.synchronize()
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    for kc, vc in caches:
                        em.attention(shape, 1, pos, q, kc, vc, o, scratch, kernel)
                secs, _ = time_graph(torch, g, reps, 2)
                us = secs / (reps * copies) * 1e6
                res[kernel] = {"us": round(us, 2), "GBps": round(kv_bytes / us / 1e3, 1)}
                del g
            out[f"{name} ctx {n_ctx}"] = res
            del caches
            torch.cuda.synchronize()
    return out


def llama7b_model(em, torch, n_layers: int = 2, n_kv_heads: int = 32, seq_len: int = 1024):
    """An em_model at Llama-2-7B dimensions, n_layers deep, int8 weights
    (random ~N(0, 0.02), drawn on the GPU, embedding ~N(0, 1), norm gains 1)."""
    import numpy as np
    D, H, V, heads = 4096, 11008, 32000, 32
    KV = n_kv_heads * (D // heads)
    g = torch.Generator(device="cuda")
    g.manual_seed(77)

    def rnd(*shape, std=0.02):
        return (torch.randn(shape, generator=g, device="cuda") * std).cpu().numpy()

    ones = np.ones(D, np.float32)
    layers = [dict(rms_att=ones, wqkv=rnd(D, D + 2 * KV), wo=rnd(D, D), rms_ffn=ones,
                   w13=rnd(D, 2 * H), w2=rnd(H, D)) for _ in range(n_layers)]
    cfg = dict(dim=D, hidden_dim=H, n_layers=n_layers, n_heads=heads, n_kv_heads=n_kv_heads,
               vocab_size=V, seq_len=seq_len)
    return em.Model(cfg, dict(token_embedding=rnd(V, D, std=1.0), rms_final=ones,
                              wcls=rnd(D, V), layers=layers), q8=True)


def llama7b_model_case(em, torch, n_layers: int = 2, n_kv_heads: int = 32, seq_len: int = 1024):
    """The device-resident forward pass (em_model) at Llama-2-7B dimensions
    (llama7b_model): a 512-token prefill, then greedy decode steps from
    position 512, each a host call that returns the logits (graph replay)."""
    import numpy as np
    model = llama7b_model(em, torch, n_layers, n_kv_heads, seq_len)
    prompt = [(7 * i + 3) % 32000 for i in range(512)]
    model.forward(prompt, 0)  # warm-up: grows every buffer
    t0 = time.perf_counter()
    reps = 3
    for _ in range(reps):
        logits = model.forward(prompt, 0)
    prefill_s = (time.perf_counter() - t0) / reps
    tok, pos, steps = int(np.argmax(logits)), 512, 32
    model.forward(tok, pos)  # eager run + capture
    t0 = time.perf_counter()
    for i in range(steps):
        tok = int(np.argmax(model.forward(tok, pos + 1 + i)))
    decode_s = (time.perf_counter() - t0) / steps
    model.close()
    return {"layers": n_layers, "n_kv_heads": n_kv_heads, "weights": "int8",
            "prefill_512_ms": round(prefill_s * 1e3, 2),
            "prefill_tokens_per_s": round(512 / prefill_s, 1),
            "decode_ms_per_token_at_ctx_512": round(decode_s * 1e3, 3),
            "note": "host-timed em_model_forward calls (logits downloaded per call); "
                    "classifier 4096x32000 included"}


def stories15m_case(em, torch, steps: int = 98):
    """The stories15M end-to-end case through the device-resident forward pass:
    stories15M (dim 288, 6 layers, 6 heads, hidden 768, vocab 32000, seq 256),
    random weights ~N(0, 0.02), a 158-token prefill then `steps` greedy
    decodes; host-timed em_model_forward calls (logits downloaded per call)."""
    import numpy as np
    D, H, L, V, S = 288, 768, 6, 32000, 256
    g = torch.Generator(device="cuda")
    g.manual_seed(15)

    def rnd(*shape):
        return (torch.randn(shape, generator=g, device="cuda") * 0.02).cpu().numpy()

    ones = np.ones(D, np.float32)
    cfg = dict(dim=D, hidden_dim=H, n_layers=L, n_heads=6, n_kv_heads=6, vocab_size=V, seq_len=S)
    w = dict(token_embedding=rnd(V, D), rms_final=ones, wcls=rnd(D, V),
             layers=[dict(rms_att=ones, wqkv=rnd(D, 3 * D), wo=rnd(D, D), rms_ffn=ones,
                          w13=rnd(D, 2 * H), w2=rnd(H, D)) for _ in range(L)])
    prompt = [(11 * i + 5) % V for i in range(158)]
    out = {}
    for wtype in ("f32", "q8"):
        model = em.Model(cfg, w, q8=wtype == "q8")
        for rep in range(2):  # the first pass grows buffers and captures the graph
            t0 = time.perf_counter()
            logits = model.forward(prompt, 0)
            prefill_s = time.perf_counter() - t0
            tok = int(np.argmax(logits))
            t0 = time.perf_counter()
            for i in range(steps):  # positions 158 .. 158 + steps - 1
                tok = int(np.argmax(model.forward(tok, 158 + i)))
            decode_s = (time.perf_counter() - t0) / steps
        out[wtype] = {"prefill_158_ms": round(prefill_s * 1e3, 3),
                      "decode_ms_per_token": round(decode_s * 1e3, 4)}
        model.close()
    return out


def timed_best(torch, fn, reps: int = 10, windows: int = 3, warm_s: float = 0.2) -> float:
    """us per call of fn: launched untimed for warm_s seconds first (the
    clocks ramp up over the first ~100 ms of work: a same-box A/B of the
    m = 512 projections ran its first window ~10 % slower than its second),
    then the fastest of `windows` event-timed windows of `reps` calls."""
    t_end = time.perf_counter() + warm_s
    while time.perf_counter() < t_end:
        fn()
        torch.cuda.synchronize()
    best = float("inf")
    for _ in range(windows):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        best = min(best, e0.elapsed_time(e1) / reps * 1e3)
    return best


def llama7b_case(em, torch, steps):
    """Per-projection and whole-layer times at decode (m = 1, cache-cold
    rotating pools of registered weights, graph replay) and prefill (m = 512,
    timed_best over the same kind of pool, one call per copy in turn, so each
    call reads its weights from HBM as a layer of a model past the Infinity
    Cache does: warmed, best of three event-timed windows)."""
    out = {"decode_m1": {}, "prefill_m512": {}}
    times1, times512 = {}, {}
    for k, n in sorted({(k, n) for _, k, n in LLAMA7B_LAYER} | {(4096, 32000)}):
        r, _ = gemv_case(em, torch, 1, True, max(4, steps // 4), 2, seed=50, k=k, n=n,
                         register=True)
        times1[(k, n)] = r["us_per_call"]
        copies = max(2, -(-POOL_MIN_BYTES // (k * n)))
        pool = Pool(em, torch, True, k, n, copies, 60)
        A = torch.randn((512, k), device="cuda")
        C = torch.empty((512, n), device="cuda")

        def sweep(pool=pool, A=A, C=C):
            for w, sc in zip(pool.ws, pool.scales):
                em.matmul(A, w, C, scale=sc)
        times512[(k, n)] = timed_best(torch, sweep, reps=2) / copies
        pool.close()
        del pool, A, C
    for name, k, n in LLAMA7B_LAYER + [("cls", 4096, 32000)]:
        t1, t5 = times1[(k, n)], times512[(k, n)]
        out["decode_m1"][name] = {"us": round(t1, 2),
                                  "GBps": round(gemv_bytes(1, k, n, True) / t1 / 1e3, 1)}
        tf = 2 * 512 * k * n / t5 / 1e6
        out["prefill_m512"][name] = {"us": round(t5, 1), "TFLOPS": round(tf, 1),
                                     "pct_of_compute_roof": round(100 * tf / q8_kernel(512)[1], 1)}
    out["decode_m1"]["layer_us"] = round(sum(times1[(k, n)] for _, k, n in LLAMA7B_LAYER), 1)
    out["prefill_m512"]["layer_us"] = round(sum(times512[(k, n)] for _, k, n in LLAMA7B_LAYER), 1)
    layer_bytes = sum(gemv_bytes(1, k, n, True) for _, k, n in LLAMA7B_LAYER)
    layer_flops = sum(2 * 512 * k * n for _, k, n in LLAMA7B_LAYER)
    out["decode_m1"]["layer_GBps"] = round(layer_bytes / out["decode_m1"]["layer_us"] / 1e3, 1)
    out["prefill_m512"]["layer_TFLOPS"] = round(layer_flops / out["prefill_m512"]["layer_us"] / 1e6, 1)
    out["prefill_m512"]["kernel"] = q8_kernel(512)[0]
    out["prefill_m512"]["compute_roof_TFLOPS"] = round(q8_kernel(512)[1], 1)
    return out


def checkpoint_load_case(em, torch) -> dict:
    """Loading a llama2.c v0 checkpoint with em_model_load: the file streamed
    to the GPU through pinned chunks, projections transposed, fused and (q8)
    quantised there (the reference reads it with load_checkpoint on the host,
    model.cpp:115-163). Files: stories15M's shape and a one-layer Llama-7B
    shape (dim 4096, hidden 11008, vocab 32000, tied classifier, 1.33 GB),
    random ~N(0, 0.02), written to a temporary directory first (not timed).
    Wall-clock seconds, best of 2, the file in the page cache."""
    import tempfile
    import numpy as np
    out = {}
    rng = np.random.default_rng(11)
    shapes = {"stories15M": (288, 768, 6, 6, 6, 32000, 256),
              "llama7b_1layer": (4096, 11008, 1, 32, 32, 32000, 512)}
    with tempfile.TemporaryDirectory() as tmp:
        for name, (D, H, L, nh, nkv, V, S) in shapes.items():
            path = os.path.join(tmp, name + ".bin")
            KV = nkv * (D // nh)
            with open(path, "wb") as f:
                f.write(np.array([D, H, L, nh, nkv, V, S], np.int32).tobytes())
                for count in (V * D, L * D, L * D * D, L * KV * D, L * KV * D, L * D * D, L * D,
                              L * H * D, L * D * H, L * H * D, D, S * (D // nh)):
                    left = count
                    while left:
                        n = min(left, 1 << 26)
                        f.write((rng.standard_normal(n, dtype=np.float32) * 0.02).tobytes())
                        left -= n
            size = os.path.getsize(path)
            row = {"file_MB": round(size / 1e6, 1)}
            for q8 in (False, True):
                best = None
                for _ in range(2):
                    t0 = time.perf_counter()
                    m = em.Model.load(path, q8=q8)
                    best = min(best or 1e9, time.perf_counter() - t0)
                    m.close()
                tag = "q8" if q8 else "f32"
                row[f"em_model_load_{tag}_s"] = round(best, 3)
                row[f"em_model_load_{tag}_GBps"] = round(size / best / 1e9, 2)
            out[name] = row
            os.remove(path)
    out["note"] = "wall-clock s, best of 2, file in the page cache after the first read"
    return out


def fp32_decode_table(em, torch, steps: int, ms=(1, 4, 8, 16, 32, 64)) -> dict:
    """The reference bench's fp32 decode table (bench_cuda.cpp:112-144: m x
    4096^2, the engine beside cuBLAS and beside the engine with its copies)
    on this build: em_matmul_f32 (automatic) over the rotating >600 MiB fp32
    pool, graph replay; torch.mm (the vendor GEMM) over the same pool by the
    same method; and the reference's "with copies" convention, host time of
    upload A (pageable) -> product -> download C, one resident W, median of
    101."""
    out = {}
    for m in ms:
        r, _ = gemv_case(em, torch, m, False, max(5, steps // 2), 2)
        pool = Pool(em, torch, False, DIM, DIM, r["copies"], 1000)
        g = torch.Generator(device="cuda")
        g.manual_seed(7 + m)
        A = torch.randn((m, DIM), generator=g, device="cuda", dtype=torch.float32)
        C = torch.empty((m, DIM), device="cuda")
        graph = graph_of(torch, lambda i: torch.mm(A, pool.ws[i % len(pool.ws)], out=C),
                         len(pool.ws))
        secs, _ = time_graph(torch, graph, max(5, steps // 2), 2)
        vendor_us = secs / (max(5, steps // 2) * len(pool.ws)) * 1e6
        del graph
        W = pool.ws[0]
        A_host = A.cpu()
        C_host = torch.empty((m, DIM), dtype=torch.float32)
        times = []
        for i in range(102):
            t0 = time.perf_counter()
            A.copy_(A_host)
            em.matmul(A, W, C)
            C_host.copy_(C)
            torch.cuda.synchronize()
            if i:
                times.append(time.perf_counter() - t0)
        pool.close()
        del pool
        times.sort()
        out[f"m{m}"] = {"us": round(r["us_per_call"], 3), "GBps": round(r["GBps"], 1),
                        "pct_of_hbm_peak": round(100 * r["GBps"] / HBM_PEAK_GBS, 1),
                        "torch_mm_us": round(vendor_us, 3),
                        "with_copies_us": round(times[len(times) // 2] * 1e6, 1)}
    return out


def host_median_convention(em, torch, A, w, s, C, reps=101):
    """The reference's bench_cuda convention: host time launch -> synchronize."""
    em.matmul(A, w, C, scale=s)
    torch.cuda.synchronize()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        em.matmul(A, w, C, scale=s)
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    return statistics.median(times)


def gemm_case(em, torch, N=4096, reps=50, warm_s=0.3):
    """fp32 tiled GEMM, N^3: `warm_s` seconds of untimed calls (the first
    tens of milliseconds run slower while the clock settles under MFMA load),
    then one window of `reps` calls timed with HIP events."""
    import time
    g = torch.Generator(device="cuda")
    g.manual_seed(3)
    A = torch.rand((N, N), generator=g, device="cuda") * 2 - 1
    B = torch.rand((N, N), generator=g, device="cuda") * 2 - 1
    C = torch.empty((N, N), device="cuda")
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < warm_s:
        for _ in range(10):
            em.matmul(A, B, C, kernel="tiled")
        torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        em.matmul(A, B, C, kernel="tiled")
    end.record()
    torch.cuda.synchronize()
    secs = start.elapsed_time(end) / 1e3 / reps
    tflops = 2 * N**3 / secs / 1e12
    return {"N": N, "ms": secs * 1e3, "TFLOPS": tflops,
            "pct_of_fp32_mfma_peak": 100 * tflops / FP32_MFMA_PEAK_TFLOPS}, (A, B)


def vendor_gemm_case(em, torch, rounds: int = 3, warm_s: float = 0.3,
                     window_s: float = 0.05) -> dict:
    """The reference bench's yardstick column (bench_cuda.cpp:58-64,93-110,
    cuBLAS sgemm there): ROCm's fp32 GEMM through torch.mm (hipBLASLt /
    rocBLAS, full fp32: TF32-style reduced precision switched off) beside the
    library's tiled kernel, N = 1024 / 2048 / 4096, same inputs, HIP events.
    The clock settles under MFMA load over tens of milliseconds, so each side
    first runs `warm_s` seconds untimed; then `rounds` windows of about
    `window_s` seconds alternate between the two, and each side reports its
    fastest window."""
    import time
    torch.backends.cuda.matmul.allow_tf32 = False
    out = {}
    for N in (1024, 2048, 4096):
        g = torch.Generator(device="cuda")
        g.manual_seed(3)
        A = torch.rand((N, N), generator=g, device="cuda") * 2 - 1
        B = torch.rand((N, N), generator=g, device="cuda") * 2 - 1
        C = torch.empty((N, N), device="cuda")
        fns = (("tiled", lambda: em.matmul(A, B, C, kernel="tiled")),
               ("vendor_torch_mm", lambda: torch.mm(A, B, out=C)))
        for _, fn in fns:
            t0 = time.perf_counter()
            while time.perf_counter() - t0 < warm_s:
                for _ in range(10):
                    fn()
                torch.cuda.synchronize()
        reps = max(5, int(window_s / (2 * N**3 / 130e12)))
        best = {}
        for _ in range(rounds):
            for name, fn in fns:
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(reps):
                    fn()
                e1.record()
                torch.cuda.synchronize()
                ms = e0.elapsed_time(e1) / reps
                best[name] = min(best.get(name, ms), ms)
        row = {name: {"ms": round(ms, 4), "TFLOPS": round(2 * N**3 / ms / 1e9, 2)}
               for name, ms in best.items()}
        row["tiled_over_vendor"] = round(row["tiled"]["TFLOPS"] / row["vendor_torch_mm"]["TFLOPS"], 3)
        out[f"N{N}"] = row
        del A, B, C
    torch.cuda.synchronize()
    return out


CALIBRATION_BYTES = 256 << 20


def profile_pass(em, torch, sweeps: int = 2) -> dict:
    """Eager launches (one dispatch per kernel, no graph) for rocprofv3 counter
    passes. First a plain elementwise copy of CALIBRATION_BYTES (torch.neg into
    a second buffer: that many bytes read and as many written, each once), the
    yardstick the HBM byte counters are scaled by; then the headline product
    (int8 m = 1, 4096^2) over the rotating pool, `sweeps` times with the pool
    registered (the bench's value: gemv_row_kernel), then `sweeps` times
    unregistered (row-major: gemv_kernel + reduce_slices)."""
    src = torch.randn(CALIBRATION_BYTES // 4, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    del src, dst
    per_copy = DIM * DIM
    copies = -(-POOL_MIN_BYTES // per_copy)
    pool = Pool(em, torch, True, DIM, DIM, copies, 1000, register=True)
    A = torch.randn((1, DIM), device="cuda")
    C = torch.empty((1, DIM), device="cuda")
    for _ in range(sweeps):
        for w, s in zip(pool.ws, pool.scales):
            em.matmul(A, w, C, scale=s)
    torch.cuda.synchronize()
    for q in pool.registered:
        em.unregister_q8(q)
    pool.registered = []
    for _ in range(sweeps):
        for w, s in zip(pool.ws, pool.scales):
            em.matmul(A, w, C, scale=s)
    torch.cuda.synchronize()
    pool.close()
    return {"calibration_bytes": CALIBRATION_BYTES, "products": 2 * sweeps * copies,
            "bytes_per_product": gemv_bytes(1, DIM, DIM, True)}


def profile_smallm_pass(em, torch, reps: int = 20) -> dict:
    """Eager int8 products at m = 4, 8, 16, 32 and 64 over the rotating
    4096^2 pool of registered weights, as bench.py's decode rows (automatic:
    the strip-copy MFMA kernel at 4 and 8 rows, the strip-copy exact split
    at 16, the row-major exact split and its slice sum at 32 and 64), for
    counter passes over the decode-batch kernels."""
    per_copy = DIM * DIM
    copies = -(-POOL_MIN_BYTES // per_copy)
    pool = Pool(em, torch, True, DIM, DIM, copies, 1000, register=True)
    for m in (4, 8, 16, 32, 64):
        A = torch.randn((m, DIM), device="cuda")
        C = torch.empty((m, DIM), device="cuda")
        for i in range(reps):
            em.matmul(A, pool.ws[i % copies], C, scale=pool.scales[i % copies])
        torch.cuda.synchronize()
    pool.close()
    return {"m": [4, 8, 16, 32, 64], "launches_each": reps}


def profile_gemm_pass(em, torch, reps: int = 5, warm_s: float = 0.3) -> dict:
    """Eager fp32 GEMMs for rocprofv3 counter passes over the MFMA kernels: at
    N = 1024, 2048 and 4096, `reps` launches of the library's `tiled` kernel
    (N = 4096 is the metric's second half), then `reps` of torch.mm (the
    vendor yardstick), each side after `warm_s` seconds of untimed launches
    so the clock has settled."""
    import time
    torch.backends.cuda.matmul.allow_tf32 = False
    done = {}
    for N in (1024, 2048, 4096):
        A = torch.rand((N, N), device="cuda") * 2 - 1
        B = torch.rand((N, N), device="cuda") * 2 - 1
        C = torch.empty((N, N), device="cuda")
        for name, fn in (("tiled", lambda: em.matmul(A, B, C, kernel="tiled")),
                         ("torch_mm", lambda: torch.mm(A, B, out=C))):
            t0 = time.perf_counter()
            warm = 0
            while time.perf_counter() - t0 < warm_s:
                fn()
                torch.cuda.synchronize()
                warm += 1
            for _ in range(reps):
                fn()
            torch.cuda.synchronize()
            done[f"{name}_N{N}"] = {"warm_launches": warm, "profiled_launches": reps,
                                    "flops_per_launch": 2 * N**3}
        del A, B, C
    return done


def profile_split_pass(em, torch, m: int = 512, reps: int = 20) -> dict:
    """Eager int8 products at m rows over the rotating 4096^2 pool with the
    `automatic` kernel (exact-split bf16 at these sizes), for counter passes."""
    per_copy = DIM * DIM
    copies = -(-POOL_MIN_BYTES // per_copy)
    pool = Pool(em, torch, True, DIM, DIM, copies, 1000)
    A = torch.randn((m, DIM), device="cuda")
    C = torch.empty((m, DIM), device="cuda")
    for i in range(reps):
        em.matmul(A, pool.ws[i % copies], C, scale=pool.scales[i % copies])
    torch.cuda.synchronize()
    return {"m": m, "launches": reps, "flops_per_launch": 2 * m * DIM * DIM}


# The Llama-7B layer's four projections at a 512-row prefill: (k, n, norm).
LLAMA7B_PROJ = [(4096, 12288, True), (4096, 4096, False), (4096, 22016, True),
                (11008, 4096, False)]


def profile_proj_pass(em, torch, m: int = 512, reps: int = 5) -> dict:
    """Eager int8 products of the Llama-7B layer's projections at m rows
    (`automatic`: the exact-split kernel; qkv and w13 with the norm fused, so
    A is pre-split), two weight copies alternating, `reps` launches each,
    for counter passes over the prefill kernels."""
    for (k, n, norm) in LLAMA7B_PROJ:
        pool = Pool(em, torch, True, k, n, 2, 2000 + n)
        A = torch.randn((m, k), device="cuda")
        C = torch.empty((m, n), device="cuda")
        w = torch.rand((k,), device="cuda") + 0.5 if norm else None
        for i in range(reps):
            em.matmul(A, pool.ws[i % 2], C, scale=pool.scales[i % 2], rms_weight=w)
        torch.cuda.synchronize()
        pool.close()
    return {"m": m, "shapes": LLAMA7B_PROJ, "launches_each": reps}


def profile_prefill_pass(em, torch, reps: int = 5) -> dict:
    """Eager 512-token prefills of the two-layer Llama-7B-shaped model
    (llama7b_model), for rocprofv3 kernel traces of the forward pass."""
    model = llama7b_model(em, torch)
    prompt = [(7 * i + 3) % 32000 for i in range(512)]
    for _ in range(reps):
        model.forward(prompt, 0)
    model.close()
    return {"layers": 2, "prefill_tokens": 512, "calls": reps}


def profile_decode_pass(em, torch, steps: int = 20) -> dict:
    """A 512-token prefill of the two-layer Llama-7B-shaped model, then
    `steps` greedy decode calls (graph replays), for kernel traces."""
    import numpy as np
    model = llama7b_model(em, torch)
    prompt = [(7 * i + 3) % 32000 for i in range(512)]
    tok = int(np.argmax(model.forward(prompt, 0)))
    for i in range(steps):
        tok = int(np.argmax(model.forward(tok, 512 + i)))
    model.close()
    return {"layers": 2, "decode_calls": steps, "context": 512}


def measured_traffic():
    """HBM bytes per headline call from the committed counter summary, or None."""
    path = os.path.join(ROOT, "profiles", "gemv_int8_m1_4096_traffic.json")
    try:
        with open(path) as f:
            return json.load(f)
    except (OSError, ValueError):
        return None


def hbm_ceiling(em, torch, nbytes: int = POOL_MIN_BYTES, reps: int = 5) -> dict:
    """What plain streaming reaches on this GPU, beside the GEMV: a device to
    device copy (the reference's ceiling, bench_cuda.cpp:79-88; bytes read +
    written), the library's read-only stream (em_stream_read) and torch's
    sum, each over a buffer past the 256 MB Infinity Cache, timed with HIP
    events on torch's stream."""
    src = torch.ones(nbytes // 4, device="cuda", dtype=torch.float32)
    dst = torch.empty_like(src)
    sink = torch.zeros(1, device="cuda", dtype=torch.int32)
    out = {}
    for name, op, moved in (("d2d_copy", lambda: dst.copy_(src), 2 * nbytes),
                            ("read_stream", lambda: em.stream_read(src, sink), nbytes),
                            ("read_sum", lambda: src.sum(), nbytes)):
        op()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            op()
        e1.record()
        torch.cuda.synchronize()
        secs = e0.elapsed_time(e1) / 1e3 / reps
        out[name + "_GBps"] = round(moved / secs / 1e9, 1)
    out["buffer_MiB"] = nbytes >> 20
    del src, dst
    return out


def graph_of(torch, fn, count: int):
    """A HIP graph of `count` back-to-back calls fn(i) on a side stream
    (one eager pass first, so nothing allocates during capture)."""
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for i in range(count):
            fn(i)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(count):
            fn(i)
    torch.cuda.synchronize()
    return graph


FLOOR_BLOCKS = (256, 512, 1024, 2048, 4096)
FLOOR_DEPTHS = (4, 8, 16)


def floor_study(em, torch, reps: int = 20) -> dict:
    """What bounds one int8 m = 1 4096^2 call, measured with the bench's method
    (HIP-graph replay of back-to-back dependent launches, HIP events):
      empty     an empty kernel per launch (1, 256 = the GEMV's grid, 1024 workgroups)
      read16    em_probe_read of one 16 MiB pool copy per launch over 38 copies
                (608 MiB, past the Infinity Cache), swept over workgroups,
                loads in flight per thread and access pattern
      read600   the same sweep as one launch over a 600 MiB buffer (the ceiling)
      gemv      em_matmul_q8 (skinny) over the headline's 38-copy quantised
                pool, row-major and unregistered: the split-K GEMV and its slice
                sum (two launches)
      gemv_packed  em_matmul_q8_packed over the same weights in the strip layout"""
    out = {"method": "HIP-graph replay, HIP events on torch's stream; us per launch"}
    copies = 38
    launches = 2 * copies
    emp = {}
    for blocks in (1, 256, 1024):
        g = graph_of(torch, lambda i, b=blocks: em.probe_empty(b), launches)
        secs, _ = time_graph(torch, g, reps, 3)
        emp[str(blocks)] = round(secs / (reps * launches) * 1e6, 3)
        del g
    out["empty_us"] = emp
    progress("floor: empty kernels done")

    mib16 = 16 << 20
    bufs = [torch.randint(-127, 128, (mib16,), dtype=torch.int8, device="cuda")
            for _ in range(copies)]
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    r16 = {}
    for contig in (True, False):
        for blocks in FLOOR_BLOCKS:
            for depth in FLOOR_DEPTHS:
                g = graph_of(torch, lambda i, b=blocks, d=depth, c=contig:
                             em.probe_read(bufs[i % copies], sink, b, d, c), copies)
                secs, _ = time_graph(torch, g, reps, 3)
                us = secs / (reps * copies) * 1e6
                r16[f"{'contig' if contig else 'stride'} b{blocks} d{depth}"] = \
                    {"us": round(us, 3), "GBps": round(mib16 / us / 1e3, 1)}
                del g
    out["read16"] = r16
    best = min(r16.items(), key=lambda kv: kv[1]["us"])
    out["read16_best"] = {"config": best[0], **best[1]}
    progress("floor: 16 MiB reads done")
    del bufs

    big = torch.ones((600 << 20) // 4, dtype=torch.float32, device="cuda")
    r600 = {}
    for contig in (True, False):
        for blocks in FLOOR_BLOCKS:
            for depth in FLOOR_DEPTHS:
                fn = lambda b=blocks, d=depth, c=contig: em.probe_read(big, sink, b, d, c)
                fn()
                torch.cuda.synchronize()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(5):
                    fn()
                e1.record()
                torch.cuda.synchronize()
                us = e0.elapsed_time(e1) * 1e3 / 5
                r600[f"{'contig' if contig else 'stride'} b{blocks} d{depth}"] = \
                    {"us": round(us, 1), "GBps": round((600 << 20) / us / 1e3, 1)}
    out["read600"] = r600
    best = min(r600.items(), key=lambda kv: kv[1]["us"])
    out["read600_best"] = {"config": best[0], **best[1]}
    del big
    progress("floor: 600 MiB reads done")

    pool = Pool(em, torch, True, DIM, DIM, copies, 1000)
    g = torch.Generator(device="cuda")
    g.manual_seed(8)
    A = torch.randn((1, DIM), generator=g, device="cuda", dtype=torch.float32)
    ref = torch.empty((1, DIM), device="cuda")
    em.matmul(A, pool.ws[0], ref, scale=pool.scales[0], kernel="skinny")
    C = torch.zeros((1, DIM), device="cuda")
    g = graph_of(torch, lambda i: em.matmul(A, pool.ws[i % copies], C,
                                            scale=pool.scales[i % copies], kernel="skinny"),
                 copies)
    secs, _ = time_graph(torch, g, reps, 3)
    del g
    us = secs / (reps * copies) * 1e6
    out["gemv"] = {"us": round(us, 3), "GBps": round(gemv_bytes(1, DIM, DIM, True) / us / 1e3, 1)}
    packed = [em.pack_q8(w) for w in pool.ws]
    C = torch.zeros((1, DIM), device="cuda")
    g = graph_of(torch, lambda i: em.matmul_packed(A, packed[i % copies], DIM,
                                                   pool.scales[i % copies], C), copies)
    secs, _ = time_graph(torch, g, reps, 3)
    del g
    us = secs / (reps * copies) * 1e6
    C.zero_()
    em.matmul_packed(A, packed[0], DIM, pool.scales[0], C)
    C2 = torch.zeros_like(C)
    em.matmul_packed(A, packed[0], DIM, pool.scales[0], C2)
    torch.cuda.synchronize()
    bound = (A.abs() @ (pool.ws[0].float().abs() * pool.scales[0])).clamp_min(1e-30)
    out["gemv_packed"] = {"us": round(us, 3),
                          "GBps": round(gemv_bytes(1, DIM, DIM, True) / us / 1e3, 1),
                          "repeat_identical": bool(torch.equal(C, C2)),
                          "max_err_over_abs_bound_vs_product": float(((C - ref).abs() / bound).max())}
    del packed
    del pool
    torch.cuda.synchronize()
    progress("floor: GEMV paths done")
    return out


def floor_study_fp32(em, torch, reps: int = 20) -> dict:
    """What bounds one fp32 m = 1 4096^2 call (the fp32 decode configuration on
    the GPU), with the bench's method (HIP-graph replay of back-to-back
    dependent launches over 10 rotating 64 MiB copies, 640 MiB):
      empty     an empty 256-workgroup launch
      read      em_probe_read of one copy per launch, contiguous chunks or a
                grid stride, by workgroups and loads in flight
      columns   em_probe_read_columns of one copy per launch: each workgroup
                one seg-byte column run of every row of its k slice (the
                layouts a GEMV over row-major weights can give its
                workgroups), by segment, slices and XCD order
      gemv      em_matmul_f32 (skinny): the split-K GEMV and its slice sum"""
    out = {"method": "HIP-graph replay, HIP events on torch's stream; us per launch",
           "matrix": "4096 x 4096 fp32 (64 MiB), 10 copies"}
    copies, rows, row_bytes = 10, DIM, DIM * 4
    nbytes = rows * row_bytes
    g = graph_of(torch, lambda i: em.probe_empty(256), 2 * copies)
    secs, _ = time_graph(torch, g, reps, 3)
    out["empty_us"] = round(secs / (reps * 2 * copies) * 1e6, 3)
    del g
    bufs = [torch.ones((rows, DIM), dtype=torch.float32, device="cuda") for _ in range(copies)]
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")

    def per_launch(fn):
        graph = graph_of(torch, fn, copies)
        secs, _ = time_graph(torch, graph, reps, 3)
        del graph
        us = secs / (reps * copies) * 1e6
        return {"us": round(us, 3), "GBps": round(nbytes / us / 1e3, 1)}

    read = {}
    for contig in (True, False):
        for blocks in FLOOR_BLOCKS:
            for depth in (8, 16):
                read[f"{'contig' if contig else 'stride'} b{blocks} d{depth}"] = per_launch(
                    lambda i, b=blocks, d=depth, c=contig: em.probe_read(bufs[i], sink, b, d, c))
    out["read"] = read
    best = min(read.items(), key=lambda kv: kv[1]["us"])
    out["read_best"] = {"config": best[0], **best[1]}
    progress("floor fp32: contiguous and strided reads done")
    cols = {}
    for seg in (64, 128, 256, 512, 1024):
        groups = row_bytes // seg
        for blocks in (256, 512, 1024):
            slices = blocks // groups
            if slices < 1:
                continue
            for depth in (8, 16):
                for xcd in (False, True):
                    cols[f"seg{seg} slices{slices} b{blocks} d{depth}{' xcd' if xcd else ''}"] = \
                        per_launch(lambda i, sg=seg, sl=slices, d=depth, x=xcd:
                                   em.probe_read_columns(bufs[i], rows, row_bytes, sg, sl, d, x, sink))
    out["columns"] = cols
    best = min(cols.items(), key=lambda kv: kv[1]["us"])
    out["columns_best"] = {"config": best[0], **best[1]}
    by_seg = {}
    for key, v in cols.items():
        seg = key.split()[0]
        if seg not in by_seg or v["us"] < by_seg[seg]["us"]:
            by_seg[seg] = {"config": key, **v}
    out["columns_best_by_segment"] = by_seg
    progress("floor fp32: column reads done")
    del bufs
    pool = Pool(em, torch, False, DIM, DIM, copies, 1000)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(8)
    A = torch.randn((1, DIM), generator=gen, device="cuda", dtype=torch.float32)
    C = torch.zeros((1, DIM), device="cuda")
    graph = graph_of(torch, lambda i: em.matmul(A, pool.ws[i], C, kernel="skinny"), copies)
    secs, _ = time_graph(torch, graph, reps, 3)
    del graph
    us = secs / (reps * copies) * 1e6
    out["gemv"] = {"us": round(us, 3), "GBps": round(gemv_bytes(1, DIM, DIM, False) / us / 1e3, 1),
                   "kernels": "gemv_kernel<float, 1, 4, 16> (64 k slices x 16 column tiles) + "
                              "reduce_slices"}
    pool.close()
    del pool
    torch.cuda.synchronize()
    progress("floor fp32: GEMV done")
    return out


def single_launch_floor(em, torch, reps: int = 20) -> dict:
    """The headline call's floors, with its method (graph replay over 38
    rotating 16 MiB copies): an empty launch, and one launch reading a whole
    copy (em_probe_read, the two best shapes of bench.py --floor)."""
    copies = 38
    g = graph_of(torch, lambda i: em.probe_empty(256), 2 * copies)
    secs, _ = time_graph(torch, g, reps, 3)
    del g
    out = {"empty_us": round(secs / (reps * 2 * copies) * 1e6, 3)}
    mib16 = 16 << 20
    bufs = [torch.randint(-127, 128, (mib16,), dtype=torch.int8, device="cuda")
            for _ in range(copies)]
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    best = None
    for blocks, depth, contig in ((256, 16, True), (512, 8, False)):
        g = graph_of(torch, lambda i, b=blocks, d=depth, c=contig:
                     em.probe_read(bufs[i % copies], sink, b, d, c), copies)
        secs, _ = time_graph(torch, g, reps, 3)
        del g
        us = secs / (reps * copies) * 1e6
        best = us if best is None else min(best, us)
    out["read16_us"] = round(best, 3)
    out["read16_GBps"] = round(mib16 / best / 1e3, 1)
    del bufs
    torch.cuda.synchronize()
    return out


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"





def cpu_baseline(A_dev, q_dev, s_dev, gemm_AB):
    """The reference's matmul_parallel (oracle/_ref) on the host, same inputs."""
    import numpy as np
    import oracle
    ref = oracle.ref()
    if ref is None:
        return None
    threads = 0  # the reference's default pool (hardware_concurrency, thread_pool.cpp)
    A = A_dev.cpu().numpy()
    q = q_dev.cpu().numpy()
    s = s_dev.cpu().numpy()
    # Bounded sample: one warm-up, then the median of up to 2001 reps (a few s).
    one = ref.time_parallel_q8(A, q, s, 1, threads)
    reps = int(max(15, min(2001, 3.0 / max(one, 1e-6)))) | 1
    secs = ref.time_parallel_q8(A, q, s, reps, threads)
    nbytes = gemv_bytes(A.shape[0], q.shape[0], q.shape[1], True)
    out = {"value": nbytes / secs / 1e9, "unit": "GB/s", "cores": ref.pool_size(),
           "kind": "reference",
           "sample": f"int8 GEMV m=1 4096x4096 (one W, no rotation), matmul_parallel, "
                     f"median of {reps} reps after 1 warm-up",
           "ms": secs * 1e3, "compiler": ref.compiler().split("(")[0].strip(),
           "library": os.path.basename(ref.path), "pool_threads": ref.pool_size(),
           "cpu_model": cpu_model(), "nproc": os.cpu_count()}
    if gemm_AB is not None:
        Ah = gemm_AB[0].cpu().numpy()
        Bh = gemm_AB[1].cpu().numpy()
        gs = ref.time_parallel_f32(Ah, Bh, 3, threads)
        out["gemm_fp32_N4096"] = {"ms": gs * 1e3, "GFLOPS": 2 * 4096**3 / gs / 1e9,
                                  "sample": "median of 3 reps (reps_for(4096), bench_matmul.cpp:43-48)"}
    return out


def progress(msg: str) -> None:
    """A stage line on stderr (stdout carries only the result line)."""
    print(f"bench: {msg}", file=sys.stderr, flush=True)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[1])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-extra", action="store_true", help="only the headline workload")
    ap.add_argument("--llama7b-layers", type=int, default=0, metavar="L",
                    help="only time the Llama-7B-shaped forward pass L layers deep (32 for "
                         "the full model; builds ~0.8 GB of host weights per layer) and print "
                         "its JSON line")
    ap.add_argument("--floor-fp32", action="store_true",
                    help="the floor study of the fp32 m = 1 4096^2 call (JSON on stdout)")
    ap.add_argument("--floor", action="store_true",
                    help="only the floor study of the headline call (empty launches, "
                         "16 MiB and 600 MiB read sweeps, single-launch GEMV variants)")
    ap.add_argument("--profile-pass", nargs="?", const="gemv",
                    choices=["gemv", "gemm", "split", "smallm", "proj", "prefill", "decode"],
                    help="eager launches for rocprofv3 --pmc: gemv (calibration copy + "
                         "headline, the default), gemm (fp32 tiled N=4096), split "
                         "(int8 m=512, exact-split), smallm (int8 m=4/16/64), proj (the Llama-7B "
                         "projections at m=512), prefill or decode (Llama-7B-shaped, 2 layers)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one MI355X: every box in this run has one GPU, and the matmul "
              "path has no multi-GPU code (it would shard W by output columns, one slab per "
              "GPU). Run with --gpus 1.", file=sys.stderr)
        return 2

    import torch
    em = load_engine()
    if not torch.cuda.is_available() or not em.available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    if args.llama7b_layers:
        out = {"metric": "Llama-7B-shaped forward pass through em_model", "n_gpus": 1,
               "data": "synthetic: random int8-quantised weights, fixed prompt"}
        for kv in (32, 8):
            t0 = time.perf_counter()
            r = llama7b_model_case(em, torch, n_layers=args.llama7b_layers, n_kv_heads=kv)
            r["wall_s_with_setup"] = round(time.perf_counter() - t0, 1)
            out["mha" if kv == 32 else "gqa8"] = r
            print(json.dumps({"done": "mha" if kv == 32 else "gqa8", **r}), file=sys.stderr,
                  flush=True)
        print(json.dumps(out))
        return 0
    if args.floor:
        print(json.dumps(floor_study(em, torch)))
        return 0
    if args.floor_fp32:
        print(json.dumps(floor_study_fp32(em, torch)))
        return 0
    if args.profile_pass == "gemm":
        print(json.dumps(profile_gemm_pass(em, torch)))
        return 0
    if args.profile_pass == "split":
        print(json.dumps(profile_split_pass(em, torch)))
        return 0
    if args.profile_pass == "smallm":
        print(json.dumps(profile_smallm_pass(em, torch)))
        return 0
    if args.profile_pass == "proj":
        print(json.dumps(profile_proj_pass(em, torch)))
        return 0
    if args.profile_pass == "prefill":
        print(json.dumps(profile_prefill_pass(em, torch)))
        return 0
    if args.profile_pass == "decode":
        print(json.dumps(profile_decode_pass(em, torch)))
        return 0
    if args.profile_pass:
        print(json.dumps(profile_pass(em, torch)))
        return 0

    head, (A1, _) = gemv_case(em, torch, 1, True, args.steps, args.warmup, register=True)
    progress("headline done")
    rowmajor, _ = gemv_case(em, torch, 1, True, max(5, args.steps // 2), 2)
    floor = single_launch_floor(em, torch)
    ceiling = hbm_ceiling(em, torch)
    steps = args.steps
    secs = head["secs"]
    avg_launch_s = secs / head["calls"]
    achieved = head["bytes_per_call"] / avg_launch_s / 1e9
    traffic = measured_traffic()
    read16 = floor["read16_GBps"]
    result = {
        "metric": METRIC,
        "value": round(head["GBps"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": secs / steps * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 (int8 weights widened to fp32; fp32 accumulate)",
        "data": "synthetic: A ~ N(0,1), W ~ N(0,0.02) quantised on the GPU (bit-exact quant.cpp)",
        "config": {"workload": "int8 GEMV m=1, A[1,4096] x Wq[4096,4096] + fp32 scales "
                               "(BASELINE configs[1]) through em_matmul_q8 (matmul_cuda's int8 "
                               "overload) on row-major weights registered at load time "
                               "(em_q8_register, as DeviceQTensor's constructor does: the library "
                               "keeps a strip-layout copy and runs the one-row product in one "
                               "launch); one step = one sweep over "
                               f"{head['copies']} weight copies ({head['pool_MiB']} MiB), "
                               "HIP-graph replay",
                   "m": 1, "k": DIM, "n": DIM, "weight_pool_copies": head["copies"],
                   "pct_of_hbm_peak": round(100 * head["GBps"] / HBM_PEAK_GBS, 2),
                   "unregistered_rowmajor": {
                       "us_per_call": round(rowmajor["us_per_call"], 3),
                       "GBps": round(rowmajor["GBps"], 1),
                       "kernel": "gemv_kernel<int8,1,16,16> + reduce_slices (split-K, two "
                                 "launches)"}},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic["hbm_bytes_per_call"] if traffic else None,
                     "traffic_note": (traffic["note"] if traffic else
                                      "no counter summary in profiles/"),
                     "kernel": "gemv_row_kernel<512,8> (one em_matmul_q8 call over a "
                               "registered matrix: one launch, no split-K partials)",
                     "avg_launch_us": round(avg_launch_s * 1e6, 3),
                     "bytes_per_launch": head["bytes_per_call"],
                     "single_launch_floor_GBps": read16,
                     "frac_of_single_launch_floor": round(achieved / read16, 4),
                     "floor_note": "em_probe_read of one 16 MiB pool copy per launch over 38 "
                                   "copies, graph replay, same run (best of contiguous 256 x 16 "
                                   "and strided 512 x 8): the fastest any one launch reads the "
                                   f"call's bytes; empty launch {floor['empty_us']} us",
                     "achievable_read_GBps": ceiling["read_stream_GBps"],
                     "frac_of_achievable": round(achieved / ceiling["read_stream_GBps"], 4),
                     "achievable_note": "em_stream_read (1024 workgroups, 16 loads in flight, "
                                        "contiguous chunks) over a 600 MiB buffer, same run; "
                                        "device-to-device copy "
                                        f"{ceiling['d2d_copy_GBps']} GB/s read + write"},
    }

    extra = {}
    q_keep = None
    gemm_AB = None
    if not args.no_extra:
        # bench_cuda.cpp:112-144's decode rows, over registered weights as
        # the headline (what DeviceQTensor callers get), with the row-major
        # (unregistered) call beside each.
        for m in (4, 8, 16, 32, 64):
            r, _ = gemv_case(em, torch, m, True, max(5, steps // 2), 2, register=True)
            rr, _ = gemv_case(em, torch, m, True, max(5, steps // 2), 2)
            kname, peak = q8_kernel(m, registered=True)
            t_mfma = r["flops_per_call"] / (peak * 1e12)
            t_hbm = r["bytes_per_call"] / (HBM_PEAK_GBS * 1e9)
            extra[f"int8_gemv_m{m}"] = {"us": round(r["us_per_call"], 3),
                                        "GBps": round(r["GBps"], 1),
                                        "TFLOPS": round(r["flops_per_call"] / r["us_per_call"] / 1e6, 2),
                                        "kernel": kname, "compute_roof_TFLOPS": round(peak, 1),
                                        "bound": "mfma" if t_mfma > t_hbm else "hbm",
                                        "pct_of_roofline": round(100 * max(t_mfma, t_hbm) * 1e6 / r["us_per_call"], 1),
                                        "unregistered_rowmajor_us": round(rr["us_per_call"], 3),
                                        "unregistered_kernel": q8_kernel(m)[0]}
        extra["fp32_decode_4096"] = fp32_decode_table(em, torch, steps)
        extra["fp32_gemv_m1"] = {k: extra["fp32_decode_4096"]["m1"][k]
                                 for k in ("us", "GBps", "pct_of_hbm_peak")}
        progress("fp32 decode table done")
        gemm, gemm_AB = gemm_case(em, torch)
        extra["fp32_gemm_N4096"] = {k: round(v, 3) if isinstance(v, float) else v
                                    for k, v in gemm.items()}
        extra["fp32_gemm_vendor"] = vendor_gemm_case(em, torch)
        progress("gemv and gemm legs done")
        extra["llama7b_layer_int8"] = llama7b_case(em, torch, steps)
        progress("llama7b layer done")
        extra["decode_attention"] = attention_case(em, torch)
        progress("attention done")
        extra["stories15m_forward"] = stories15m_case(em, torch)
        progress("stories15M done")
        extra["checkpoint_load"] = checkpoint_load_case(em, torch)
        progress("checkpoint load done")
        extra["llama7b_model_2layers_int8"] = llama7b_model_case(em, torch)
        extra["llama7b_model_2layers_int8_gqa8"] = llama7b_model_case(em, torch, n_kv_heads=8)
        progress("llama7b models done")
        extra["hbm_ceiling"] = ceiling
        # The reference's own convention (bench_cuda.cpp:41-54): host time of
        # one launch -> synchronize, median of 101, one W (cache-resident).
        pool = Pool(em, torch, True, DIM, DIM, 1, 99)
        C = torch.empty((1, DIM), device="cuda")
        host_s = host_median_convention(em, torch, A1, pool.ws[0], pool.scales[0], C)
        extra["reference_convention_int8_m1"] = {
            "ms": round(host_s * 1e3, 4),
            "GBps_of_B": round(DIM * DIM / host_s / 1e9, 1),
            "note": "host launch->sync median, single W (cache-resident), as bench_cuda.cpp"}
        q_keep = (pool.ws[0], pool.scales[0])
        result["extra"] = extra
        result["config"]["fp32_gemm_N4096_TFLOPS"] = extra["fp32_gemm_N4096"]["TFLOPS"]
        result["config"]["fp32_gemm_pct_of_mfma_peak"] = \
            extra["fp32_gemm_N4096"]["pct_of_fp32_mfma_peak"]

    if not args.no_cpu:
        if q_keep is None:
            pool = Pool(em, torch, True, DIM, DIM, 1, 99)
            q_keep = (pool.ws[0], pool.scales[0])
        cb = cpu_baseline(A1, q_keep[0], q_keep[1], gemm_AB)
        if cb is not None:
            result["cpu_baseline"] = cb

    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
