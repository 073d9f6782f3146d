"""Writes the golden fixtures under tests/golden/ from the reference's own code.

Run in the build container, where oracle/_ref (the reference's matmul.cpp,
quant.cpp, thread_pool.cpp and ops.cpp compiled from /root/reference by
oracle/Makefile) exists:

    python tests/golden/make_golden.py

Inputs come from tests/inputs.py (seeded, numpy-version independent), so
a fixture stores seeds, a SHA-256 of each input and the reference's outputs.
Large shapes store only digests of the outputs.

Fixtures:
  quant_small.npz    quantize_q8 (quant.cpp:6-28) of small matrices, full q and scale,
                     including the 37x21 round-trip matrix of tests/test_quant.cpp:34-37
  quant_digests.json quantize_q8 of the config shapes (4096^2, Llama-7B, classifier):
                     SHA-256 of input, q bytes and scale bytes
  matmul_small.npz   matmul_naive / matmul_parallel (fp32 and int8) on the edge
                     shapes of tests/test_matmul.cpp:89-100 and tests/test_quant.cpp:73-75
  rmsnorm.npz        rmsnorm (ops.cpp:8-26) on seeded rows
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from tests import inputs  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


# The 37x21 matrix of test_quant.cpp:34-37, made with this build's generator:
# U(-2, 2), row 5 scaled by (c + 1) per column, column 4 all zero.
def round_trip_matrix() -> np.ndarray:
    B = inputs.uniform((37, 21), -2.0, 2.0, seed=3)
    B[5, :] *= np.arange(1, 22, dtype=np.float32)
    B[:, 4] = 0.0
    return B


# Columns whose products B * inv land exactly on k + 0.5: absmax 127 gives
# scale 1 and inv 1, so lround's half-away-from-zero rule shows.
def ties_matrix() -> np.ndarray:
    col = np.array([127.0, 0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 126.5, -126.5, 63.5], np.float32)
    B = np.stack([col, -col, col * 0.0, col / 2.0], axis=1)
    return B.astype(np.float32)


QUANT_SMALL = [  # name, shape, std/lo-hi, seed
    ("u_1x1", (1, 1), 11),
    ("u_5x3", (5, 3), 12),
    ("u_64x16", (64, 16), 13),
    ("n_288x300", (288, 300), 14),
    ("n_33x257", (33, 257), 15),
]

QUANT_BIG = [  # config shapes: W ~ N(0, 0.02)
    ("w_4096x4096", (4096, 4096), 1001),
    ("w1_4096x11008", (4096, 11008), 1002),
    ("w2_11008x4096", (11008, 4096), 1003),
    ("cls_4096x32000", (4096, 32000), 1004),
    ("s15m_wqkv_288x864", (288, 864), 1005),
    ("s15m_cls_288x32000", (288, 32000), 1006),
]

# (m, k, n): test_matmul.cpp:89-100 and test_quant.cpp:73-75 edge shapes.
MATMUL_SHAPES = [
    (1, 1, 1), (1, 17, 1), (3, 5, 7), (4, 256, 16), (5, 257, 17), (63, 300, 65),
    (64, 255, 128), (130, 70, 103), (20, 513, 33), (1, 300, 1030), (2, 64, 411),
    (3, 1000, 70), (4, 4097, 33), (5, 200, 300), (8, 513, 249), (1, 0, 5), (6, 0, 3),
]


def main() -> None:
    ref = oracle.ref()
    if ref is None:
        raise SystemExit("oracle/_ref is not built; run make -C oracle first")
    print("reference build:", ref.path, "|", ref.compiler())

    # quant_small.npz
    out = {}
    mats = {"round_trip_37x21": round_trip_matrix(), "ties_10x4": ties_matrix()}
    for name, shape, seed in QUANT_SMALL:
        if name.startswith("u_"):
            mats[name] = inputs.uniform(shape, -1.0, 1.0, seed)
        else:
            mats[name] = inputs.normal(shape, 0.02, seed)
    seeds = {name: seed for name, _, seed in QUANT_SMALL}
    for name, B in mats.items():
        q, s = ref.quantize_q8(B)
        if B.size <= 4096 or name not in seeds:
            out[f"{name}__B"] = B
        else:  # regenerable: keep the seed and a digest of the input
            out[f"{name}__seed"] = np.int64(seeds[name])
            out[f"{name}__shaB"] = np.bytes_(sha(B))
        out[f"{name}__q"] = q
        out[f"{name}__scale"] = s
    np.savez_compressed(os.path.join(HERE, "quant_small.npz"), **out)
    print("quant_small.npz:", len(mats), "matrices")

    # quant_digests.json
    digests = {}
    for name, shape, seed in QUANT_BIG:
        B = inputs.normal(shape, 0.02, seed)
        q, s = ref.quantize_q8(B)
        digests[name] = {"shape": list(shape), "std": 0.02, "seed": seed, "B": sha(B),
                         "q": sha(q), "scale": sha(s)}
        print(" ", name, digests[name]["q"][:16])
    with open(os.path.join(HERE, "quant_digests.json"), "w") as f:
        json.dump(digests, f, indent=1, sort_keys=True)

    # matmul_small.npz
    out = {}
    for i, (m, k, n) in enumerate(MATMUL_SHAPES):
        A = inputs.uniform((m, k), -1.0, 1.0, 2000 + i)
        B = inputs.uniform((k, n), -1.0, 1.0, 3000 + i)
        Bq_src = inputs.uniform((k, n), -0.5, 0.5, 4000 + i)
        q, s = ref.quantize_q8(Bq_src)
        key = f"{m}x{k}x{n}"
        out[f"{key}__seedA"] = np.int64(2000 + i)
        out[f"{key}__seedB"] = np.int64(3000 + i)
        out[f"{key}__seedQ"] = np.int64(4000 + i)
        out[f"{key}__shaA"] = np.bytes_(sha(A))
        out[f"{key}__shaB"] = np.bytes_(sha(B))
        out[f"{key}__naive"] = ref.matmul(A, B, "naive")
        out[f"{key}__parallel"] = ref.matmul(A, B, "parallel")
        out[f"{key}__parallel_q8"] = ref.matmul_q8(A, q, s)
    np.savez_compressed(os.path.join(HERE, "matmul_small.npz"), **out)
    print("matmul_small.npz:", len(MATMUL_SHAPES), "shapes")

    # rmsnorm.npz
    x = inputs.normal((7, 288), 1.0, 77)
    w = inputs.uniform((288,), 0.5, 1.5, 78)
    x[3, :] = 0.0  # an all-zero row: eps keeps it finite
    np.savez_compressed(os.path.join(HERE, "rmsnorm.npz"), x=x, w=w, y=ref.rmsnorm(x, w),
                        y_eps0=ref.rmsnorm(x[:3], w, 0.0))
    print("rmsnorm.npz written")

    with open(os.path.join(HERE, "PROVENANCE.txt"), "w") as f:
        f.write("Generated by tests/golden/make_golden.py from oracle/_ref\n")
        f.write(f"library: {os.path.basename(ref.path)}\n")
        f.write(f"compiler: {ref.compiler()}\n")
        f.write("sources: /root/reference/src/{matmul,quant,thread_pool,ops}.cpp\n")


if __name__ == "__main__":
    main()
