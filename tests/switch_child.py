"""Child process of test_gpu_switches.py: runs one switch's check with the
environment the parent set (the library reads these switches once per
process). Prints "ok" and exits 0 when the check holds."""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402
import torch  # noqa: E402

import oracle  # noqa: E402
from tests import engine, inputs  # noqa: E402

em = engine.load()
orc = oracle.oracle()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def within_bound(got, A, q, s):
    want = orc.matmul_fused(A, Bq=q, scale=s)
    bound = orc.abs_bound(A, orc.dequantize(q, s))
    assert np.all(np.abs(got.astype(np.float64) - want) <= 1e-4 * bound + 1e-30)


def main(mode: str) -> None:
    k, n = 4096, 4096
    q, s = orc.quantize_q8(inputs.normal((k, n), 0.02, 401))
    qd, sd = dev(q), dev(s)
    rows = {m: inputs.normal((m, k), 1.0, 402 + m) for m in (1, 4, 12)}
    plain = {m: host(em.matmul(dev(A), qd, scale=sd)).copy() for m, A in rows.items()}
    em.register_q8(qd)
    try:
        reg = {m: host(em.matmul(dev(A), qd, scale=sd)).copy() for m, A in rows.items()}
        P = em.pack_q8(qd)
        packed = {m: host(em.matmul_packed(dev(A), P, n, sd)).copy() for m, A in rows.items()}
        if mode == "strip_copy_off":
            # No copy kept: every registered product is the row-major one.
            assert not em.registered_q8(qd)
            for m in rows:
                assert np.array_equal(reg[m], plain[m]), m
        elif mode == "decode_mfma_off":
            # The copy is kept, one row and 9-16 rows still run over it; 2-8
            # rows go back to the row-major kernels.
            assert em.registered_q8(qd)
            assert np.array_equal(reg[1], packed[1])
            assert np.array_equal(reg[12], packed[12])
            assert np.array_equal(reg[4], plain[4])
        else:
            raise SystemExit(f"unknown mode {mode}")
        for m, A in rows.items():
            within_bound(reg[m], A, q, s)
    finally:
        em.unregister_q8(qd)
    print("ok", flush=True)


if __name__ == "__main__":
    main(sys.argv[1])
