"""GPU quantize_q8 / dequantize against the reference, bit for bit.

The golden fixtures hold the reference's own quant.cpp output (compiled from
source in the build container): full bytes for small matrices, SHA-256
digests for the config shapes."""
import hashlib
import json
import os

import numpy as np
import pytest

import oracle
from tests import engine, inputs
from tests.test_oracle import golden_quant_small

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
em = engine.load()
orc = oracle.oracle()
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def gpu_quant(B):
    q, s = em.quantize_q8(torch.from_numpy(np.ascontiguousarray(B)).cuda())
    torch.cuda.synchronize()
    return q.cpu().numpy(), s.cpu().numpy()


def test_small_fixtures_bit_exact():
    for name, (B, q_ref, s_ref) in golden_quant_small().items():
        q, s = gpu_quant(B)
        assert np.array_equal(q, q_ref), name
        assert np.array_equal(s.view(np.uint32), s_ref.view(np.uint32)), name


@pytest.mark.parametrize("name", ["w_4096x4096", "w2_11008x4096", "s15m_wqkv_288x864",
                                  "s15m_cls_288x32000", "cls_4096x32000"])
def test_config_shapes_match_reference_digest(name):
    d = json.load(open(os.path.join(GOLDEN, "quant_digests.json")))[name]
    B = inputs.normal(tuple(d["shape"]), d["std"], d["seed"])
    assert sha(B) == d["B"]
    q, s = gpu_quant(B)
    assert sha(q) == d["q"], f"{name}: q bytes differ from quant.cpp"
    assert sha(s) == d["scale"], f"{name}: scales differ from quant.cpp"


def test_edge_matrices():
    cases = {
        "empty_rows": np.zeros((0, 5), np.float32),
        "one_col": inputs.normal((300, 1), 1.0, 3),
        "zeros": np.zeros((7, 9), np.float32),
        "odd": inputs.uniform((33, 257), -3.0, 3.0, 4),
        "ties": np.array([[127.0], [0.5], [-0.5], [2.5], [-2.5], [126.5], [-126.5]], np.float32),
    }
    for name, B in cases.items():
        q, s = gpu_quant(B)
        q2, s2 = orc.quantize_q8(B)
        assert np.array_equal(q, q2), name
        assert np.array_equal(s.view(np.uint32), s2.view(np.uint32)), name


def test_dequantize_matches_oracle():
    q, s = orc.quantize_q8(inputs.normal((130, 70), 0.02, 5))
    out = em.dequantize_q8(torch.from_numpy(q).cuda(), torch.from_numpy(s).cuda())
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), orc.dequantize(q, s))


def test_repeat_is_bit_identical():
    B = inputs.normal((512, 1000), 0.02, 8)
    a = gpu_quant(B)
    b = gpu_quant(B)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
