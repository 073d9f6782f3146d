"""em_model_load without a GPU: every rejection of the reference's loader
(load_checkpoint, model.cpp:61-90,115-163; tests/test_model.cpp:248-261)
happens on the host before any HIP call, with the reference's message and
EM_EIO (std::runtime_error in the C++ layer). A file the loader accepts gets
as far as the device check."""
import os

import numpy as np
import pytest

import oracle
from tests import e2e_model, engine

em = engine.load()
ref = oracle.ref_model_lib()


def write(tmp_path, name="model.bin", drop=0, patch=None, **kw):
    m = e2e_model.fixture_model(kw.pop("heads", 4), kw.pop("kv_heads", 4), kw.pop("shared", True),
                                seed=1, **kw)
    path = str(tmp_path / name)
    e2e_model.write_raw(path, m)
    if patch is not None:
        with open(path, "r+b") as f:
            h = np.frombuffer(f.read(28), np.int32).copy()
            for i, v in patch.items():
                h[i] = v
            f.seek(0)
            f.write(h.tobytes())
    if drop:
        size = os.path.getsize(path)
        with open(path, "r+b") as f:
            f.truncate(size - drop)
    return path


def load_error(path):
    """The error em_model_load gives; where the reference's own loader
    (oracle/_ref, compiled from model.cpp) rejects the file too, the two
    messages must be the same text."""
    with pytest.raises(em.EngineError) as e:
        em.Model.load(path)
    if ref is not None and e.value.code == em.EM_EIO:
        with pytest.raises(ValueError) as r:
            oracle.RefCheckpoint(ref, path)
        assert str(r.value) == str(e.value)
    return e.value


def test_missing_file(tmp_path):
    path = str(tmp_path / "model.bin.missing")
    e = load_error(path)
    assert e.code == em.EM_EIO and str(e) == f"cannot open checkpoint {path}"
    assert isinstance(e, RuntimeError)


def test_short_file(tmp_path):
    # test_model.cpp:252-254: a file 4 bytes short.
    path = write(tmp_path, drop=4)
    e = load_error(path)
    assert e.code == em.EM_EIO and "header implies" in str(e)
    size = os.path.getsize(path)
    assert str(e) == f"checkpoint {path} is {size} bytes, header implies {size + 4}"


def test_long_file(tmp_path):
    path = write(tmp_path)
    with open(path, "ab") as f:
        f.write(b"\0" * 8)
    e = load_error(path)
    assert e.code == em.EM_EIO and "header implies" in str(e)


def test_kv_heads_not_a_divisor(tmp_path):
    # test_model.cpp:256-259: 4 query heads don't split into groups of 3.
    path = write(tmp_path, patch={4: 3})
    e = load_error(path)
    assert e.code == em.EM_EIO
    assert str(e) == (f"checkpoint {path}: dim must split into even-sized heads, and query heads "
                      "into whole groups per kv head")


def test_odd_head_size(tmp_path):
    path = write(tmp_path, heads=16, kv_heads=16)  # dim 16 / 16 heads: head size 1
    e = load_error(path)
    assert e.code == em.EM_EIO and "even-sized heads" in str(e)


@pytest.mark.parametrize("field,value", [(0, 0), (1, -40), (3, 0), (6, -8), (5, 0)])
def test_bad_header_field(tmp_path, field, value):
    path = write(tmp_path, patch={field: value})
    e = load_error(path)
    assert e.code == em.EM_EIO
    assert str(e) == f"checkpoint {path}: bad header field {field} = {value}"


def test_truncated_header(tmp_path):
    path = str(tmp_path / "tiny.bin")
    with open(path, "wb") as f:
        f.write(np.arange(3, dtype=np.int32).tobytes())
    e = load_error(path)
    assert e.code == em.EM_EIO and str(e) == f"checkpoint {path} ended early"


def test_valid_file_passes_the_checks(tmp_path):
    # Tied and untied classifiers both pass the header and size checks: with
    # no GPU the load stops at the device check, with one it loads.
    for shared in (True, False):
        path = write(tmp_path, name=f"ok{int(shared)}.bin", shared=shared, heads=4, kv_heads=2)
        if em.available():
            em.Model.load(path).close()
        else:
            assert load_error(path).code == em.EM_ENODEV


def test_shape_the_attention_kernels_cannot_run(tmp_path):
    # A header the CPU loader accepts but the forward pass cannot run is
    # EM_EINVAL, as em_model_create rejects it.
    path = write(tmp_path, heads=1, kv_heads=1, dim=1026, hidden=8)  # head size 1026
    e = load_error(path)
    assert e.code == em.EM_EINVAL, str(e)
