"""The C ABI without a GPU: it loads, exports every symbol include/*.h
declares, and rejects bad arguments on the host before any HIP call, with
the reference's messages (cuda_matmul.cu:406-422, test_cuda.cpp:277-287)."""
import os
import re

import pytest

from tests import engine

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
em = engine.load()


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "llm_engine_amd.h")).read()
    return sorted(set(re.findall(r"\b(em_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = em.lib()
    names = declared_symbols()
    assert len(names) >= 12
    for name in names:
        assert hasattr(lib, name), name
    assert sorted(em.EXPORTS) == names


def test_exports_match_nm():
    import subprocess
    out = subprocess.run(["nm", "-D", "--defined-only", em.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (em_[a-z0-9_]+)$", out, re.M))
    assert set(declared_symbols()) <= exported


def err(fn):
    with pytest.raises(em.EngineError) as e:
        fn()
    return e.value


def test_skinny_rejects_more_than_8_rows():
    e = err(lambda: em.matmul_f32_raw(9, 2, 2, 16, 16, 16, "skinny"))
    assert e.code == em.EM_EINVAL
    assert "at most 8 rows" in str(e) and "9x2" in str(e) and "2x2" in str(e)


def test_more_than_2_pow_31_elements():
    e = err(lambda: em.matmul_f32_raw(1 << 16, 1 << 16, 1, 16, 16, 16))
    assert e.code == em.EM_EINVAL and "2^31" in str(e)
    e = err(lambda: em.matmul_q8_raw(2, 3, 1 << 30, 16, 16, 16, 16))
    assert e.code == em.EM_EINVAL and "2^31" in str(e)
    # Just below the limit is accepted by the checks (no GPU here: no device).
    e = err(lambda: em.matmul_f32_raw(1, 1, (1 << 31) - 1, 16, 16, 16, "naive"))
    assert e.code == em.EM_ENODEV


def test_unknown_kernel():
    e = err(lambda: em.matmul_f32_raw(1, 1, 1, 16, 16, 16, 7))
    assert e.code == em.EM_EINVAL and "unknown kernel" in str(e)


def test_null_pointers():
    assert err(lambda: em.matmul_f32_raw(2, 3, 4, 16, 16, None)).code == em.EM_EINVAL
    assert err(lambda: em.matmul_f32_raw(2, 3, 4, None, 16, 16)).code == em.EM_EINVAL
    e = err(lambda: em.matmul_q8_raw(2, 3, 4, 16, 16, None, 16))
    assert e.code == em.EM_EINVAL and "scales" in str(e)
    assert err(lambda: em.quantize_q8_raw(3, 3, None, 16, 16)).code == em.EM_EINVAL


def test_empty_products_are_no_ops():
    # m == 0 or n == 0 return before any check that needs a device
    # (cuda_matmul.cu:418), even with null pointers.
    em.matmul_f32_raw(0, 5, 7, None, None, None)
    em.matmul_q8_raw(3, 0, 7, None, None, None, None)
    em.quantize_q8_raw(5, 0, None, None, None)
    em.dequantize_q8_raw(0, 4, None, None, None)


def test_no_device_is_reported():
    if em.available():
        pytest.skip("a GPU is present")
    e = err(lambda: em.matmul_f32_raw(1, 1, 1, 16, 16, 16))
    assert e.code == em.EM_ENODEV
    assert err(em.synchronize).code == em.EM_ENODEV
    assert em.scratch_generation() == 0


def test_noalloc_checks_before_the_gpu():
    # em_matmul_q8_noalloc validates as em_matmul_q8 with the skinny kernel,
    # on the host, before it looks for the device's static scratch.
    e = err(lambda: em.matmul_q8_noalloc_raw(9, 2, 2, 16, 16, 16, 16))
    assert e.code == em.EM_EINVAL and "at most 8 rows" in str(e)
    e = err(lambda: em.matmul_q8_noalloc_raw(2, 3, 4, 16, 16, None, 16))
    assert e.code == em.EM_EINVAL and "scales" in str(e)
    e = err(lambda: em.matmul_q8_noalloc_raw(2, 3, 1 << 30, 16, 16, 16, 16))
    assert e.code == em.EM_EINVAL and "2^31" in str(e)
    em.matmul_q8_noalloc_raw(0, 3, 4, None, None, None, None)  # empty: a no-op
    if not em.available():
        assert err(lambda: em.matmul_q8_noalloc_raw(1, 16, 16, 16, 16, 16, 16)).code == \
            em.EM_ENODEV


def test_skinny_check_precedes_size_check():
    # As in matmul_impl: kernel choice, then the skinny row limit, then 2^31.
    e = err(lambda: em.matmul_f32_raw(9, 1 << 16, 1 << 16, 16, 16, 16, "skinny"))
    assert "at most 8 rows" in str(e)


def test_attention_check_rejects_like_the_reference():
    # test_cuda_attention.cpp:194-210, plus the LDS cap of single_block.
    em = engine.load()
    S = em.AttentionShape

    def rejects(shape, kernel):
        try:
            em.attention_check(shape, kernel)
        except em.InvalidArgument:
            return True
        return False

    assert rejects(S(2, 2, 6, 64, 36, 12, 12), "split")        # head_size % 4
    assert not rejects(S(2, 2, 6, 64, 36, 12, 12), "single_block")
    assert rejects(S(6, 4, 8, 64, 96, 32, 48), "automatic")    # 6 % 4 heads
    assert rejects(S(4, 4, 8, 0, 64, 32, 32), "automatic")     # seq_len 0
    assert rejects(S(4, 1, 128, 20000, 768, 128, 512), "single_block")
    assert not rejects(S(4, 1, 128, 20000, 768, 128, 512), "split")
    assert rejects(S(4, 4, 8, 64, 64, 32, 32), 7)              # unknown kernel
    assert em.attention_scratch_floats(S(4, 4, 8, 64, 64, 32, 32), 3, "single_block") == 0
    assert em.attention_scratch_floats(S(4, 4, 8, 64, 64, 32, 32), 3, "split") > 0


def test_attention_scratch_for_rows_serves_fewer_rows():
    # automatic may split the tile kernel over the context too, and a grid of
    # fewer row tiles takes more chunks, so the size for `rows` must cover
    # every smaller call: it never shrinks as rows grow, and it holds the
    # split tile's (max, sum, output) for each row, head and chunk, with
    # chunks = min(ceil(1024 / (heads * ceil(rows / 16))), ceil(seq_len / 256))
    # wherever that grid has under 512 workgroups and more than one chunk.
    em = engine.load()
    for heads, kv, hs, T in ((32, 8, 128, 4096), (32, 32, 128, 1024), (8, 2, 64, 700),
                             (4, 2, 128, 3000), (6, 6, 48, 256)):
        shape = em.attention_shape(heads, kv, hs, T)
        cut = 5 if T > 512 else 12
        prev = 0
        for rows in range(1, min(T, 600) + 1):
            n = em.attention_scratch_floats(shape, rows, "automatic")
            assert n >= prev, (heads, hs, T, rows)
            prev = n
            tiles = heads * -(-rows // 16)
            if rows > cut and tiles < 512:
                chunks = min(-(-1024 // tiles), -(-T // 256))
                if chunks > 1:
                    assert n >= rows * heads * chunks * (hs + 2), (heads, hs, T, rows)


def test_stream_read_checks_before_the_gpu():
    # Size and alignment are rejected on the host, GPU or not; zero bytes is
    # a no-op.
    em = engine.load()
    L = em.lib()
    assert L.em_stream_read(None, 0, None, None) == em.EM_OK
    assert L.em_stream_read(None, 16, 16, None) == em.EM_EINVAL
    assert L.em_stream_read(16, 24, 16, None) == em.EM_EINVAL
    assert b"multiples of 16" in L.em_last_error()
    assert L.em_stream_read(8, 32, 16, None) == em.EM_EINVAL


def test_packed_layout_checks_before_the_gpu():
    # The strip layout's entry points reject bad shapes and alignment on the
    # host; m == 0 / n == 0 / k == 0 packing are no-ops.
    L = em.lib()
    assert L.em_pack_q8(4, 17, 16, 16, None) == em.EM_EINVAL
    assert b"multiple of 16" in L.em_last_error()
    assert L.em_pack_q8(5, 16, 16, 16, None) == em.EM_EINVAL
    assert b"k of 4" in L.em_last_error()
    assert L.em_pack_q8(0, 16, None, None, None) == em.EM_OK
    assert L.em_pack_q8(4, 16, None, 16, None) == em.EM_EINVAL
    assert L.em_pack_q8(4, 16, 8, 16, None) == em.EM_EINVAL
    assert b"16-byte aligned" in L.em_last_error()
    assert L.em_unpack_q8(4, 20, 16, 16, None) == em.EM_EINVAL
    e = err(lambda: em._check(L.em_matmul_q8_packed(17, 16, 4, 16, 16, 16, 16, 0, None, None)))
    assert e.code == em.EM_EINVAL and "at most 16 rows" in str(e) and "17x4" in str(e)
    # 9 to 16 rows (the 16-row strip kernel) need 16-byte A, C, scales, norm weight.
    e = err(lambda: em._check(L.em_matmul_q8_packed(9, 16, 4, 8, 16, 16, 16, 0, None, None)))
    assert e.code == em.EM_EINVAL and "16-byte aligned" in str(e) and "9x4" in str(e)
    e = err(lambda: em._check(L.em_matmul_q8_packed(9, 16, 4, 16, 16, 16, 16, 0, 4, None)))
    assert e.code == em.EM_EINVAL and "16-byte aligned" in str(e)
    e = err(lambda: em._check(L.em_matmul_q8_packed(1, 20, 4, 16, 16, 16, 16, 0, None, None)))
    assert e.code == em.EM_EINVAL and "multiple of 16" in str(e)
    e = err(lambda: em._check(L.em_matmul_q8_packed(1, 16, 5, 16, 16, 16, 16, 0, None, None)))
    assert e.code == em.EM_EINVAL and "k of 4" in str(e)
    e = err(lambda: em._check(L.em_matmul_q8_packed(1, 16, 4, 16, 8, 16, 16, 0, None, None)))
    assert e.code == em.EM_EINVAL and "aligned" in str(e)
    e = err(lambda: em._check(L.em_matmul_q8_packed(1, 16, 4, 16, 16, None, 16, 0, None, None)))
    assert e.code == em.EM_EINVAL and "null" in str(e)
    assert L.em_matmul_q8_packed(0, 16, 4, None, None, None, None, 0, None, None) == em.EM_OK
    e = err(lambda: em._check(L.em_matmul_q8_packed(1, 1 << 16, 1 << 16, 16, 16, 16, 16, 0,
                                                    None, None)))
    assert "2^31" in str(e)


def test_probes_check_before_the_gpu():
    L = em.lib()
    assert L.em_probe_empty(0, None) == em.EM_EINVAL
    assert L.em_probe_read(16, 64, 16, 256, 5, 0, None) == em.EM_EINVAL
    assert b"depth" in L.em_last_error()
    assert L.em_probe_read(16, 64, 16, 0, 8, 0, None) == em.EM_EINVAL
    # rows, row_bytes, seg_bytes, slices, depth, xcd
    assert L.em_probe_read_columns(16, 4, 1024, 96, 1, 8, 0, 16, None) == em.EM_EINVAL
    assert b"segment" in L.em_last_error()
    assert L.em_probe_read_columns(16, 4, 1000, 64, 1, 8, 0, 16, None) == em.EM_EINVAL
    assert L.em_probe_read_columns(16, 4, 1024, 64, 5, 8, 0, 16, None) == em.EM_EINVAL
    assert L.em_probe_read_columns(16, 4, 1024, 64, 1, 4, 0, 16, None) == em.EM_EINVAL
    assert b"depth" in L.em_last_error()
    assert L.em_probe_read_columns(16, 1 << 20, 4096, 64, 1, 8, 0, 16, None) == em.EM_EINVAL
    assert L.em_probe_read_columns(16, 0, 1024, 64, 1, 8, 0, 16, None) == em.EM_OK


def test_q8_register_checks_before_the_gpu():
    L = em.lib()
    assert L.em_q8_register(None, 4, 16, None) == em.EM_EINVAL
    assert L.em_q8_register(None, 0, 16, None) == em.EM_OK
    assert L.em_q8_register(16, 1 << 16, 1 << 16, None) == em.EM_EINVAL
    # A shape the strip layout cannot hold stays row-major: nothing registered.
    assert L.em_q8_register(16, 4, 20, None) == em.EM_OK
    assert L.em_q8_registered(16, 4, 20) == 0
    assert L.em_q8_register(8, 4, 16, None) == em.EM_OK
    assert L.em_q8_registered(8, 4, 16) == 0
    # A shape it can hold needs the GPU.
    assert L.em_q8_register(16, 4, 16, None) == em.EM_ENODEV
    assert L.em_q8_registered(16, 4, 16) == 0
    assert L.em_q8_unregister(16) == em.EM_OK
