"""Python front of libllm_engine_amd.so, the MI355X matmul hot path.

A thin ctypes binding of the C ABI in include/llm_engine_amd.h, plus torch
helpers that pass device tensors' data pointers and torch's current stream.
There is no fallback: if the HIP library is missing, loading raises.

The directory name has a hyphen, so load it by path:

    import importlib.util, os
    spec = importlib.util.spec_from_file_location(
        "llm_engine_amd", os.path.join(ROOT, "llm-engine_amd", "__init__.py"))
    em = importlib.util.module_from_spec(spec); spec.loader.exec_module(em)
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libllm_engine_amd.so")

EM_OK, EM_EINVAL, EM_EDEVICE, EM_ENODEV = 0, 1, 2, 3
KERNELS = {"automatic": 0, "naive": 1, "tiled": 2, "tiled_split": 3, "skinny": 4}
STREAM_PER_THREAD = 2

# Every symbol include/llm_engine_amd.h declares.
EXPORTS = (
    "em_last_error", "em_available", "em_synchronize", "em_scratch_generation",
    "em_malloc", "em_free", "em_memcpy_h2d", "em_memcpy_d2h",
    "em_matmul_f32", "em_matmul_q8", "em_quantize_q8", "em_dequantize_q8",
)


class EngineError(Exception):
    def __init__(self, code: int, msg: str):
        super().__init__(msg)
        self.code = code


class InvalidArgument(EngineError, ValueError):
    """EM_EINVAL: the reference's std::invalid_argument."""


class DeviceError(EngineError, RuntimeError):
    """EM_EDEVICE / EM_ENODEV: the reference's std::runtime_error."""


_sz = ctypes.c_size_t
_vp = ctypes.c_void_p
_lib: Optional[ctypes.CDLL] = None


def build() -> str:
    """Compile the library for gfx950 (hipcc); see build.py."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("_em_build", os.path.join(HERE, "build.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    path = mod.build_library()
    mod.build_cpp_tests()
    return path


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is not built: run python llm-engine_amd/build.py")
        L = ctypes.CDLL(LIB_PATH)
        L.em_last_error.restype = ctypes.c_char_p
        L.em_available.restype = ctypes.c_int
        L.em_synchronize.restype = ctypes.c_int
        L.em_scratch_generation.restype = _sz
        L.em_malloc.argtypes = [ctypes.POINTER(_vp), _sz]
        L.em_free.argtypes = [_vp]
        L.em_memcpy_h2d.argtypes = [_vp, _vp, _sz]
        L.em_memcpy_d2h.argtypes = [_vp, _vp, _sz]
        L.em_matmul_f32.argtypes = [_sz, _sz, _sz, _vp, _vp, _vp, ctypes.c_int, ctypes.c_int,
                                    _vp, _vp]
        L.em_matmul_q8.argtypes = [_sz, _sz, _sz, _vp, _vp, _vp, _vp, ctypes.c_int,
                                   ctypes.c_int, _vp, _vp]
        L.em_quantize_q8.argtypes = [_sz, _sz, _vp, _vp, _vp, _vp]
        L.em_dequantize_q8.argtypes = [_sz, _sz, _vp, _vp, _vp, _vp]
        for name in EXPORTS:
            getattr(L, name).restype = getattr(L, name).restype or ctypes.c_int
        _lib = L
    return _lib


def _check(rc: int) -> None:
    if rc == EM_OK:
        return
    msg = lib().em_last_error().decode()
    if rc == EM_EINVAL:
        raise InvalidArgument(rc, msg)
    raise DeviceError(rc, msg)


def available() -> bool:
    return bool(lib().em_available())


def synchronize() -> None:
    _check(lib().em_synchronize())


def scratch_generation() -> int:
    return int(lib().em_scratch_generation())


def kernel_code(kernel) -> int:
    return KERNELS[kernel] if isinstance(kernel, str) else int(kernel)


# ---- raw entry points (integer device pointers) ----------------------------

def matmul_f32_raw(m, n, k, A, B, C, kernel="automatic", accumulate=False, rms_weight=None,
                   stream=None) -> None:
    _check(lib().em_matmul_f32(m, n, k, A, B, C, kernel_code(kernel), int(bool(accumulate)),
                               rms_weight, stream))


def matmul_q8_raw(m, n, k, A, B, scale, C, kernel="automatic", accumulate=False,
                  rms_weight=None, stream=None) -> None:
    _check(lib().em_matmul_q8(m, n, k, A, B, scale, C, kernel_code(kernel),
                              int(bool(accumulate)), rms_weight, stream))


def quantize_q8_raw(rows, cols, B, q, scale, stream=None) -> None:
    _check(lib().em_quantize_q8(rows, cols, B, q, scale, stream))


def dequantize_q8_raw(rows, cols, q, scale, out, stream=None) -> None:
    _check(lib().em_dequantize_q8(rows, cols, q, scale, out, stream))


# ---- torch helpers -----------------------------------------------------------

def _stream_ptr(stream) -> Optional[int]:
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return int(s.cuda_stream) or None


def _dev(t, dtype) -> int:
    import torch
    if not t.is_cuda or t.dtype != dtype or not t.is_contiguous():
        raise InvalidArgument(EM_EINVAL, f"expected a contiguous {dtype} device tensor")
    return t.data_ptr()


def matmul(A, B, C=None, *, scale=None, kernel="automatic", accumulate=False, rms_weight=None,
           stream=None):
    """C = [C +] rmsnorm?(A) x B on torch's current stream. B fp32 or int8 (+ scale)."""
    import torch
    m, k = A.shape
    if B.shape[0] != k:
        raise InvalidArgument(EM_EINVAL, f"matmul_cuda: inner dimensions differ (A is {m}x{k}, "
                                         f"B is {B.shape[0]}x{B.shape[1]})")
    n = B.shape[1]
    if C is None:
        C = torch.empty((m, n), dtype=torch.float32, device=A.device)
    rw = _dev(rms_weight, torch.float32) if rms_weight is not None else None
    s = _stream_ptr(stream)
    if B.dtype == torch.int8:
        matmul_q8_raw(m, n, k, _dev(A, torch.float32), _dev(B, torch.int8),
                      _dev(scale, torch.float32), _dev(C, torch.float32), kernel, accumulate, rw, s)
    else:
        matmul_f32_raw(m, n, k, _dev(A, torch.float32), _dev(B, torch.float32),
                       _dev(C, torch.float32), kernel, accumulate, rw, s)
    return C


def quantize_q8(B, stream=None):
    """(q int8 [k, n], scale fp32 [n]) of a device fp32 matrix, on the GPU."""
    import torch
    rows, cols = B.shape
    q = torch.empty((rows, cols), dtype=torch.int8, device=B.device)
    scale = torch.empty((cols,), dtype=torch.float32, device=B.device)
    quantize_q8_raw(rows, cols, _dev(B, torch.float32), _dev(q, torch.int8),
                    _dev(scale, torch.float32), _stream_ptr(stream))
    return q, scale


def dequantize_q8(q, scale, stream=None):
    import torch
    rows, cols = q.shape
    out = torch.empty((rows, cols), dtype=torch.float32, device=q.device)
    dequantize_q8_raw(rows, cols, _dev(q, torch.int8), _dev(scale, torch.float32),
                      _dev(out, torch.float32), _stream_ptr(stream))
    return out
