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

EM_OK, EM_EINVAL, EM_EDEVICE, EM_ENODEV, EM_ERANGE, EM_EIO = 0, 1, 2, 3, 4, 5
KERNELS = {"automatic": 0, "naive": 1, "tiled": 2, "tiled_split": 3, "skinny": 4}
STREAM_PER_THREAD = 2

# Every symbol include/llm_engine_amd.h declares.
EXPORTS = (
    "em_last_error", "em_available", "em_synchronize", "em_scratch_generation",
    "em_malloc", "em_free", "em_memcpy_h2d", "em_memcpy_d2h",
    "em_matmul_f32", "em_matmul_q8", "em_matmul_q8_noalloc", "em_quantize_q8", "em_dequantize_q8", "em_stream_read",
    "em_probe_empty", "em_probe_read", "em_probe_read_columns",
    "em_pack_q8", "em_unpack_q8", "em_matmul_q8_packed",
    "em_q8_register", "em_q8_unregister", "em_q8_registered",
    "em_attention_check", "em_attention_scratch_floats", "em_attention",
    "em_model_create", "em_model_destroy", "em_model_forward",
    "em_model_load", "em_model_config_get", "em_model_read_weight",
)
ATTN_KERNELS = {"automatic": 0, "single_block": 1, "split": 2}


class ModelConfig(ctypes.Structure):
    """em_model_config (the reference's Config, model.h:11-22)."""
    _fields_ = [(k, ctypes.c_size_t) for k in ("dim", "hidden_dim", "n_layers", "n_heads",
                                                "n_kv_heads", "vocab_size", "seq_len")]


class LayerWeights(ctypes.Structure):
    """em_layer_weights (the reference's LayerWeights, model.h:29-36)."""
    _fields_ = [(k, ctypes.c_void_p) for k in ("rms_att", "wqkv", "wo", "rms_ffn", "w13", "w2")]


class AttentionShape(ctypes.Structure):
    """em_attention_shape (the reference's AttentionShape, cuda_attention.h:8-13)."""
    _fields_ = [("n_heads", ctypes.c_int), ("n_kv_heads", ctypes.c_int),
                ("head_size", ctypes.c_int), ("seq_len", ctypes.c_int),
                ("q_stride", ctypes.c_size_t), ("kv_stride", ctypes.c_size_t),
                ("out_stride", ctypes.c_size_t)]


class EngineError(Exception):
    def __init__(self, code: int, msg: str):
        super().__init__(msg)
        self.code = code


class InvalidArgument(EngineError, ValueError):
    """EM_EINVAL: the reference's std::invalid_argument."""


class DeviceError(EngineError, RuntimeError):
    """EM_EDEVICE / EM_ENODEV: the reference's std::runtime_error."""


class OutOfRange(EngineError, IndexError):
    """EM_ERANGE: the reference's std::out_of_range (check_feed)."""


class CheckpointError(EngineError, RuntimeError):
    """EM_EIO: the reference's std::runtime_error from load_checkpoint."""


_sz = ctypes.c_size_t
_vp = ctypes.c_void_p
_lib: Optional[ctypes.CDLL] = None


def build() -> str:
    """Compile the library for gfx950 (hipcc); see build.py."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("_em_build", os.path.join(HERE, "build.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.build_library()


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is not built: run python llm-engine_amd/build.py")
        # PyTorch ships its own HIP runtime under the same soname
        # (libamdhip64.so.7). Loaded first, it is the one this library binds
        # to, so one process has one runtime; loaded after this library
        # brought in /opt/rocm's, torch finds no device.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
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
        L.em_matmul_q8_noalloc.argtypes = [_sz, _sz, _sz, _vp, _vp, _vp, _vp, ctypes.c_int, _vp,
                                           _vp]
        L.em_quantize_q8.argtypes = [_sz, _sz, _vp, _vp, _vp, _vp]
        L.em_dequantize_q8.argtypes = [_sz, _sz, _vp, _vp, _vp, _vp]
        L.em_stream_read.argtypes = [_vp, _sz, _vp, _vp]
        L.em_pack_q8.argtypes = [_sz, _sz, _vp, _vp, _vp]
        L.em_unpack_q8.argtypes = [_sz, _sz, _vp, _vp, _vp]
        L.em_matmul_q8_packed.argtypes = [_sz, _sz, _sz, _vp, _vp, _vp, _vp, ctypes.c_int, _vp,
                                          _vp]
        L.em_q8_register.argtypes = [_vp, _sz, _sz, _vp]
        L.em_q8_unregister.argtypes = [_vp]
        L.em_q8_registered.argtypes = [_vp, _sz, _sz]
        L.em_probe_empty.argtypes = [ctypes.c_uint, _vp]
        L.em_probe_read.argtypes = [_vp, _sz, _vp, ctypes.c_uint, ctypes.c_uint, ctypes.c_int, _vp]
        L.em_probe_read_columns.argtypes = [_vp, ctypes.c_uint, ctypes.c_uint, ctypes.c_uint,
                                            ctypes.c_uint, ctypes.c_uint, ctypes.c_int, _vp, _vp]
        shp = ctypes.POINTER(AttentionShape)
        L.em_attention_check.argtypes = [shp, ctypes.c_int]
        L.em_attention_scratch_floats.argtypes = [shp, _sz, ctypes.c_int]
        L.em_attention_scratch_floats.restype = _sz
        L.em_attention.argtypes = [shp, _sz, _vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_int, _vp]
        L.em_model_create.argtypes = [ctypes.POINTER(ModelConfig), _vp,
                                      ctypes.POINTER(LayerWeights), _vp, _vp, ctypes.c_int,
                                      ctypes.POINTER(_vp)]
        L.em_model_destroy.argtypes = [_vp]
        L.em_model_forward.argtypes = [_vp, _vp, _sz, _sz, _vp]
        L.em_model_load.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.POINTER(_vp)]
        L.em_model_config_get.argtypes = [_vp, ctypes.POINTER(ModelConfig)]
        L.em_model_read_weight.argtypes = [_vp, ctypes.c_char_p, _sz, _vp, _sz]
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
    if rc == EM_ERANGE:
        raise OutOfRange(rc, msg)
    if rc == EM_EIO:
        raise CheckpointError(rc, msg)
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


def matmul_q8_noalloc_raw(m, n, k, A, B, scale, C, accumulate=False, rms_weight=None,
                          stream=None) -> None:
    _check(lib().em_matmul_q8_noalloc(m, n, k, A, B, scale, C, int(bool(accumulate)),
                                      rms_weight, stream))


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


def matmul_q8_noalloc(A, B, C, scale, *, accumulate=False, rms_weight=None, stream=None):
    """em_matmul_q8_noalloc: C = [C +] rmsnorm?(A) x dequantize(B, scale) for
    m <= 8 rows through the skinny GEMV, its split-K partials in the
    library's static per-GPU scratch (nothing allocated). C is given."""
    import torch
    m, k = A.shape
    n = B.shape[1]
    if B.shape[0] != k or tuple(C.shape) != (m, n):
        raise InvalidArgument(EM_EINVAL, f"matmul_q8_noalloc: shapes differ (A is {m}x{k}, "
                                         f"B is {B.shape[0]}x{n}, C is {tuple(C.shape)})")
    rw = _dev(rms_weight, torch.float32) if rms_weight is not None else None
    matmul_q8_noalloc_raw(m, n, k, _dev(A, torch.float32), _dev(B, torch.int8),
                          _dev(scale, torch.float32), _dev(C, torch.float32), accumulate, rw,
                          _stream_ptr(stream))
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


def stream_read(buf, sink, stream=None) -> None:
    """One read-only pass over a device tensor (its bytes a multiple of 16)
    on torch's current stream; sink is a 1-element int32 device tensor."""
    _check(lib().em_stream_read(buf.data_ptr(), buf.numel() * buf.element_size(),
                                sink.data_ptr(), _stream_ptr(stream)))


def pack_q8(q, stream=None):
    """The strip layout (em_pack_q8) of a row-major int8 device matrix [k, n]:
    a new int8 tensor of the same size, 1-D."""
    import torch
    k, n = q.shape
    packed = torch.empty((k * n,), dtype=torch.int8, device=q.device)
    _check(lib().em_pack_q8(k, n, _dev(q, torch.int8), packed.data_ptr(), _stream_ptr(stream)))
    return packed


def unpack_q8(packed, k: int, n: int, stream=None):
    """Row-major [k, n] int8 from the strip layout (em_unpack_q8)."""
    import torch
    q = torch.empty((k, n), dtype=torch.int8, device=packed.device)
    _check(lib().em_unpack_q8(k, n, _dev(packed, torch.int8), q.data_ptr(), _stream_ptr(stream)))
    return q


def matmul_packed(A, packed, n: int, scale, C=None, *, accumulate=False, rms_weight=None,
                  stream=None):
    """C = [C +] rmsnorm?(A) x B with B in the strip layout (em_matmul_q8_packed)."""
    import torch
    m, k = A.shape
    if C is None:
        C = torch.empty((m, n), dtype=torch.float32, device=A.device)
    rw = _dev(rms_weight, torch.float32) if rms_weight is not None else None
    _check(lib().em_matmul_q8_packed(m, n, k, _dev(A, torch.float32), _dev(packed, torch.int8),
                                     _dev(scale, torch.float32), _dev(C, torch.float32),
                                     int(bool(accumulate)), rw, _stream_ptr(stream)))
    return C


# data_ptr -> the finalizer that unregisters it when its tensor is collected.
_registered: dict = {}


def _unregister_ptr(ptr: int) -> None:
    _registered.pop(ptr, None)
    if _lib is not None:
        _lib.em_q8_unregister(ctypes.c_void_p(ptr))


def register_q8(q, stream=None) -> None:
    """em_q8_register: the library keeps a strip-layout copy of row-major int8
    weights q [k, n]; matmul() over q then runs decode-shaped products in one
    launch. The registration ends with unregister_q8(q) or when q is
    collected, whichever comes first, so torch's caching allocator cannot
    hand q's address to other bytes while a copy of the old ones is kept."""
    import torch
    import weakref
    k, n = q.shape
    ptr = _dev(q, torch.int8)
    _check(lib().em_q8_register(ptr, k, n, _stream_ptr(stream)))
    old = _registered.pop(ptr, None)
    if old is not None:
        old.detach()
    _registered[ptr] = weakref.finalize(q, _unregister_ptr, ptr)


def unregister_q8(q) -> None:
    fin = _registered.pop(q.data_ptr(), None)
    if fin is not None:
        fin.detach()
    _check(lib().em_q8_unregister(q.data_ptr()))


def registered_q8(q) -> bool:
    k, n = q.shape
    return bool(lib().em_q8_registered(q.data_ptr(), k, n))


def probe_empty(blocks: int, stream=None) -> None:
    """em_probe_empty: one empty launch of `blocks` workgroups."""
    _check(lib().em_probe_empty(blocks, _stream_ptr(stream)))


def probe_read_columns(buf, rows: int, row_bytes: int, seg_bytes: int, slices: int, depth: int,
                       xcd: bool, sink, stream=None) -> None:
    """em_probe_read_columns over a device tensor holding rows x row_bytes."""
    _check(lib().em_probe_read_columns(buf.data_ptr(), rows, row_bytes, seg_bytes, slices, depth,
                                       int(bool(xcd)), sink.data_ptr(), _stream_ptr(stream)))


def probe_read(buf, sink, blocks: int, depth: int, contiguous: bool, stream=None) -> None:
    """em_probe_read over a device tensor's bytes."""
    _check(lib().em_probe_read(buf.data_ptr(), buf.numel() * buf.element_size(), sink.data_ptr(),
                               blocks, depth, int(bool(contiguous)), _stream_ptr(stream)))


def dequantize_q8(q, scale, stream=None):
    import torch
    rows, cols = q.shape
    out = torch.empty((rows, cols), dtype=torch.float32, device=q.device)
    dequantize_q8_raw(rows, cols, _dev(q, torch.int8), _dev(scale, torch.float32),
                      _dev(out, torch.float32), _stream_ptr(stream))
    return out


# ---- attention ---------------------------------------------------------------

def attention_shape(n_heads, n_kv_heads, head_size, seq_len, q_stride=None, kv_stride=None,
                    out_stride=None) -> AttentionShape:
    """The model's geometry by default: q rows strided like its qkv buffer."""
    dim, kv = n_heads * head_size, n_kv_heads * head_size
    return AttentionShape(n_heads, n_kv_heads, head_size, seq_len,
                          dim + 2 * kv if q_stride is None else q_stride,
                          kv if kv_stride is None else kv_stride,
                          dim if out_stride is None else out_stride)


def attention_check(shape: AttentionShape, kernel="automatic") -> None:
    _check(lib().em_attention_check(ctypes.byref(shape), ATTN_KERNELS.get(kernel, kernel)))


def attention_scratch_floats(shape: AttentionShape, rows: int, kernel="automatic") -> int:
    return int(lib().em_attention_scratch_floats(ctypes.byref(shape), rows,
                                                 ATTN_KERNELS.get(kernel, kernel)))


def attention(shape: AttentionShape, rows: int, pos_dev, q, key_cache, value_cache, out=None,
              scratch=None, kernel="automatic", stream=None):
    """em_attention on torch tensors: pos_dev is a 1-element int32 device tensor."""
    import torch
    if out is None:
        out = torch.empty((rows, shape.out_stride), dtype=torch.float32, device=q.device)
    if scratch is None:
        n = attention_scratch_floats(shape, rows, kernel)
        scratch = torch.empty((max(1, n),), dtype=torch.float32, device=q.device)
    _check(lib().em_attention(ctypes.byref(shape), rows, _dev(pos_dev, torch.int32),
                              _dev(q, torch.float32), _dev(key_cache, torch.float32),
                              _dev(value_cache, torch.float32), _dev(out, torch.float32),
                              _dev(scratch, torch.float32), ATTN_KERNELS.get(kernel, kernel),
                              _stream_ptr(stream)))
    return out


# ---- the forward pass --------------------------------------------------------

class Model:
    """em_model: the device-resident forward pass (the reference's
    CudaTransformer, cuda_model.h:24-89). `weights` holds numpy fp32 arrays in
    the CPU model's layout: token_embedding (vocab x dim), rms_final (dim),
    wcls (dim x vocab) and `layers`, a list of dicts with rms_att, wqkv, wo,
    rms_ffn, w13, w2 (projections in x out)."""

    @classmethod
    def load(cls, path: str, q8: bool = False) -> "Model":
        """em_model_load: a llama2.c v0 checkpoint straight onto the GPU."""
        self = cls.__new__(cls)
        handle = _vp()
        _check(lib().em_model_load(os.fsencode(path), int(bool(q8)), ctypes.byref(handle)))
        self.h = handle.value
        cfg = ModelConfig()
        _check(lib().em_model_config_get(self.h, ctypes.byref(cfg)))
        self.config = {k: int(getattr(cfg, k)) for k, _ in ModelConfig._fields_}
        self.q8 = bool(q8)
        self._keep = []
        return self

    def weight(self, name: str, layer: int = 0):
        """em_model_read_weight: the stored array (numpy), fp32, or int8 for an
        int8 model's projections ("<name>.scale" for their scales)."""
        import numpy as np
        c = self.config
        D, H, V = c["dim"], c["hidden_dim"], c["vocab_size"]
        KV = c["n_kv_heads"] * (D // c["n_heads"])
        shapes = {"token_embedding": (V, D), "rms_final": (D,), "wcls": (D, V), "rms_att": (D,),
                  "rms_ffn": (D,), "wqkv": (D, D + 2 * KV), "wo": (D, D), "w13": (D, 2 * H),
                  "w2": (H, D)}
        base = name.split(".")[0]
        shape = shapes[base]
        if name.endswith(".scale"):
            out = np.empty((shape[1],), np.float32)
        elif self.q8 and base in ("wcls", "wqkv", "wo", "w13", "w2"):
            out = np.empty(shape, np.int8)
        else:
            out = np.empty(shape, np.float32)
        _check(lib().em_model_read_weight(self.h, name.encode(), layer, out.ctypes.data,
                                          out.nbytes))
        return out

    def __init__(self, config: dict, weights: dict, q8: bool = False):
        import numpy as np
        self.config = dict(config)
        self.q8 = bool(q8)
        self._keep = []

        def host(a):
            a = np.ascontiguousarray(a, np.float32)
            self._keep.append(a)
            return a.ctypes.data

        cfg = ModelConfig(**{k: int(config[k]) for k, _ in ModelConfig._fields_})
        layers = (LayerWeights * len(weights["layers"]))()
        for i, lw in enumerate(weights["layers"]):
            layers[i] = LayerWeights(*(host(lw[k]) for k, _ in LayerWeights._fields_))
        handle = _vp()
        _check(lib().em_model_create(ctypes.byref(cfg), host(weights["token_embedding"]), layers,
                                     host(weights["rms_final"]), host(weights["wcls"]),
                                     int(bool(q8)), ctypes.byref(handle)))
        self._keep = []  # the library has its own copies
        self.h = handle.value

    def forward(self, tokens, pos: int):
        """Logits (vocab,) after feeding tokens at [pos, pos + len(tokens))."""
        import numpy as np
        t = np.ascontiguousarray(np.atleast_1d(tokens), np.int32)
        out = np.empty((int(self.config["vocab_size"]),), np.float32)
        _check(lib().em_model_forward(self.h, t.ctypes.data, t.size, pos, out.ctypes.data))
        return out

    def close(self) -> None:
        if getattr(self, "h", None):
            lib().em_model_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()
