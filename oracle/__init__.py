"""CPU oracle for the matmul hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg import this package, and only as the checker (or, for bench.py, as the
timed CPU baseline). The product library never loads it.

Two libraries sit behind it:

* ``liboracle.so`` -- the C restatement in ``oracle.c`` (quant.cpp:6-36,
  matmul.cpp:205-217, ops.cpp:8-26 of the reference).
* ``_ref/libref_v{3,4}.so`` -- the reference's own ``matmul.cpp``,
  ``quant.cpp``, ``thread_pool.cpp`` and ``ops.cpp`` compiled from source by
  ``oracle/Makefile`` (amdclang++ -O3), behind ``ref_shim.cpp``. Present in
  the build container and shipped prebuilt to the GPU box; ``ref()`` returns
  None where it is missing.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))

_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_i8p = ctypes.POINTER(ctypes.c_int8)
_sz = ctypes.c_size_t


def build(reference: str = "/root/reference") -> None:
    """Compile liboracle.so and, where the reference sources exist, _ref/."""
    subprocess.run(["make", "-s", "-C", HERE, f"REF={reference}", "all"], check=True)


def _ptr(a: np.ndarray, t):
    return a.ctypes.data_as(t)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


class Oracle:
    """ctypes front of liboracle.so; every function takes and returns numpy arrays."""

    def __init__(self, path: Optional[str] = None):
        path = path or os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run oracle.build() (make -C oracle)")
        lib = ctypes.CDLL(path)
        lib.orc_quantize_q8.argtypes = [_sz, _sz, _f32p, _i8p, _f32p]
        lib.orc_dequantize.argtypes = [_sz, _sz, _i8p, _f32p, _f32p]
        lib.orc_matmul_naive.argtypes = [_sz, _sz, _sz, _f32p, _f32p, _f32p]
        lib.orc_rmsnorm.argtypes = [_sz, _sz, _f32p, _f32p, ctypes.c_float, _f32p]
        lib.orc_matmul_fused.argtypes = [_sz, _sz, _sz, _f32p, _f32p, _i8p, _f32p, _f32p,
                                         ctypes.c_int, _f32p]
        lib.orc_abs_bound.argtypes = [_sz, _sz, _sz, _f32p, _f32p, _f64p]
        lib.orc_matmul_f64.argtypes = [_sz, _sz, _sz, _f32p, _f32p, _f64p]
        lib.orc_argmax.argtypes = [_sz, _f32p]
        lib.orc_argmax.restype = _sz
        lib.orc_attention.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, _sz, _sz, _f32p,
                                      _sz, _f32p, _f32p, _sz, _f64p, _sz]
        self.lib = lib

    def quantize_q8(self, B):
        B = _f32(B)
        k, n = B.shape
        q = np.empty((k, n), np.int8)
        s = np.empty((n,), np.float32)
        self.lib.orc_quantize_q8(k, n, _ptr(B, _f32p), _ptr(q, _i8p), _ptr(s, _f32p))
        return q, s

    def dequantize(self, q, scale):
        q = np.ascontiguousarray(q, np.int8)
        scale = _f32(scale)
        out = np.empty(q.shape, np.float32)
        self.lib.orc_dequantize(q.shape[0], q.shape[1], _ptr(q, _i8p), _ptr(scale, _f32p),
                                _ptr(out, _f32p))
        return out

    def matmul_naive(self, A, B):
        A, B = _f32(A), _f32(B)
        m, k = A.shape
        n = B.shape[1]
        assert B.shape[0] == k
        C = np.empty((m, n), np.float32)
        self.lib.orc_matmul_naive(m, n, k, _ptr(A, _f32p), _ptr(B, _f32p), _ptr(C, _f32p))
        return C

    def rmsnorm(self, x, w, eps: float = 1e-5):
        x, w = _f32(x), _f32(w)
        y = np.empty(x.shape, np.float32)
        self.lib.orc_rmsnorm(x.shape[0], x.shape[1], _ptr(x, _f32p), _ptr(w, _f32p), eps,
                             _ptr(y, _f32p))
        return y

    def matmul_fused(self, A, B=None, Bq=None, scale=None, w=None, C0=None):
        """C = [C0 +] rmsnorm(A, w) x B', B' = B or dequantize(Bq, scale)."""
        A = _f32(A)
        m, k = A.shape
        n = (Bq if B is None else B).shape[1]
        C = np.zeros((m, n), np.float32) if C0 is None else _f32(C0).copy()
        Bp = _ptr(_f32(B), _f32p) if B is not None else None
        if Bq is not None:
            Bq = np.ascontiguousarray(Bq, np.int8)
            scale = _f32(scale)
        wp = None
        if w is not None:
            w = _f32(w)
            wp = _ptr(w, _f32p)
        self.lib.orc_matmul_fused(m, n, k, _ptr(A, _f32p), Bp,
                                  _ptr(Bq, _i8p) if Bq is not None else None,
                                  _ptr(scale, _f32p) if Bq is not None else None,
                                  wp, int(C0 is not None), _ptr(C, _f32p))
        return C

    def abs_bound(self, A, B):
        A, B = _f32(A), _f32(B)
        m, k = A.shape
        n = B.shape[1]
        out = np.empty((m, n), np.float64)
        self.lib.orc_abs_bound(m, n, k, _ptr(A, _f32p), _ptr(B, _f32p), _ptr(out, _f64p))
        return out

    def matmul_f64(self, A, B):
        A, B = _f32(A), _f32(B)
        m, k = A.shape
        n = B.shape[1]
        out = np.empty((m, n), np.float64)
        self.lib.orc_matmul_f64(m, n, k, _ptr(A, _f32p), _ptr(B, _f32p), _ptr(out, _f64p))
        return out

    def argmax(self, x) -> int:
        x = _f32(x).ravel()
        return int(self.lib.orc_argmax(x.size, _ptr(x, _f32p)))

    def attention(self, n_heads, n_kv_heads, head_size, rows, pos, q, kc, vc):
        """Double-precision causal attention; q is rows x q_stride, the caches
        positions x kv_stride; returns rows x (n_heads * head_size) float64."""
        q, kc, vc = _f32(q), _f32(kc), _f32(vc)
        dim = n_heads * head_size
        out = np.zeros((rows, dim), np.float64)
        self.lib.orc_attention(n_heads, n_kv_heads, head_size, rows, pos, _ptr(q, _f32p),
                               q.shape[1], _ptr(kc, _f32p), _ptr(vc, _f32p), kc.shape[1],
                               _ptr(out, _f64p), dim)
        return out


def _cpu_has_avx512() -> bool:
    try:
        with open("/proc/cpuinfo") as f:
            flags = set()
            for line in f:
                if line.startswith("flags"):
                    flags = set(line.split(":", 1)[1].split())
                    break
    except OSError:
        return False
    return {"avx512f", "avx512bw", "avx512cd", "avx512dq", "avx512vl"} <= flags


class Ref:
    """ctypes front of the reference's own CPU code (oracle/_ref)."""

    def __init__(self, path: str):
        self.path = path
        lib = ctypes.CDLL(path)
        lib.ref_last_error.restype = ctypes.c_char_p
        lib.ref_pool_size.restype = ctypes.c_uint
        lib.ref_quantize_q8.argtypes = [_sz, _sz, _f32p, _i8p, _f32p]
        lib.ref_dequantize.argtypes = [_sz, _sz, _i8p, _f32p, _f32p]
        lib.ref_matmul_f32.argtypes = [ctypes.c_int, _sz, _sz, _sz, _f32p, _f32p, _f32p,
                                       ctypes.c_uint]
        lib.ref_matmul_parallel_q8.argtypes = [_sz, _sz, _sz, _f32p, _i8p, _f32p, _f32p,
                                               ctypes.c_uint]
        lib.ref_shape_error.argtypes = [_sz, _sz, _sz, _sz]
        lib.ref_rmsnorm.argtypes = [_sz, _sz, _f32p, _f32p, ctypes.c_float, _f32p]
        lib.ref_time_parallel_f32.argtypes = [_sz, _sz, _sz, _f32p, _f32p, ctypes.c_int,
                                              ctypes.c_uint]
        lib.ref_time_parallel_f32.restype = ctypes.c_double
        lib.ref_time_parallel_q8.argtypes = [_sz, _sz, _sz, _f32p, _i8p, _f32p, ctypes.c_int,
                                             ctypes.c_uint]
        lib.ref_time_parallel_q8.restype = ctypes.c_double
        self.lib = lib

    def _check(self, rc: int):
        if rc:
            raise ValueError(self.lib.ref_last_error().decode())

    def compiler(self) -> str:
        p = os.path.join(os.path.dirname(self.path), "COMPILER.txt")
        return open(p).read().strip() if os.path.exists(p) else "unknown"

    def pool_size(self) -> int:
        return int(self.lib.ref_pool_size())

    def quantize_q8(self, B):
        B = _f32(B)
        k, n = B.shape
        q = np.empty((k, n), np.int8)
        s = np.empty((n,), np.float32)
        self._check(self.lib.ref_quantize_q8(k, n, _ptr(B, _f32p), _ptr(q, _i8p), _ptr(s, _f32p)))
        return q, s

    def dequantize(self, q, scale):
        q = np.ascontiguousarray(q, np.int8)
        scale = _f32(scale)
        out = np.empty(q.shape, np.float32)
        self._check(self.lib.ref_dequantize(q.shape[0], q.shape[1], _ptr(q, _i8p),
                                            _ptr(scale, _f32p), _ptr(out, _f32p)))
        return out

    def matmul(self, A, B, which: str = "parallel", threads: int = 0):
        A, B = _f32(A), _f32(B)
        m, k = A.shape
        n = B.shape[1]
        C = np.empty((m, n), np.float32)
        code = {"naive": 0, "blocked": 1, "parallel": 2}[which]
        self._check(self.lib.ref_matmul_f32(code, m, n, k, _ptr(A, _f32p), _ptr(B, _f32p),
                                            _ptr(C, _f32p), threads))
        return C

    def matmul_q8(self, A, q, scale, threads: int = 0):
        A = _f32(A)
        q = np.ascontiguousarray(q, np.int8)
        scale = _f32(scale)
        m, k = A.shape
        n = q.shape[1]
        C = np.empty((m, n), np.float32)
        self._check(self.lib.ref_matmul_parallel_q8(m, n, k, _ptr(A, _f32p), _ptr(q, _i8p),
                                                    _ptr(scale, _f32p), _ptr(C, _f32p), threads))
        return C

    def shape_error(self, ar, ac, br, bc) -> str:
        rc = self.lib.ref_shape_error(ar, ac, br, bc)
        return self.lib.ref_last_error().decode() if rc else ""

    def rmsnorm(self, x, w, eps: float = 1e-5):
        x, w = _f32(x), _f32(w)
        y = np.empty(x.shape, np.float32)
        self._check(self.lib.ref_rmsnorm(x.shape[0], x.shape[1], _ptr(x, _f32p), _ptr(w, _f32p),
                                         eps, _ptr(y, _f32p)))
        return y

    def time_parallel_f32(self, A, B, reps: int, threads: int = 0) -> float:
        A, B = _f32(A), _f32(B)
        return float(self.lib.ref_time_parallel_f32(A.shape[0], B.shape[1], A.shape[1],
                                                    _ptr(A, _f32p), _ptr(B, _f32p), reps, threads))

    def time_parallel_q8(self, A, q, scale, reps: int, threads: int = 0) -> float:
        A = _f32(A)
        q = np.ascontiguousarray(q, np.int8)
        scale = _f32(scale)
        return float(self.lib.ref_time_parallel_q8(A.shape[0], q.shape[1], A.shape[1],
                                                   _ptr(A, _f32p), _ptr(q, _i8p),
                                                   _ptr(scale, _f32p), reps, threads))


_oracle: Optional[Oracle] = None
_ref: Optional[Ref] = None
_ref_probed = False


def oracle() -> Oracle:
    global _oracle
    if _oracle is None:
        _oracle = Oracle()
    return _oracle


def ref() -> Optional[Ref]:
    """The compiled reference for this host's CPU, or None if not built."""
    global _ref, _ref_probed
    if not _ref_probed:
        _ref_probed = True
        name = "libref_v4.so" if _cpu_has_avx512() else "libref_v3.so"
        path = os.path.join(HERE, "_ref", name)
        if os.path.exists(path):
            _ref = Ref(path)
    return _ref


# ---- the reference's CPU model (oracle/_ref/libref_model.so) ----------------

class RefCheckpoint:
    """A checkpoint loaded by the reference's own loader (load_checkpoint,
    model.cpp:115-163): config plus weights in the CPU model's layout."""

    NAMES = ("token_embedding", "rms_final", "wcls")
    LAYER_NAMES = ("rms_att", "wqkv", "wo", "rms_ffn", "w13", "w2")

    def __init__(self, lib, path: Optional[str] = None, config: Optional[dict] = None,
                 weights: Optional[dict] = None):
        """From a llama2.c file (the reference's loader), or from `config` and
        `weights` already in the CPU model's layout."""
        self.lib = lib
        if path is not None:
            self.h = lib.ref_ckpt_load(path.encode())
        else:
            keys = ("dim", "hidden_dim", "n_layers", "n_heads", "n_kv_heads", "vocab_size",
                    "seq_len")
            cfg = (ctypes.c_size_t * 7)(*(int(config[k]) for k in keys))
            keep = []

            def p(a):
                a = np.ascontiguousarray(a, np.float32)
                keep.append(a)
                return a.ctypes.data

            ptrs = [p(lw[k]) for lw in weights["layers"] for k in self.LAYER_NAMES]
            arr = (ctypes.c_void_p * len(ptrs))(*ptrs)
            self.h = lib.ref_ckpt_new(cfg, p(weights["token_embedding"]), arr,
                                      p(weights["rms_final"]), p(weights["wcls"]))
        if not self.h:
            raise ValueError(lib.ref_model_error().decode())
        cfg = (ctypes.c_size_t * 7)()
        lib.ref_ckpt_config(self.h, cfg)
        keys = ("dim", "hidden_dim", "n_layers", "n_heads", "n_kv_heads", "vocab_size", "seq_len")
        self.config = dict(zip(keys, (int(x) for x in cfg)))

    def array(self, name: str, layer: int = 0) -> np.ndarray:
        n = int(self.lib.ref_ckpt_array(self.h, name.encode(), layer, None, 0))
        out = np.empty((n,), np.float32)
        self.lib.ref_ckpt_array(self.h, name.encode(), layer, _ptr(out, _f32p), n)
        return out

    def weights(self) -> dict:
        c = self.config
        D, H, V = c["dim"], c["hidden_dim"], c["vocab_size"]
        KV = c["n_kv_heads"] * (D // c["n_heads"])
        shapes = {"wqkv": (D, D + 2 * KV), "wo": (D, D), "w13": (D, 2 * H), "w2": (H, D)}
        w = {"token_embedding": self.array("token_embedding").reshape(V, D),
             "rms_final": self.array("rms_final"),
             "wcls": self.array("wcls").reshape(D, V), "layers": []}
        for l in range(c["n_layers"]):
            w["layers"].append({k: (self.array(k, l).reshape(shapes[k]) if k in shapes
                                    else self.array(k, l)) for k in self.LAYER_NAMES})
        return w

    def rope_tables(self):
        c = self.config
        half = c["dim"] // c["n_heads"] // 2
        cos = np.empty((c["seq_len"] * half,), np.float32)
        sin = np.empty_like(cos)
        self.lib.ref_rope_tables(self.h, _ptr(cos, _f32p), _ptr(sin, _f32p))
        return cos, sin

    def __del__(self):
        if getattr(self, "h", None):
            self.lib.ref_ckpt_free(self.h)
            self.h = None


class RefTransformer:
    """The reference's CPU Transformer (model.h:79-108) over a RefCheckpoint."""

    def __init__(self, lib, ckpt: RefCheckpoint, q8: bool):
        self.lib, self.vocab = lib, ckpt.config["vocab_size"]
        self.h = lib.ref_model_new(ckpt.h, int(q8))
        if not self.h:
            raise ValueError(lib.ref_model_error().decode())

    def run(self, tokens, pos: int, single: bool = False) -> np.ndarray:
        """prefill(tokens, pos), or forward(tokens[0], pos) when single."""
        t = np.ascontiguousarray(tokens, np.int32)
        out = np.empty((self.vocab,), np.float32)
        rc = self.lib.ref_model_run(self.h, t.ctypes.data_as(ctypes.POINTER(ctypes.c_int)),
                                    t.size, pos, int(single), _ptr(out, _f32p))
        if rc == 1:
            raise IndexError(self.lib.ref_model_error().decode())
        if rc:
            raise ValueError(self.lib.ref_model_error().decode())
        return out

    def __del__(self):
        if getattr(self, "h", None):
            self.lib.ref_model_free(self.h)
            self.h = None


_ref_model_lib = None


def ref_model_lib():
    """ctypes handle of oracle/_ref/libref_model.so, or None if not built."""
    global _ref_model_lib
    if _ref_model_lib is None:
        path = os.path.join(HERE, "_ref", "libref_model.so")
        if not os.path.exists(path):
            return None
        lib = ctypes.CDLL(path)
        vp = ctypes.c_void_p
        lib.ref_model_error.restype = ctypes.c_char_p
        lib.ref_ckpt_load.restype = vp
        lib.ref_ckpt_load.argtypes = [ctypes.c_char_p]
        lib.ref_ckpt_free.argtypes = [vp]
        lib.ref_ckpt_new.restype = vp
        lib.ref_ckpt_new.argtypes = [ctypes.POINTER(ctypes.c_size_t), vp, ctypes.POINTER(vp), vp,
                                     vp]
        lib.ref_ckpt_config.argtypes = [vp, ctypes.POINTER(ctypes.c_size_t)]
        lib.ref_ckpt_array.restype = _sz
        lib.ref_ckpt_array.argtypes = [vp, ctypes.c_char_p, _sz, _f32p, _sz]
        lib.ref_model_new.restype = vp
        lib.ref_model_new.argtypes = [vp, ctypes.c_int]
        lib.ref_model_free.argtypes = [vp]
        lib.ref_model_run.argtypes = [vp, ctypes.POINTER(ctypes.c_int), _sz, _sz, ctypes.c_int,
                                      _f32p]
        lib.ref_rope_tables.argtypes = [vp, _f32p, _f32p]
        _ref_model_lib = lib
    return _ref_model_lib
