"""numpy front end of the CPU oracle — TEST INFRASTRUCTURE ONLY.

Loads ``liblinear_oracle.so`` (built from ``linear_oracle.c`` by ``make`` in
this directory).  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module; the product
(the HIP library and its bindings) never does.

Each wrapper names the reference function it restates; see
``linear_oracle.h`` for the pinning of each one.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# INFER_ORACLE_LIBRARY names another build of the oracle (its sanitizer
# build, which is never built on demand); by default the in-tree build.
_LIB_PATH = os.environ.get("INFER_ORACLE_LIBRARY") or os.path.join(_HERE, "liblinear_oracle.so")
_lib = None


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc, OpenMP)."""
    if os.environ.get("INFER_ORACLE_LIBRARY"):
        if not os.path.exists(_LIB_PATH):
            raise FileNotFoundError(_LIB_PATH)
        return _LIB_PATH
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-B" if force else "all", "-C", _HERE],
                       check=True, stdout=subprocess.DEVNULL)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        p = ctypes.c_void_p
        i = ctypes.c_int
        lib.orc_f32_to_bf16.argtypes = [ctypes.c_float]
        lib.orc_f32_to_bf16.restype = ctypes.c_uint16
        lib.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
        lib.orc_bf16_to_f32.restype = ctypes.c_float
        lib.orc_f32_to_bf16_array.argtypes = [p, p, ctypes.c_size_t]
        lib.orc_bf16_to_f32_array.argtypes = [p, p, ctypes.c_size_t]
        lib.orc_linear_fp32.argtypes = [p, p, p, p, i, i, i]
        lib.orc_linear_fp32_batch.argtypes = [p, p, p, p, i, i, i, i]
        lib.orc_argmax.argtypes = [p, i]
        lib.orc_argmax.restype = i
        lib.orc_dequant_w8a16.argtypes = [p, p, i, i, i, p, i]
        lib.orc_dequant_w8a16.restype = i
        lib.orc_w8a16_reference.argtypes = [p, p, i, p, p, p, p, i, i, i, i]
        lib.orc_w8a16_reference.restype = i
        lib.orc_bf16_linear_reference.argtypes = [p, p, p, p, i, i, i, i]
        lib.orc_lm_head.argtypes = [p, p, i, i, p, p, i]
        lib.orc_lm_head.restype = i
        lib.orc_default_threads.restype = i
        _lib = lib
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return None if a is None else np.ascontiguousarray(a, dtype=dtype)


def default_threads() -> int:
    return _load().orc_default_threads()


def f32_to_bf16(values) -> np.ndarray:
    """export_model.py:123-131 (RNE, NaN quieted); returns uint16 words."""
    a = _c(values, np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    _load().orc_f32_to_bf16_array(_ptr(a), _ptr(out), a.size)
    return out


def bf16_to_f32(words) -> np.ndarray:
    """export_model.py:134-136."""
    a = _c(words, np.uint16)
    out = np.empty(a.shape, dtype=np.float32)
    _load().orc_bf16_to_f32_array(_ptr(a), _ptr(out), a.size)
    return out


def linear_fp32(weight, bias, x, threads: int = 0) -> np.ndarray:
    """cpu_ops.cpp:23-30: y = W x (+ b) in FP32."""
    w = _c(weight, np.float32)
    xx = _c(x, np.float32)
    b = _c(bias, np.float32)
    n, k = w.shape
    assert xx.shape == (k,)
    out = np.empty(n, dtype=np.float32)
    _load().orc_linear_fp32(_ptr(w), _ptr(b), _ptr(xx), _ptr(out), n, k, threads)
    return out


def linear_fp32_batch(weight, bias, x, threads: int = 0) -> np.ndarray:
    """cpu_ops.cpp:108-123: Y = X W^T (+ b) in FP32."""
    w = _c(weight, np.float32)
    xx = _c(x, np.float32)
    b = _c(bias, np.float32)
    n, k = w.shape
    m = xx.shape[0]
    assert xx.shape == (m, k)
    out = np.empty((m, n), dtype=np.float32)
    _load().orc_linear_fp32_batch(_ptr(w), _ptr(b), _ptr(xx), _ptr(out), m, n,
                                  k, threads)
    return out


def argmax(values) -> int:
    """cpu_ops.cpp:175-177: first index of the maximum."""
    a = _c(values, np.float32)
    return int(_load().orc_argmax(_ptr(a), a.size))


def dequant_w8a16(q, scales_bf16, group_size: int = 64,
                  threads: int = 0) -> np.ndarray:
    """Exact FP32 dequantization q * s[n, k // group]."""
    if group_size <= 0:
        raise ValueError("bad group_size")
    qq = _c(q, np.int8)
    s = _c(scales_bf16, np.uint16)
    n, k = qq.shape
    assert s.shape == (n, -(-k // group_size))
    out = np.empty((n, k), dtype=np.float32)
    rc = _load().orc_dequant_w8a16(_ptr(qq), _ptr(s), group_size, n, k,
                                   _ptr(out), threads)
    if rc != 0:
        raise ValueError("bad group_size")
    return out


def w8a16_reference(q, scales_bf16, group_size, bias_bf16, x_bf16,
                    threads: int = 0):
    """test_cuda.cpp:492-517.  Returns (fp32 sums, bf16 words), [M, N]."""
    qq = _c(q, np.int8)
    s = _c(scales_bf16, np.uint16)
    b = _c(bias_bf16, np.uint16)
    xx = _c(x_bf16, np.uint16)
    if xx.ndim == 1:
        xx = xx.reshape(1, -1)
    n, k = qq.shape
    m = xx.shape[0]
    out32 = np.empty((m, n), dtype=np.float32)
    out16 = np.empty((m, n), dtype=np.uint16)
    rc = _load().orc_w8a16_reference(_ptr(qq), _ptr(s), group_size, _ptr(b),
                                     _ptr(xx), _ptr(out32), _ptr(out16), m, n,
                                     k, threads)
    if rc != 0:
        raise ValueError("bad group_size")
    return out32, out16


def bf16_linear_reference(w_bf16, bias_bf16, x_bf16,
                          threads: int = 0) -> np.ndarray:
    """test_cuda.cpp:474-490 on BF16 operands; FP32 output [M, N]."""
    w = _c(w_bf16, np.uint16)
    b = _c(bias_bf16, np.uint16)
    xx = _c(x_bf16, np.uint16)
    if xx.ndim == 1:
        xx = xx.reshape(1, -1)
    n, k = w.shape
    m = xx.shape[0]
    out = np.empty((m, n), dtype=np.float32)
    _load().orc_bf16_linear_reference(_ptr(w), _ptr(b), _ptr(xx), _ptr(out), m,
                                      n, k, threads)
    return out


def lm_head(e_bf16, h_bf16, threads: int = 0):
    """qwen2.cpp:421-424 CPU step.  Returns (fp32 logits, bf16 logits, argmax)."""
    e = _c(e_bf16, np.uint16)
    h = _c(h_bf16, np.uint16)
    v, k = e.shape
    out32 = np.empty(v, dtype=np.float32)
    out16 = np.empty(v, dtype=np.uint16)
    idx = _load().orc_lm_head(_ptr(e), _ptr(h), v, k, _ptr(out32), _ptr(out16),
                              threads)
    if idx < 0:
        raise ValueError("in_features out of range")
    return out32, out16, int(idx)


# --------------------------------------------------------- model oracle --
# model_oracle.c: the non-Linear ops of cpu_ops.cpp and the CPU decode /
# prefill order of qwen2.cpp (see model_oracle.h for the pinning).

class _ModelConfig(ctypes.Structure):
    _fields_ = [("layers", ctypes.c_int), ("hidden", ctypes.c_int),
                ("heads", ctypes.c_int), ("kv_heads", ctypes.c_int),
                ("inter", ctypes.c_int), ("vocab", ctypes.c_int),
                ("max_seq", ctypes.c_int), ("eps", ctypes.c_float),
                ("theta", ctypes.c_float), ("threads", ctypes.c_int)]


class _ModelWeights(ctypes.Structure):
    _fields_ = [(name, ctypes.c_void_p) for name in (
        "embed", "final_norm", "in_norm", "post_norm", "wq", "bq", "wk", "bk",
        "wv", "bv", "wo", "wg", "wu", "wd")]


def _model_lib():
    lib = _load()
    if not getattr(lib, "_model_ready", False):
        p, i, f = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
        lib.orc_rms_norm.argtypes = [p, p, p, i, f]
        lib.orc_rope.argtypes = [p, p, i, i, i, i, f]
        lib.orc_attention_decode.argtypes = [p, p, p, p, i, i, i, i, i, i]
        lib.orc_silu_mul.argtypes = [p, p, p, i]
        lib.orc_model_create.argtypes = [p, p]
        lib.orc_model_create.restype = p
        lib.orc_model_destroy.argtypes = [p]
        lib.orc_model_prefill.argtypes = [p, p, i, p]
        lib.orc_model_prefill.restype = i
        lib.orc_model_decode.argtypes = [p, i, i, p]
        lib.orc_model_decode.restype = i
        lib._model_ready = True
    return lib


def rms_norm(x, weight, eps: float) -> np.ndarray:
    """cpu_ops.cpp:15-21."""
    xx, w = _c(x, np.float32), _c(weight, np.float32)
    out = np.empty_like(xx)
    _model_lib().orc_rms_norm(_ptr(xx), _ptr(w), _ptr(out), xx.size, eps)
    return out


def rope(q, k, heads: int, kv_heads: int, head_dim: int, position: int,
         theta: float):
    """cpu_ops.cpp:33-56 (returns rotated copies)."""
    qq, kk = _c(q, np.float32).copy(), _c(k, np.float32).copy()
    _model_lib().orc_rope(_ptr(qq), _ptr(kk), heads, kv_heads, head_dim,
                          position, theta)
    return qq, kk


def attention_decode(q, key_cache, value_cache, heads: int, kv_heads: int,
                     head_dim: int, seq_len: int, max_seq: int,
                     threads: int = 0) -> np.ndarray:
    """cpu_ops.cpp:58-91; caches [kv_heads, max_seq, head_dim]."""
    qq = _c(q, np.float32)
    kc, vc = _c(key_cache, np.float32), _c(value_cache, np.float32)
    out = np.empty(heads * head_dim, np.float32)
    _model_lib().orc_attention_decode(_ptr(qq), _ptr(kc), _ptr(vc), _ptr(out),
                                      heads, kv_heads, head_dim, seq_len,
                                      max_seq, threads)
    return out


def silu_mul(gate, up) -> np.ndarray:
    """cpu_ops.cpp:168-173."""
    g, u = _c(gate, np.float32), _c(up, np.float32)
    out = np.empty_like(g)
    _model_lib().orc_silu_mul(_ptr(g), _ptr(u), _ptr(out), g.size)
    return out


class Model:
    """The reference's CPU FP32 Qwen2 model (qwen2.cpp:376-494) on FP32
    weights.  ``weights`` maps the names of orc_model_weights (embed,
    final_norm, in_norm, post_norm, wq, bq, wk, bk, wv, bv, wo, wg, wu, wd)
    to float32 arrays, the per-layer ones stacked over layers."""

    def __init__(self, weights: dict, layers: int, hidden: int, heads: int,
                 kv_heads: int, inter: int, vocab: int, max_seq: int,
                 eps: float = 1e-6, theta: float = 1e6, threads: int = 0):
        self._keep = {k: _c(v, np.float32) for k, v in weights.items()}
        w = _ModelWeights(**{k: _ptr(v) for k, v in self._keep.items()})
        c = _ModelConfig(layers, hidden, heads, kv_heads, inter, vocab, max_seq,
                         eps, theta, threads)
        self.vocab = vocab
        self._handle = _model_lib().orc_model_create(ctypes.byref(c), ctypes.byref(w))
        if not self._handle:
            raise ValueError("bad model shape or out of memory")

    def prefill(self, tokens, logits: bool = False):
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.empty(self.vocab, np.float32) if logits else None
        idx = _model_lib().orc_model_prefill(self._handle, _ptr(t), t.size, _ptr(out))
        if idx < 0:
            raise ValueError("bad prefill input")
        return (idx, out) if logits else idx

    def decode(self, token: int, position: int, logits: bool = False):
        out = np.empty(self.vocab, np.float32) if logits else None
        idx = _model_lib().orc_model_decode(self._handle, int(token), int(position),
                                            _ptr(out))
        if idx < 0:
            raise ValueError("bad decode input")
        return (idx, out) if logits else idx

    def close(self):
        if self._handle:
            _model_lib().orc_model_destroy(self._handle)
            self._handle = None

    def __del__(self):
        self.close()
