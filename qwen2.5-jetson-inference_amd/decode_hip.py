"""Python binding of the fused decode-step operators (include/infer_decode.h).

Each function launches one of the kernels the HIP decode runtime runs for a
token, on caller-owned device memory: arguments are device pointers
(``int``) or contiguous torch CUDA tensors, ``None`` is a null pointer, and
a nonzero status raises :class:`linear_hip.InferError`.  They replace short
sequences of the reference's per-op calls on its decode path
(src/qwen2.cpp:597-674, Greedy-cy/qwen2.5-jetson-inference); the header
names the sequence each one stands for.
"""
from __future__ import annotations

import ctypes

import linear_hip
from linear_hip import _check, _ptr, _stream

# Every symbol include/infer_decode.h declares.
EXPORTED_SYMBOLS = (
    "infer_hip_rms_norm_gemv_w8a16",
    "infer_hip_rms_norm_gemv_bf16",
    "infer_hip_rms_norm_gate_up_silu_w8a16",
    "infer_hip_rms_norm_gate_up_silu_bf16",
    "infer_hip_rms_norm_qkv_rope_w8a16",
    "infer_hip_rms_norm_qkv_rope_bf16",
    "infer_hip_rope_row",
    "infer_hip_attention_decode_bf16",
    "infer_hip_attention_decode_halves_bf16",
    "infer_hip_attention_halves_o_proj_w8a16",
    "infer_hip_attention_halves_o_proj_bf16",
    "infer_hip_attention_decode_parts_bf16",
    "infer_hip_attention_parts_o_proj_w8a16",
    "infer_hip_attention_parts_o_proj_bf16",
    "infer_hip_gemv_w8a16_rows",
    "infer_hip_gemv_bf16_rows",
    "infer_hip_attention_decode_spans_bf16",
    "infer_hip_attention_decode_span",
    "infer_hip_attention_decode_splits",
    "infer_hip_attention_merge_o_proj",
    "infer_hip_lm_head_decode_workspace_bytes",
    "infer_hip_rms_norm_lm_head_argmax",
)


class W8A16Weight(ctypes.Structure):
    """infer_hip_w8a16_weight."""
    _fields_ = [("weight", ctypes.c_void_p), ("scales", ctypes.c_void_p),
                ("bias", ctypes.c_void_p)]


class NormGemv(ctypes.Structure):
    """infer_hip_norm_gemv."""
    _fields_ = [("weight", ctypes.c_void_p), ("scales", ctypes.c_void_p),
                ("bias", ctypes.c_void_p), ("output", ctypes.c_void_p),
                ("out_features", ctypes.c_int)]


class Bf16Weight(ctypes.Structure):
    """infer_hip_bf16_weight."""
    _fields_ = [("weight", ctypes.c_void_p), ("bias", ctypes.c_void_p)]


class NormGemvBf16(ctypes.Structure):
    """infer_hip_norm_gemv_bf16."""
    _fields_ = [("weight", ctypes.c_void_p), ("bias", ctypes.c_void_p),
                ("output", ctypes.c_void_p), ("out_features", ctypes.c_int)]


_bound = False


def load():
    global _bound
    lib = linear_hip.load()
    if _bound:
        return lib
    p, i, f = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
    sigs = {
        "infer_hip_rms_norm_gemv_w8a16": ([p, p, f, i, ctypes.POINTER(NormGemv), i, p], i),
        "infer_hip_rms_norm_gemv_bf16": ([p, p, f, i, ctypes.POINTER(NormGemvBf16), i, p], i),
        "infer_hip_rms_norm_gate_up_silu_w8a16": ([p, p, f, i, p, p, p, p, p, i, p], i),
        "infer_hip_rms_norm_gate_up_silu_bf16": ([p, p, f, i, p, p, p, i, p], i),
        "infer_hip_rms_norm_qkv_rope_w8a16": ([p, p, f, i, ctypes.POINTER(W8A16Weight),
                                               ctypes.POINTER(W8A16Weight),
                                               ctypes.POINTER(W8A16Weight), p, p, p, p, p,
                                               i, i, i, i, p], i),
        "infer_hip_rms_norm_qkv_rope_bf16": ([p, p, f, i, ctypes.POINTER(Bf16Weight),
                                              ctypes.POINTER(Bf16Weight),
                                              ctypes.POINTER(Bf16Weight), p, p, p, p, p,
                                              i, i, i, i, p], i),
        "infer_hip_rope_row": ([f, i, i, ctypes.POINTER(ctypes.c_float)], i),
        "infer_hip_attention_decode_bf16": ([p, p, p, p, p, i, i, i, i, p], i),
        "infer_hip_attention_decode_halves_bf16": ([p, p, p, p, p, i, i, i, i, p], i),
        "infer_hip_attention_halves_o_proj_w8a16": ([p, p, i, i, p, p, p, i, p], i),
        "infer_hip_attention_halves_o_proj_bf16": ([p, p, i, i, p, p, i, p], i),
        "infer_hip_attention_decode_parts_bf16": ([p, p, p, p, p, i, i, i, i, i, p], i),
        "infer_hip_attention_parts_o_proj_w8a16": ([p, p, i, i, i, p, p, p, i, p], i),
        "infer_hip_attention_parts_o_proj_bf16": ([p, p, i, i, i, p, p, i, p], i),
        "infer_hip_gemv_w8a16_rows": ([p, p, p, p, p, i, i, p], i),
        "infer_hip_gemv_bf16_rows": ([p, p, p, p, i, i, p], i),
        "infer_hip_attention_decode_spans_bf16": ([p, p, p, p, p, i, i, i, i, p], i),
        "infer_hip_attention_decode_span": ([i, i], i),
        "infer_hip_attention_decode_splits": ([i, i], i),
        "infer_hip_attention_merge_o_proj": ([p, p, i, i, i, i, i, p, p, p, i, p], i),
        "infer_hip_lm_head_decode_workspace_bytes": ([i], ctypes.c_size_t),
        "infer_hip_rms_norm_lm_head_argmax": ([p, p, f, p, i, i, p, p, p, p], i),
    }
    for name, (args, res) in sigs.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    _bound = True
    return lib


def rms_norm_gemv_w8a16(input, norm_weight, epsilon: float, in_features: int, gemvs,
                        stream=None) -> None:
    """gemvs: up to three (weight, scales, bias, output, out_features)."""
    arr = (NormGemv * max(1, len(gemvs)))()
    for k, (w, s, b, y, n) in enumerate(gemvs):
        arr[k] = NormGemv(_ptr(w), _ptr(s), _ptr(b), _ptr(y), int(n))
    _check(load().infer_hip_rms_norm_gemv_w8a16(_ptr(input), _ptr(norm_weight), epsilon,
                                                in_features, arr, len(gemvs),
                                                _stream(stream)))


def rms_norm_gemv_bf16(input, norm_weight, epsilon: float, in_features: int, gemvs,
                       stream=None) -> None:
    """gemvs: up to three (weight, bias, output, out_features)."""
    arr = (NormGemvBf16 * max(1, len(gemvs)))()
    for k, (w, b, y, n) in enumerate(gemvs):
        arr[k] = NormGemvBf16(_ptr(w), _ptr(b), _ptr(y), int(n))
    _check(load().infer_hip_rms_norm_gemv_bf16(_ptr(input), _ptr(norm_weight), epsilon,
                                               in_features, arr, len(gemvs), _stream(stream)))


def rms_norm_gate_up_silu_w8a16(input, norm_weight, epsilon: float, in_features: int,
                                gate_weight, gate_scales, up_weight, up_scales, output,
                                intermediate_size: int, stream=None) -> None:
    _check(load().infer_hip_rms_norm_gate_up_silu_w8a16(
        _ptr(input), _ptr(norm_weight), epsilon, in_features, _ptr(gate_weight),
        _ptr(gate_scales), _ptr(up_weight), _ptr(up_scales), _ptr(output),
        intermediate_size, _stream(stream)))


def rms_norm_gate_up_silu_bf16(input, norm_weight, epsilon: float, in_features: int,
                               gate_weight, up_weight, output, intermediate_size: int,
                               stream=None) -> None:
    _check(load().infer_hip_rms_norm_gate_up_silu_bf16(
        _ptr(input), _ptr(norm_weight), epsilon, in_features, _ptr(gate_weight),
        _ptr(up_weight), _ptr(output), intermediate_size, _stream(stream)))


def rms_norm_qkv_rope_w8a16(input, norm_weight, epsilon: float, in_features: int, q_proj,
                            k_proj, v_proj, q_out, key_cache, value_cache, rope_row, position,
                            num_heads: int, num_kv_heads: int, head_dim: int,
                            max_sequence_length: int, stream=None) -> None:
    """q_proj / k_proj / v_proj: (weight, scales, bias) each."""
    ws = [W8A16Weight(_ptr(w), _ptr(s), _ptr(b)) for (w, s, b) in (q_proj, k_proj, v_proj)]
    _check(load().infer_hip_rms_norm_qkv_rope_w8a16(
        _ptr(input), _ptr(norm_weight), epsilon, in_features, ctypes.byref(ws[0]),
        ctypes.byref(ws[1]), ctypes.byref(ws[2]), _ptr(q_out), _ptr(key_cache),
        _ptr(value_cache), _ptr(rope_row), _ptr(position), num_heads, num_kv_heads, head_dim,
        max_sequence_length, _stream(stream)))


def rms_norm_qkv_rope_bf16(input, norm_weight, epsilon: float, in_features: int, q_proj,
                           k_proj, v_proj, q_out, key_cache, value_cache, rope_row, position,
                           num_heads: int, num_kv_heads: int, head_dim: int,
                           max_sequence_length: int, stream=None) -> None:
    """q_proj / k_proj / v_proj: (weight, bias) each."""
    ws = [Bf16Weight(_ptr(w), _ptr(b)) for (w, b) in (q_proj, k_proj, v_proj)]
    _check(load().infer_hip_rms_norm_qkv_rope_bf16(
        _ptr(input), _ptr(norm_weight), epsilon, in_features, ctypes.byref(ws[0]),
        ctypes.byref(ws[1]), ctypes.byref(ws[2]), _ptr(q_out), _ptr(key_cache),
        _ptr(value_cache), _ptr(rope_row), _ptr(position), num_heads, num_kv_heads, head_dim,
        max_sequence_length, _stream(stream)))


def rope_row(theta: float, head_dim: int, position: int):
    """(cos, sin) pairs of one position as a float32 array [head_dim / 2, 2]."""
    import numpy as np
    out = np.empty(head_dim, np.float32)
    _check(load().infer_hip_rope_row(theta, head_dim, position,
                                     out.ctypes.data_as(ctypes.POINTER(ctypes.c_float))))
    return out.reshape(-1, 2)


def attention_decode_bf16(q, key_cache, value_cache, position, output, num_heads: int,
                          num_kv_heads: int, head_dim: int, max_sequence_length: int,
                          stream=None) -> None:
    _check(load().infer_hip_attention_decode_bf16(
        _ptr(q), _ptr(key_cache), _ptr(value_cache), _ptr(position), _ptr(output), num_heads,
        num_kv_heads, head_dim, max_sequence_length, _stream(stream)))


PART_RECORD = 68  # floats per (head, part) record of the halves / parts attention
HALF_RECORD = PART_RECORD


def attention_decode_halves_bf16(q, key_cache, value_cache, position, records,
                                 num_heads: int, num_kv_heads: int, head_dim: int,
                                 max_sequence_length: int, stream=None) -> None:
    """records: float32 [num_heads, 2, PART_RECORD]."""
    _check(load().infer_hip_attention_decode_halves_bf16(
        _ptr(q), _ptr(key_cache), _ptr(value_cache), _ptr(position), _ptr(records), num_heads,
        num_kv_heads, head_dim, max_sequence_length, _stream(stream)))


def attention_halves_o_proj_w8a16(records, position, num_heads: int, max_sequence_length: int,
                                  weight, scales, residual, out_features: int,
                                  stream=None) -> None:
    _check(load().infer_hip_attention_halves_o_proj_w8a16(
        _ptr(records), _ptr(position), num_heads, max_sequence_length, _ptr(weight),
        _ptr(scales), _ptr(residual), out_features, _stream(stream)))


def attention_halves_o_proj_bf16(records, position, num_heads: int, max_sequence_length: int,
                                 weight, residual, out_features: int, stream=None) -> None:
    _check(load().infer_hip_attention_halves_o_proj_bf16(
        _ptr(records), _ptr(position), num_heads, max_sequence_length, _ptr(weight),
        _ptr(residual), out_features, _stream(stream)))


def attention_decode_parts_bf16(q, key_cache, value_cache, position, records,
                                num_heads: int, num_kv_heads: int, head_dim: int,
                                max_sequence_length: int, num_parts: int, stream=None) -> None:
    """records: float32 [num_heads, num_parts, PART_RECORD]; num_parts 2 or 4."""
    _check(load().infer_hip_attention_decode_parts_bf16(
        _ptr(q), _ptr(key_cache), _ptr(value_cache), _ptr(position), _ptr(records), num_heads,
        num_kv_heads, head_dim, max_sequence_length, num_parts, _stream(stream)))


def attention_parts_o_proj_w8a16(records, position, num_heads: int, max_sequence_length: int,
                                 num_parts: int, weight, scales, residual, out_features: int,
                                 stream=None) -> None:
    _check(load().infer_hip_attention_parts_o_proj_w8a16(
        _ptr(records), _ptr(position), num_heads, max_sequence_length, num_parts, _ptr(weight),
        _ptr(scales), _ptr(residual), out_features, _stream(stream)))


def attention_parts_o_proj_bf16(records, position, num_heads: int, max_sequence_length: int,
                                num_parts: int, weight, residual, out_features: int,
                                stream=None) -> None:
    _check(load().infer_hip_attention_parts_o_proj_bf16(
        _ptr(records), _ptr(position), num_heads, max_sequence_length, num_parts, _ptr(weight),
        _ptr(residual), out_features, _stream(stream)))


def gemv_w8a16_rows(weight, scales, bias, input, output, out_features: int,
                    in_features: int, stream=None) -> None:
    _check(load().infer_hip_gemv_w8a16_rows(_ptr(weight), _ptr(scales), _ptr(bias),
                                            _ptr(input), _ptr(output), out_features,
                                            in_features, _stream(stream)))


def gemv_bf16_rows(weight, bias, input, output, out_features: int, in_features: int,
                   stream=None) -> None:
    _check(load().infer_hip_gemv_bf16_rows(_ptr(weight), _ptr(bias), _ptr(input), _ptr(output),
                                           out_features, in_features, _stream(stream)))


def attention_decode_spans_bf16(q, key_cache, value_cache, position, partials, num_heads: int,
                                num_kv_heads: int, head_dim: int, max_sequence_length: int,
                                stream=None) -> None:
    """partials: float32 [num_heads, attention_decode_splits(), head_dim + 2]."""
    _check(load().infer_hip_attention_decode_spans_bf16(
        _ptr(q), _ptr(key_cache), _ptr(value_cache), _ptr(position), _ptr(partials), num_heads,
        num_kv_heads, head_dim, max_sequence_length, _stream(stream)))


def attention_decode_span(max_sequence_length: int, head_dim: int = 64) -> int:
    return load().infer_hip_attention_decode_span(max_sequence_length, head_dim)


def attention_decode_splits(max_sequence_length: int, head_dim: int = 64) -> int:
    return load().infer_hip_attention_decode_splits(max_sequence_length, head_dim)


def attention_merge_o_proj(partials, position, num_heads: int, head_dim: int, span: int,
                           max_splits: int, max_sequence_length: int, weight, scales,
                           residual, out_features: int, stream=None) -> None:
    _check(load().infer_hip_attention_merge_o_proj(
        _ptr(partials), _ptr(position), num_heads, head_dim, span, max_splits,
        max_sequence_length, _ptr(weight), _ptr(scales), _ptr(residual), out_features,
        _stream(stream)))


def lm_head_decode_workspace_bytes(vocab: int) -> int:
    return load().infer_hip_lm_head_decode_workspace_bytes(vocab)


def rms_norm_lm_head_argmax(input, norm_weight, epsilon: float, weight, vocab: int,
                            in_features: int, logits, workspace, argmax, stream=None) -> None:
    _check(load().infer_hip_rms_norm_lm_head_argmax(
        _ptr(input), _ptr(norm_weight), epsilon, _ptr(weight), vocab, in_features,
        _ptr(logits), _ptr(workspace), _ptr(argmax), _stream(stream)))
