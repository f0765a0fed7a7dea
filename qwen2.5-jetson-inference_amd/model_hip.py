"""Python binding of the HIP Qwen2 decode runtime (include/infer_model.h).

:class:`Qwen2Model` mirrors the reference's ``infer::Qwen2Model``
(include/infer/qwen2.hpp:41-67, Greedy-cy/qwen2.5-jetson-inference):
``prefill``, ``decode_next``, ``generate``, ``last_logits_host``,
``reset``, ``position``, ``has_prefilled``, ``kv_cache_bytes`` and
``workspace_bytes`` keep their meaning; errors raise
:class:`linear_hip.InferError` where the reference throws ``infer::Error``.
It also exposes ``decode_steps``, the host-sync-free greedy decode loop.

Weights are given by archive tensor name (``synthetic.random_model`` makes
a random-init set), as numpy arrays (uploaded to ``cuda:0``) or torch CUDA
tensors; the model keeps them alive.
"""
from __future__ import annotations

import ctypes
import dataclasses

import numpy as np

import linear_hip
from linear_hip import InferError, _check
from synthetic import LINEARS, ModelConfig

PRECISIONS = {"w16a16": 1, "w8a16": 2}

EXPORTED_SYMBOLS = (
    "infer_hip_model_create",
    "infer_hip_model_destroy",
    "infer_hip_model_reset",
    "infer_hip_model_prefill",
    "infer_hip_model_decode_next",
    "infer_hip_model_decode_steps",
    "infer_hip_model_rewind",
    "infer_hip_model_generate",
    "infer_hip_model_last_logits",
    "infer_hip_model_position",
    "infer_hip_model_has_prefilled",
    "infer_hip_model_kv_cache_bytes",
    "infer_hip_model_workspace_bytes",
    "infer_hip_model_stream",
    "infer_hip_model_kernel_times",
    "infer_hip_model_kernel_name",
    "infer_hip_attention_prefill_bf16",
    "infer_hip_gemm_gate_up_silu_w8a16",
    "infer_hip_gemm_gate_up_silu_bf16",
)
KERNEL_KINDS = 9


class _Config(ctypes.Structure):
    _fields_ = [("hidden_size", ctypes.c_int), ("intermediate_size", ctypes.c_int),
                ("num_layers", ctypes.c_int), ("num_heads", ctypes.c_int),
                ("num_kv_heads", ctypes.c_int), ("vocab_size", ctypes.c_int),
                ("eos_token_id", ctypes.c_int), ("rms_norm_eps", ctypes.c_float),
                ("rope_theta", ctypes.c_float)]


class _Linear(ctypes.Structure):
    _fields_ = [("weight", ctypes.c_void_p), ("scales", ctypes.c_void_p),
                ("bias", ctypes.c_void_p)]


class _Layer(ctypes.Structure):
    _fields_ = [("input_layernorm", ctypes.c_void_p),
                ("post_attention_layernorm", ctypes.c_void_p)] + [
        (name.split(".")[1], _Linear) for name in LINEARS]


class _Weights(ctypes.Structure):
    _fields_ = [("embed_tokens", ctypes.c_void_p), ("norm", ctypes.c_void_p),
                ("lm_head", ctypes.c_void_p), ("layers", ctypes.POINTER(_Layer))]


class _Options(ctypes.Structure):
    _fields_ = [("precision", ctypes.c_int), ("max_sequence_length", ctypes.c_int),
                ("use_graph", ctypes.c_int)]


class _Stats(ctypes.Structure):
    _fields_ = [("prompt_tokens", ctypes.c_int), ("generated_tokens", ctypes.c_int),
                ("ttft_ms", ctypes.c_double), ("decode_ms", ctypes.c_double),
                ("total_ms", ctypes.c_double)]


@dataclasses.dataclass
class GenerationStats:
    """include/infer/qwen2.hpp:23-34."""
    prompt_tokens: int
    generated_tokens: int
    ttft_ms: float
    decode_ms: float
    total_ms: float

    def decode_tokens_per_second(self) -> float:
        if self.decode_ms > 0 and self.generated_tokens > 1:
            return (self.generated_tokens - 1) * 1000.0 / self.decode_ms
        return 0.0


_bound = False


def load():
    global _bound
    lib = linear_hip.load()
    if _bound:
        return lib
    p, i = ctypes.c_void_p, ctypes.c_int
    ip = ctypes.POINTER(ctypes.c_int)
    sigs = {
        "infer_hip_model_create": ([ctypes.POINTER(_Config), ctypes.POINTER(_Weights),
                                    ctypes.POINTER(_Options), ctypes.POINTER(p)], i),
        "infer_hip_model_destroy": ([p], i),
        "infer_hip_model_reset": ([p], i),
        "infer_hip_model_prefill": ([p, ip, i, ip], i),
        "infer_hip_model_decode_next": ([p, i, ip], i),
        "infer_hip_model_decode_steps": ([p, i, ip], i),
        "infer_hip_model_rewind": ([p, i, i], i),
        "infer_hip_model_generate": ([p, ip, i, i, i, ip, ip, ctypes.POINTER(_Stats)], i),
        "infer_hip_model_last_logits": ([p, ctypes.POINTER(ctypes.c_float)], i),
        "infer_hip_model_position": ([p], i),
        "infer_hip_model_has_prefilled": ([p], i),
        "infer_hip_model_kv_cache_bytes": ([p], ctypes.c_size_t),
        "infer_hip_model_workspace_bytes": ([p], ctypes.c_size_t),
        "infer_hip_model_stream": ([p], p),
        "infer_hip_model_kernel_times": ([p, i, i, ctypes.POINTER(ctypes.c_double),
                                          ctypes.POINTER(ctypes.c_double), ip, i], i),
        "infer_hip_model_kernel_name": ([i], ctypes.c_char_p),
        "infer_hip_attention_prefill_bf16": ([p, p, p, p, i, i, i, i, i, p], i),
        "infer_hip_gemm_gate_up_silu_w8a16": ([p, p, p, p, p, p, i, p, p, i, i, i, p], i),
        "infer_hip_gemm_gate_up_silu_bf16": ([p, p, p, p, p, p, i, i, i, p], i),
        "infer_hip_model_open": ([ctypes.c_char_p, ctypes.POINTER(_Options), ctypes.POINTER(p)],
                                 i),
    }
    for name, (args, res) in sigs.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    _bound = True
    return lib


def attention_prefill_bf16(q, key_cache, value_cache, output, token_count: int,
                           num_heads: int, num_kv_heads: int, head_dim: int,
                           max_sequence_length: int, stream=None) -> None:
    """infer::cuda::attention_prefill_bf16 (cuda_ops.hpp:92-97) on device
    tensors (BF16 as int16/uint16/bfloat16 words)."""
    lib = load()
    _check(lib.infer_hip_attention_prefill_bf16(
        linear_hip._ptr(q), linear_hip._ptr(key_cache), linear_hip._ptr(value_cache),
        linear_hip._ptr(output), token_count, num_heads, num_kv_heads, head_dim,
        max_sequence_length, linear_hip._stream(stream)))


def gemm_gate_up_silu_w8a16(gate_w, gate_s, gate_b, up_w, up_s, up_b, group_size: int,
                            x, y, tokens: int, intermediate: int, hidden: int,
                            stream=None) -> None:
    """gate_proj and up_proj of x, then SiLU-mul, in one launch
    (infer_hip_gemm_gate_up_silu_w8a16); biases may be None."""
    lib = load()
    P = linear_hip._ptr
    _check(lib.infer_hip_gemm_gate_up_silu_w8a16(
        P(gate_w), P(gate_s), P(gate_b), P(up_w), P(up_s), P(up_b), group_size, P(x), P(y),
        tokens, intermediate, hidden, linear_hip._stream(stream)))


def gemm_gate_up_silu_bf16(gate_w, gate_b, up_w, up_b, x, y, tokens: int, intermediate: int,
                           hidden: int, stream=None) -> None:
    """The BF16-weight form of gemm_gate_up_silu_w8a16."""
    lib = load()
    P = linear_hip._ptr
    _check(lib.infer_hip_gemm_gate_up_silu_bf16(
        P(gate_w), P(gate_b), P(up_w), P(up_b), P(x), P(y), tokens, intermediate, hidden,
        linear_hip._stream(stream)))


def _dtype_name(t) -> str:
    """int8 / bfloat16 / other for a numpy array (BF16 as uint16 words) or
    a torch tensor."""
    if isinstance(t, np.ndarray):
        return {np.dtype(np.int8): "int8", np.dtype(np.uint16): "bfloat16"}.get(t.dtype,
                                                                                str(t.dtype))
    import torch
    return {torch.int8: "int8", torch.bfloat16: "bfloat16",
            torch.uint16: "bfloat16", torch.int16: "bfloat16"}.get(t.dtype, str(t.dtype))


def _int_array(values):
    arr = (ctypes.c_int * max(1, len(values)))()
    for k, v in enumerate(values):
        arr[k] = int(v)
    return arr


class Qwen2Model:
    """The HIP decode runtime over one set of device weights."""

    def __init__(self, config: ModelConfig, tensors: dict, precision: str = "w8a16",
                 max_sequence_length: int = 2048, use_graph: bool = True, device=None):
        import torch
        lib = load()
        if precision not in PRECISIONS:
            raise InferError(linear_hip.INVALID_ARGUMENT, "precision must be w8a16 or w16a16")
        self.config = config
        self.precision = precision
        self._device = torch.device(device or "cuda:0")
        self._keep = {}

        def dev(name, required=True, dtype=None):
            if name not in tensors:
                if required:
                    raise InferError(linear_hip.INVALID_ARGUMENT, f"missing weight: {name}")
                return None
            t = tensors[name]
            if dtype is not None and _dtype_name(t) != dtype:
                # src/qwen2.cpp:239-256: the record's dtype selects the kernel.
                raise InferError(linear_hip.INVALID_ARGUMENT,
                                 f"{name}: expected {dtype} under {precision}, got "
                                 f"{_dtype_name(t)}")
            if isinstance(t, np.ndarray):
                a = np.ascontiguousarray(t)
                if a.dtype == np.uint16:
                    a = a.view(np.int16)  # BF16 words; torch copies int16 everywhere
                t = torch.from_numpy(a).to(self._device)
            self._keep[name] = t
            return linear_hip._ptr(t)

        layers = (_Layer * config.num_layers)()
        for i in range(config.num_layers):
            p = f"model.layers.{i}."
            L = layers[i]
            L.input_layernorm = dev(p + "input_layernorm.weight")
            L.post_attention_layernorm = dev(p + "post_attention_layernorm.weight")
            for name in LINEARS:
                lin = getattr(L, name.split(".")[1])
                lin.weight = dev(p + name + ".weight",
                                 dtype="int8" if precision == "w8a16" else "bfloat16")
                lin.scales = dev(p + name + ".weight.scale", precision == "w8a16")
                lin.bias = dev(p + name + ".bias", False)
        w = _Weights(dev("model.embed_tokens.weight"), dev("model.norm.weight"),
                     dev("lm_head.weight", False), layers)
        cfg = _Config(config.hidden_size, config.intermediate_size, config.num_layers,
                      config.num_heads, config.num_kv_heads, config.vocab_size,
                      config.eos_token_id, config.rms_norm_eps, config.rope_theta)
        opts = _Options(PRECISIONS[precision], max_sequence_length, 1 if use_graph else 0)
        torch.cuda.synchronize(self._device)  # uploads complete before use
        handle = ctypes.c_void_p()
        _check(lib.infer_hip_model_create(ctypes.byref(cfg), ctypes.byref(w),
                                          ctypes.byref(opts), ctypes.byref(handle)))
        self._lib = lib
        self._h = handle
        self.max_sequence_length = max_sequence_length

    @classmethod
    def open(cls, model_directory, precision: str = "w8a16", max_sequence_length: int = 2048,
             use_graph: bool = True) -> "Qwen2Model":
        """Qwen2Model(model_directory, options) (src/qwen2.cpp:30-78): loads
        <dir>/config.json and <dir>/model.<precision>.qbin into weights the
        model owns, on the current device (infer_hip_model_open)."""
        import os
        import archive_hip
        lib = load()
        if precision not in PRECISIONS:
            raise InferError(linear_hip.INVALID_ARGUMENT, "precision must be w8a16 or w16a16")
        self = cls.__new__(cls)
        self.config, _ = archive_hip.load_config(os.path.join(model_directory, "config.json"))
        self.precision = precision
        self._keep = {}
        opts = _Options(PRECISIONS[precision], max_sequence_length, 1 if use_graph else 0)
        handle = ctypes.c_void_p()
        _check(lib.infer_hip_model_open(os.fsencode(os.fspath(model_directory)),
                                        ctypes.byref(opts), ctypes.byref(handle)))
        self._lib = lib
        self._h = handle
        self.max_sequence_length = max_sequence_length
        return self

    # -- reference surface (include/infer/qwen2.hpp:46-67) --
    def prefill(self, prompt_tokens) -> int:
        toks = _int_array(prompt_tokens)
        out = ctypes.c_int()
        _check(self._lib.infer_hip_model_prefill(self._h, toks, len(prompt_tokens),
                                                 ctypes.byref(out)))
        return out.value

    def decode_next(self, token: int) -> int:
        out = ctypes.c_int()
        _check(self._lib.infer_hip_model_decode_next(self._h, int(token), ctypes.byref(out)))
        return out.value

    def decode_steps(self, steps: int) -> list:
        buf = (ctypes.c_int * max(1, steps))()
        _check(self._lib.infer_hip_model_decode_steps(self._h, steps, buf))
        return list(buf[:steps])

    def rewind(self, position: int, token: int) -> None:
        """Keep the first `position` positions of the context and decode
        `token` next (infer_hip_model_rewind)."""
        _check(self._lib.infer_hip_model_rewind(self._h, int(position), int(token)))

    def generate(self, prompt_tokens, max_new_tokens: int, stop_on_eos: bool = True):
        toks = _int_array(prompt_tokens)
        out = (ctypes.c_int * max(1, max_new_tokens))()
        n = ctypes.c_int()
        st = _Stats()
        _check(self._lib.infer_hip_model_generate(self._h, toks, len(prompt_tokens),
                                                  max_new_tokens, 1 if stop_on_eos else 0, out,
                                                  ctypes.byref(n), ctypes.byref(st)))
        stats = GenerationStats(st.prompt_tokens, st.generated_tokens, st.ttft_ms,
                                st.decode_ms, st.total_ms)
        return list(out[:n.value]), stats

    def last_logits_host(self) -> np.ndarray:
        out = np.empty(self.config.vocab_size, np.float32)
        _check(self._lib.infer_hip_model_last_logits(
            self._h, out.ctypes.data_as(ctypes.POINTER(ctypes.c_float))))
        return out

    def reset(self) -> None:
        _check(self._lib.infer_hip_model_reset(self._h))

    @property
    def position(self) -> int:
        return self._lib.infer_hip_model_position(self._h)

    @property
    def has_prefilled(self) -> bool:
        return bool(self._lib.infer_hip_model_has_prefilled(self._h))

    def kv_cache_bytes(self) -> int:
        return self._lib.infer_hip_model_kv_cache_bytes(self._h)

    def workspace_bytes(self) -> int:
        return self._lib.infer_hip_model_workspace_bytes(self._h)

    @property
    def stream(self) -> int:
        return self._lib.infer_hip_model_stream(self._h) or 0

    def kernel_times(self, position: int, reps: int = 3) -> dict:
        """Per launch kind of the decode step: {name: (us per launch, bytes per
        launch, launches per step)}, timed with HIP events on the model's
        stream at KV context `position` (infer_hip_model_kernel_times)."""
        n = KERNEL_KINDS
        us = (ctypes.c_double * n)()
        nb = (ctypes.c_double * n)()
        ln = (ctypes.c_int * n)()
        _check(self._lib.infer_hip_model_kernel_times(self._h, position, reps, us, nb, ln, n))
        out = {}
        for k in range(n):
            if ln[k]:
                name = self._lib.infer_hip_model_kernel_name(k).decode()
                out[name] = (us[k], nb[k], ln[k])
        return out

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.infer_hip_model_destroy(self._h)
            self._h = None
        self._keep = {}

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
