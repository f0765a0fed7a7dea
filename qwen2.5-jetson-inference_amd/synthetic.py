"""Random-init Qwen2 weights in the archive's tensor layout (numpy, host).

No checkpoint can be fetched here, so models are random-initialised with
the architecture's shapes and stored as the reference's exporter would
store them (tools/export_model.py, Greedy-cy/qwen2.5-jetson-inference):

* tensor names as in the QWENBIN1 archive (``model.layers.<i>.self_attn.
  q_proj.weight`` ...), the W8A16 scales as the sibling ``<name>.scale``
  (export_model.py:299);
* BF16 tensors as little-endian uint16 words, FP32 -> BF16 round to nearest
  even with NaNs quieted (export_model.py:123-131);
* W8A16 Linear weights (2-D tensors other than the embedding / LM head,
  export_model.py:220-223) quantized per row in groups of 64 along K:
  s = max|w| / 127 in FP32 (0 -> 1), q = clip(rint(w / s), -127, 127) with
  the FP32 s, scale stored as BF16 (export_model.py:226-247, 288-289).
"""
from __future__ import annotations

import dataclasses

import numpy as np


@dataclasses.dataclass(frozen=True)
class ModelConfig:
    """include/infer/model_config.hpp:7-20."""
    hidden_size: int
    intermediate_size: int
    num_layers: int
    num_heads: int
    num_kv_heads: int
    vocab_size: int
    eos_token_id: int = -1
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_heads

    @property
    def kv_dim(self) -> int:
        return self.num_kv_heads * self.head_dim


# Qwen2.5-0.5B(-Instruct): the model every BASELINE configuration uses.
QWEN25_0_5B = ModelConfig(hidden_size=896, intermediate_size=4864, num_layers=24,
                          num_heads=14, num_kv_heads=2, vocab_size=151936,
                          eos_token_id=151645, rms_norm_eps=1e-6, rope_theta=1e6)

LINEARS = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
           "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")
BIASED = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj")


def float32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """FP32 -> BF16 words, round to nearest even, NaN quieted."""
    v = np.ascontiguousarray(a, dtype=np.float32)
    bits = v.view(np.uint32)
    out = ((bits + (np.uint32(0x7FFF) + ((bits >> 16) & np.uint32(1)))) >> 16).astype(np.uint16)
    nan = np.isnan(v)
    if np.any(nan):
        out[nan] = ((bits[nan] >> 16) | np.uint32(0x0040)).astype(np.uint16)
    return out


def bf16_bits_to_float32(a: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(a, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def quantize_groupwise(w: np.ndarray, group_size: int = 64):
    """Symmetric per-row group quantization; returns (int8 q, FP32 scales
    [rows, ceil(cols / group_size)]).  The last group may be short."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    groups = (cols + group_size - 1) // group_size
    q = np.empty((rows, cols), np.int8)
    scales = np.empty((rows, groups), np.float32)
    full = cols // group_size
    spans = []
    if full:
        spans.append((0, full * group_size, full))
    if cols % group_size:
        spans.append((full * group_size, cols, 1))
    g0 = 0
    for begin, end, count in spans:
        blocks = w[:, begin:end].reshape(rows, count, -1)
        s = (np.abs(blocks).max(axis=2) / np.float32(127.0)).astype(np.float32)
        s = np.where(s == 0.0, np.float32(1.0), s).astype(np.float32)
        q[:, begin:end] = np.clip(np.rint(blocks / s[:, :, None]), -127, 127).astype(
            np.int8).reshape(rows, end - begin)
        scales[:, g0:g0 + count] = s
        g0 += count
    return q, scales


def linear_shapes(c: ModelConfig):
    h, i, kv = c.hidden_size, c.intermediate_size, c.kv_dim
    return {"self_attn.q_proj": (h, h), "self_attn.k_proj": (kv, h),
            "self_attn.v_proj": (kv, h), "self_attn.o_proj": (h, h),
            "mlp.gate_proj": (i, h), "mlp.up_proj": (i, h), "mlp.down_proj": (h, i)}


def random_model(c: ModelConfig, precision: str = "w8a16", seed: int = 4,
                 std: float = 0.02, plain_init: bool = False) -> dict:
    """Random-init tensors by archive name: Linear weights and the embedding
    ~ N(0, std); norm weights 1 + N(0, std) and biases N(0, std), or with
    plain_init the initial values of a freshly built model (norm weights 1,
    biases 0); W8A16 quantizes the Linear weights as the
    exporter does, W16A16 stores them as BF16."""
    if precision not in ("w8a16", "w16a16"):
        raise ValueError("precision must be w8a16 or w16a16")
    rng = np.random.default_rng(seed)

    def normal(*shape):
        return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std))

    def norm_weight():
        return float32_to_bf16_bits(np.ones(c.hidden_size, np.float32) if plain_init
                                    else 1 + normal(c.hidden_size))

    t = {"model.embed_tokens.weight": float32_to_bf16_bits(normal(c.vocab_size, c.hidden_size)),
         "model.norm.weight": norm_weight()}
    shapes = linear_shapes(c)
    for layer in range(c.num_layers):
        p = f"model.layers.{layer}."
        t[p + "input_layernorm.weight"] = norm_weight()
        t[p + "post_attention_layernorm.weight"] = norm_weight()
        for name in LINEARS:
            w = normal(*shapes[name])
            if precision == "w8a16":
                q, s = quantize_groupwise(w)
                t[p + name + ".weight"] = q
                t[p + name + ".weight.scale"] = float32_to_bf16_bits(s)
            else:
                t[p + name + ".weight"] = float32_to_bf16_bits(w)
            if name in BIASED:
                n = shapes[name][0]
                t[p + name + ".bias"] = float32_to_bf16_bits(
                    np.zeros(n, np.float32) if plain_init else normal(n))
    return t


def random_checkpoint(c: ModelConfig, seed: int = 4, std: float = 0.02,
                      tied: bool = True, plain_init: bool = False) -> dict:
    """Random FP32 checkpoint tensors by archive name, in the order a
    Hugging Face checkpoint lists them: what the archive exporter reads.
    With tied=False an lm_head.weight is included; with plain_init the norm
    weights are 1 and the biases 0 (a freshly built model),
    else 1 + N(0, std) and N(0, std)."""
    rng = np.random.default_rng(seed)

    def normal(*shape):
        return rng.standard_normal(shape, dtype=np.float32) * np.float32(std)

    def norm_weight():
        return np.ones(c.hidden_size, np.float32) if plain_init else 1 + normal(c.hidden_size)

    t = {"model.embed_tokens.weight": normal(c.vocab_size, c.hidden_size)}
    shapes = linear_shapes(c)
    for layer in range(c.num_layers):
        p = f"model.layers.{layer}."
        t[p + "input_layernorm.weight"] = norm_weight()
        for name in LINEARS:
            t[p + name + ".weight"] = normal(*shapes[name])
            if name in BIASED:
                n = shapes[name][0]
                t[p + name + ".bias"] = np.zeros(n, np.float32) if plain_init else normal(n)
        t[p + "post_attention_layernorm.weight"] = norm_weight()
    t["model.norm.weight"] = norm_weight()
    if not tied:
        t["lm_head.weight"] = normal(c.vocab_size, c.hidden_size)
    return t


def dequantized_fp32(t: dict, c: ModelConfig) -> dict:
    """The FP32 weights the model computes with (q * bf16 scale, exact in
    FP32; BF16 tensors widened), layer-stacked for a CPU FP32 model."""
    def f(name):
        return bf16_bits_to_float32(t[name])

    def linear(name):
        w = t[name + ".weight"]
        if w.dtype == np.int8:
            s = bf16_bits_to_float32(t[name + ".weight.scale"])
            return (w.reshape(w.shape[0], -1, 64).astype(np.float32) * s[:, :, None]).reshape(
                w.shape)
        return bf16_bits_to_float32(w)

    L = c.num_layers
    out = {"embed": f("model.embed_tokens.weight").reshape(c.vocab_size, c.hidden_size),
           "final_norm": f("model.norm.weight")}
    key = {"self_attn.q_proj": "wq", "self_attn.k_proj": "wk", "self_attn.v_proj": "wv",
           "self_attn.o_proj": "wo", "mlp.gate_proj": "wg", "mlp.up_proj": "wu",
           "mlp.down_proj": "wd"}
    out["in_norm"] = np.stack([f(f"model.layers.{i}.input_layernorm.weight") for i in range(L)])
    out["post_norm"] = np.stack(
        [f(f"model.layers.{i}.post_attention_layernorm.weight") for i in range(L)])
    for name, k in key.items():
        out[k] = np.stack([linear(f"model.layers.{i}.{name}") for i in range(L)])
    for name, k in (("self_attn.q_proj", "bq"), ("self_attn.k_proj", "bk"),
                    ("self_attn.v_proj", "bv")):
        out[k] = np.stack([f(f"model.layers.{i}.{name}.bias") for i in range(L)])
    return out
