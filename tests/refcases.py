"""Input generators for the parity tests.

Two families:

* The reference's own test generators, restated from their closed forms
  (Greedy-cy/qwen2.5-jetson-inference, tests/test_cuda.cpp and
  tools/linear_benchmark.cpp), so that the cases here are the cases the
  reference tests, with the same bytes.
* The BASELINE synthetic distributions (configs 1-3), drawn from numpy's
  counter-based Philox generator with the config's seed.

BF16 tensors are numpy ``uint16`` words; int8 weights are ``int8``.  The
BF16 encoding used here is the reference's RNE bit method via the oracle's
twin in numpy (``bf16_words``), which tests/test_oracle.py checks against
torch's independent float->bfloat16 conversion.
"""
from __future__ import annotations

import numpy as np

GROUP = 64

# The seven decoder Linear shapes (N, K) and whether the layer has a bias
# (src/qwen2.cpp:615-656): q/k/v carry biases, o/gate/up/down do not.
QWEN_LINEARS = (
    ("q_proj", 896, 896, True),
    ("k_proj", 128, 896, True),
    ("v_proj", 128, 896, True),
    ("o_proj", 896, 896, False),
    ("gate_proj", 4864, 896, False),
    ("up_proj", 4864, 896, False),
    ("down_proj", 896, 4864, False),
)
VOCAB = 151936
HIDDEN = 896


def bf16_words(values) -> np.ndarray:
    """FP32 -> BF16 words, round to nearest even, NaN quieted."""
    f = np.ascontiguousarray(values, dtype=np.float32)
    bits = f.view(np.uint32).astype(np.uint64)
    rounded = ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(f)
    if nan.any():
        rounded[nan] = ((bits[nan] >> 16) | 0x40).astype(np.uint16)
    return rounded


def bf16_values(words) -> np.ndarray:
    """BF16 words -> FP32 values."""
    w = np.ascontiguousarray(words, dtype=np.uint16).astype(np.uint32)
    return (w << 16).view(np.float32)


# --------------------------------------------------- reference generators --

def w8a16_linear_case(tokens: int, out_features: int, in_features: int):
    """check_w8a16_linear_case, tests/test_cuda.cpp:519-557.

    Returns (q int8 [N,K], scales bf16 [N,G], x bf16 [M,K], bias bf16 [N]).
    """
    n, k = out_features, in_features
    groups = -(-k // GROUP)
    idx = np.arange(n * k, dtype=np.uint64)
    q = (((idx * np.uint64(17)) % np.uint64(31)).astype(np.int64) - 15).astype(np.int8)
    if q.size >= 2:
        q[0] = -127
        q[1] = 127
    s = ((1 + (np.arange(n * groups) % 7)) / 1024.0).astype(np.float32)
    xi = np.arange(tokens * k, dtype=np.uint64)
    x = ((((xi * np.uint64(13)) % np.uint64(29)).astype(np.int64) - 14) / 64.0).astype(np.float32)
    b = (((np.arange(n) % 9) - 4) / 32.0).astype(np.float32)
    if k > GROUP:
        row = n - 1
        q[row * k: row * k + GROUP] = 0
        s[row * groups] = 1.0
    return (q.reshape(n, k), bf16_words(s).reshape(n, groups),
            bf16_words(x).reshape(tokens, k), bf16_words(b))


# Cases of tests/test_cuda.cpp:885-886, 896-899, 906-908, 915-918 as
# (tokens, N, K, bias).
W8A16_TAIL_CASES = ((3, 5, 70, True), (2, 7, 65, False))
W8A16_QWEN_CASES = ((2, 896, 896, True), (2, 128, 896, True),
                    (2, 4864, 896, False), (2, 896, 4864, False))
W8A16_PREFILL_CASES = tuple((m, n, k, bias) for m in (32, 128, 512)
                            for (n, k, bias) in ((896, 896, True),
                                                 (4864, 896, False),
                                                 (896, 4864, False)))
W8A16_ALIGNED_K_CASES = ((1, 896, 1024, True), (1, 896, 1216, False),
                         (1, 24, 896, True), (1, 96, 912, False))


def bf16_linear_case(tokens: int, out_features: int, in_features: int):
    """check_bf16_linear_case, tests/test_cuda.cpp:621-642.

    Returns (w bf16 [N,K], x bf16 [M,K], bias bf16 [N]).
    """
    n, k = out_features, in_features
    w = (((np.arange(n * k) % 17) - 8) * 0.015625).astype(np.float32)
    x = (((np.arange(tokens * k) % 13) - 6) * 0.03125).astype(np.float32)
    b = (((np.arange(n) % 5) - 2) * 0.0625).astype(np.float32)
    return (bf16_words(w).reshape(n, k), bf16_words(x).reshape(tokens, k),
            bf16_words(b))


# tests/test_cuda.cpp:697-702 as (tokens, N, K, bias).
BF16_LINEAR_CASES = ((3, 11, 14, True), (2, 5, 7, True), (3, 23, 14, False),
                     (32, 64, 64, True), (31, 37, 33, True), (65, 70, 67, False))


def make_gemv_weight(out_features: int, in_features: int, seed: int) -> np.ndarray:
    """make_gemv_weight, tests/test_cuda.cpp:707-716."""
    i = np.arange(out_features * in_features, dtype=np.int64)
    v = (((i + seed) % 19) - 9) * 0.0078125
    return bf16_words(v.astype(np.float32)).reshape(out_features, in_features)


def bf16_gemv_qwen_case(out_features: int, in_features: int):
    """check_bf16_gemv_qwen_case, tests/test_cuda.cpp:718-735."""
    w = make_gemv_weight(out_features, in_features, 5)
    c = np.arange(in_features)
    x = bf16_words((((c % 11) - 5) * 0.015625).astype(np.float32))
    r = np.arange(out_features)
    b = bf16_words((((r % 7) - 3) * 0.03125).astype(np.float32))
    return w, x, b


# tests/test_cuda.cpp:778-785 as (N, K, bias).
BF16_GEMV_QWEN_CASES = ((896, 896, True), (128, 896, True), (4864, 896, False),
                        (896, 4864, False), (1024, 1024, True), (897, 896, False),
                        (3, 1024, False), (512, 70, True))


def lm_head_fused_case(vocab: int, hidden: int, tie_a: int, tie_b: int):
    """check_lm_head_fused_case, tests/test_cuda.cpp:790-804.

    Returns (E bf16 [V,K], h bf16 [K]); rows tie_a and tie_b are all 2.0 and
    h[0] = 100, so those two rows tie for the maximum.
    """
    e = make_gemv_weight(vocab, hidden, 11)
    e[tie_a, :] = bf16_words(np.float32(2.0))
    e[tie_b, :] = bf16_words(np.float32(2.0))
    c = np.arange(hidden)
    h = (((c % 13) - 6) * 0.0234375).astype(np.float32)
    h[0] = 100.0
    return e, bf16_words(h)


# tests/test_cuda.cpp:875-879 as (V, K, tie_a, tie_b).
LM_HEAD_TIE_CASES = ((512, 64, 3, 4), (1002, 64, 7, 71), (200, 10, 5, 22),
                     (8, 4, 0, 3), (64, 896, 1, 31))


def linear_benchmark_input(tokens: int, in_features: int) -> np.ndarray:
    """make_input, tools/linear_benchmark.cpp:127-135."""
    i = np.arange(tokens * in_features, dtype=np.int64)
    v = (((i * 17 + 3) % 31) - 15) * 0.00390625
    return bf16_words(v.astype(np.float32)).reshape(tokens, in_features)


# ------------------------------------------------- BASELINE distributions --

def philox(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.Philox(seed))


def w8a16_synthetic(rng: np.random.Generator, n: int, k: int):
    """Config 1/3 weights: q ~ U{-127..127}, s = bf16(|N(0, 0.02)| / 127)."""
    q = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    s = np.abs(rng.normal(0.0, 0.02, size=(n, -(-k // GROUP)))) / 127.0
    return q, bf16_words(s.astype(np.float32))


def bf16_normal(rng: np.random.Generator, shape, std: float = 1.0) -> np.ndarray:
    return bf16_words(rng.normal(0.0, std, size=shape).astype(np.float32))
