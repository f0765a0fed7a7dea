"""Pins the CPU oracle (oracle/linear_oracle.c) against things other than
itself: the reference's known answers, float64 brute force, an independent
library (torch's float->bfloat16, numpy's BLAS matmul), closed forms and
invariants.  Each check is chosen so that a plausible slip (a dropped term,
a transposed operand, a wrong group index, a wrong tie rule) fails it."""
import numpy as np
import pytest

import refcases as rc


# --------------------------------------------------------------- BF16 RNE --

def test_bf16_known_answers(orc, golden):
    # export_model.py:414-428, test_core.cpp:53,117-118.
    got = orc.f32_to_bf16(golden["bf16/known_in"])
    np.testing.assert_array_equal(got, golden["bf16/known_out"])
    assert orc.bf16_to_f32(np.array([0x3F80], np.uint16))[0] == 1.0
    assert orc.bf16_to_f32(np.array([0xC020], np.uint16))[0] == -2.5


def test_bf16_nan_stays_quiet_nan(orc):
    nan_bits = np.array([0x7FC00000, 0x7F800001, 0xFF812345], np.uint32).view(np.float32)
    w = orc.f32_to_bf16(nan_bits)
    assert np.all(np.isnan(orc.bf16_to_f32(w)))
    assert np.all(w & 0x0040)


def test_bf16_matches_torch_conversion(orc, golden):
    # torch's float -> bfloat16 is an independent RNE implementation.
    np.testing.assert_array_equal(orc.f32_to_bf16(golden["bf16/in"]), golden["bf16/out"])
    np.testing.assert_array_equal(rc.bf16_words(golden["bf16/in"]), golden["bf16/out"])


def test_bf16_is_nearest_with_ties_to_even(orc):
    rng = rc.philox(11)
    x = rng.normal(0, 10, 20000).astype(np.float32)
    w = orc.f32_to_bf16(x).astype(np.int64)
    v = orc.bf16_to_f32(w.astype(np.uint16)).astype(np.float64)
    # neighbours one BF16 step either side (same sign region for normal x)
    up = orc.bf16_to_f32((w + 1).astype(np.uint16)).astype(np.float64)
    dn = orc.bf16_to_f32((w - 1).astype(np.uint16)).astype(np.float64)
    d = np.abs(x - v)
    assert np.all(d <= np.abs(x - up)) and np.all(d <= np.abs(x - dn))
    # exact midpoints go to the even word
    mids = (orc.bf16_to_f32(np.arange(0x3F80, 0x3F90, dtype=np.uint16)).astype(np.float64)
            + 2.0 ** -8)
    wm = orc.f32_to_bf16(mids.astype(np.float32))
    assert np.all(wm % 2 == 0)


# ------------------------------------------------------------ linear FP32 --

def test_linear_fp32_vs_float64_brute_force(orc):
    rng = rc.philox(3)
    for n, k in ((7, 5), (33, 130), (128, 896), (96, 4864)):
        w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
        x = rng.normal(0, 1, k).astype(np.float32)
        b = rng.normal(0, 1, n).astype(np.float32)
        y = orc.linear_fp32(w, b, x)
        ref = w.astype(np.float64) @ x.astype(np.float64) + b
        mag = np.abs(w.astype(np.float64)) @ np.abs(x.astype(np.float64)) + np.abs(b)
        assert np.all(np.abs(y - ref) <= 4 * np.sqrt(k) * 2**-24 * mag + 1e-30)


def test_linear_fp32_matches_numpy_blas(orc):
    rng = rc.philox(4)
    w = rng.normal(0, 0.02, (300, 896)).astype(np.float32)
    x = rng.normal(0, 1, 896).astype(np.float32)
    np.testing.assert_allclose(orc.linear_fp32(w, None, x), w @ x, rtol=1e-4, atol=1e-5)


def test_linear_fp32_identity_and_permutation_are_exact(orc):
    rng = rc.philox(5)
    x = rng.normal(0, 1, 64).astype(np.float32)
    np.testing.assert_array_equal(orc.linear_fp32(np.eye(64, dtype=np.float32), None, x), x)
    perm = rng.permutation(64)
    p = np.eye(64, dtype=np.float32)[perm]
    np.testing.assert_array_equal(orc.linear_fp32(p, None, x), x[perm])
    # a non-square selector catches a transposed weight: row r picks column 2r
    sel = np.zeros((32, 64), np.float32)
    sel[np.arange(32), 2 * np.arange(32)] = 1.0
    np.testing.assert_array_equal(orc.linear_fp32(sel, None, x), x[::2])


def test_linear_fp32_is_linear_in_x(orc):
    rng = rc.philox(6)
    w = rng.normal(0, 0.02, (50, 200)).astype(np.float32)
    x1 = rng.normal(0, 1, 200).astype(np.float32)
    x2 = rng.normal(0, 1, 200).astype(np.float32)
    lhs = orc.linear_fp32(w, None, (2 * x1 - 3 * x2).astype(np.float32))
    rhs = 2 * orc.linear_fp32(w, None, x1) - 3 * orc.linear_fp32(w, None, x2)
    np.testing.assert_allclose(lhs, rhs, rtol=1e-4, atol=1e-5)


def test_linear_batch_equals_per_row(orc):
    # test_ops.cpp:133-163: batched == per-row within 1e-5.
    rng = rc.philox(8)
    w = rng.normal(0, 0.02, (37, 70)).astype(np.float32)
    x = rng.normal(0, 1, (5, 70)).astype(np.float32)
    b = rng.normal(0, 1, 37).astype(np.float32)
    yb = orc.linear_fp32_batch(w, b, x)
    for t in range(5):
        np.testing.assert_allclose(yb[t], orc.linear_fp32(w, b, x[t]), atol=1e-5)


# ------------------------------------------------------------------ argmax --

def test_argmax_first_maximum(orc):
    v = np.array([1.0, 3.0, 2.0, 3.0, -1.0], np.float32)
    assert orc.argmax(v) == 1
    assert orc.argmax(np.full(10, -np.inf, np.float32)) == 0
    rng = rc.philox(9)
    r = rng.normal(size=1000).astype(np.float32)
    assert orc.argmax(r) == int(np.argmax(r))


# ------------------------------------------------------------ W8A16 dequant --

def test_dequant_is_bit_exact_product(orc):
    rng = rc.philox(10)
    q, s = rc.w8a16_synthetic(rng, 96, 4864)
    w = orc.dequant_w8a16(q, s)
    exact = q.astype(np.float64) * np.repeat(rc.bf16_values(s).astype(np.float64), 64, axis=1)
    # the product has at most 8 + 8 significant bits, so FP32 holds it exactly
    np.testing.assert_array_equal(w.astype(np.float64), exact)


def test_dequant_group_indexing_and_ragged_k(orc):
    # scale of group g is g+1: a wrong group index changes the value
    n, k = 3, 70
    q = np.ones((n, k), np.int8)
    s = rc.bf16_words(np.tile(np.array([1.0, 2.0], np.float32), (n, 1)))
    w = orc.dequant_w8a16(q, s)
    assert np.all(w[:, :64] == 1.0) and np.all(w[:, 64:] == 2.0)
    with pytest.raises(ValueError):
        orc.dequant_w8a16(q, s, group_size=0)


def test_w8a16_reference_extremes_and_zero_group(orc):
    # q = +-127 and the zeroed first group of the last row (test_cuda.cpp:
    # 532-535, 546-551) contribute exactly what the closed form says.
    q, s, x, b = rc.w8a16_linear_case(2, 7, 130)
    y32, _ = orc.w8a16_reference(q, s, 64, None, x)
    xv = rc.bf16_values(x).astype(np.float64)
    sv = rc.bf16_values(s).astype(np.float64)
    # last row: group 0 is zero, so only columns 64..129 contribute
    last = (q[-1, 64:].astype(np.float64) * np.repeat(sv[-1, 1:], 64)[:66]) @ xv[:, 64:].T
    np.testing.assert_allclose(y32[:, -1], last, rtol=1e-6)
    assert q[0, 0] == -127 and q[0, 1] == 127


# ---------------------------------------------------------------- LM head --

def test_lm_head_planted_ties_pick_lowest_index(orc, golden):
    for i, (v, k, ta, tb) in enumerate(rc.LM_HEAD_TIE_CASES):
        e, h = rc.lm_head_fused_case(v, k, ta, tb)
        l32, l16, idx = orc.lm_head(e, h)
        assert idx == ta == int(golden[f"lm_tie/{i}/argmax"])
        np.testing.assert_allclose(l32, golden[f"lm_tie/{i}/logits"], rtol=1e-5, atol=1e-4)
        np.testing.assert_array_equal(l16, rc.bf16_words(l32))
