"""The oracle against the committed golden fixtures (float64 brute force over
the reference's own test generators, tests/golden/make_golden.py)."""
import hashlib

import numpy as np
import pytest

import refcases as rc


def _digest(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        if a is not None:
            h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def _bound(abs_sum, k):
    # FP32 sum of k terms: a statistically generous bound far below one
    # dropped term (~abs_sum / k) for the case sizes here.
    return 8.0 * np.sqrt(k) * 2.0 ** -24 * abs_sum + 1e-12


CPU_W8_CASES = (rc.W8A16_TAIL_CASES + rc.W8A16_QWEN_CASES
                + rc.W8A16_ALIGNED_K_CASES + rc.W8A16_PREFILL_CASES[:3])


@pytest.mark.parametrize("case", CPU_W8_CASES, ids=lambda c: "x".join(map(str, c)))
def test_w8a16_reference_matches_golden(orc, golden, case):
    m, n, k, bias = case
    key = f"w8a16/{m}x{n}x{k}x{int(bias)}"
    q, s, x, b = rc.w8a16_linear_case(m, n, k)
    bb = b if bias else None
    assert _digest(q, s, x, bb) == str(golden[key + "/sha256"])
    y32, y16 = orc.w8a16_reference(q, s, 64, bb, x)
    t, r = golden[key + "/tokens"], golden[key + "/rows"]
    exp, mag = golden[key + "/expected"], golden[key + "/abs_sum"]
    got = y32[t, r].astype(np.float64)
    assert np.all(np.abs(got - exp) <= _bound(mag, k)), key
    np.testing.assert_array_equal(y16, rc.bf16_words(y32))


def test_w8a16_golden_covers_all_reference_cases(golden):
    for (m, n, k, bias) in (rc.W8A16_TAIL_CASES + rc.W8A16_QWEN_CASES
                            + rc.W8A16_PREFILL_CASES + rc.W8A16_ALIGNED_K_CASES):
        assert f"w8a16/{m}x{n}x{k}x{int(bias)}/expected" in golden


@pytest.mark.parametrize("case", rc.BF16_LINEAR_CASES, ids=lambda c: "x".join(map(str, c)))
def test_bf16_reference_matches_golden(orc, golden, case):
    m, n, k, bias = case
    key = f"bf16/{m}x{n}x{k}x{int(bias)}"
    w, x, b = rc.bf16_linear_case(m, n, k)
    bb = b if bias else None
    assert _digest(w, x, bb) == str(golden[key + "/sha256"])
    y = orc.bf16_linear_reference(w, bb, x)
    t, r = golden[key + "/tokens"], golden[key + "/rows"]
    got = y[t, r].astype(np.float64)
    assert np.all(np.abs(got - golden[key + "/expected"]) <= _bound(golden[key + "/abs_sum"], k))


@pytest.mark.parametrize("case", rc.BF16_GEMV_QWEN_CASES, ids=lambda c: "x".join(map(str, c)))
def test_linear_fp32_on_bf16_gemv_cases_matches_golden(orc, golden, case):
    n, k, bias = case
    key = f"bf16gemv/{n}x{k}x{int(bias)}"
    w, x, b = rc.bf16_gemv_qwen_case(n, k)
    bb = b if bias else None
    assert _digest(w, x, bb) == str(golden[key + "/sha256"])
    y = orc.linear_fp32(rc.bf16_values(w), None if bb is None else rc.bf16_values(bb),
                        rc.bf16_values(x))
    r = golden[key + "/rows"]
    got = y[r].astype(np.float64)
    assert np.all(np.abs(got - golden[key + "/expected"]) <= _bound(golden[key + "/abs_sum"], k))
