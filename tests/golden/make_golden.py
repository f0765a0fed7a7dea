"""Writes tests/golden/linear_golden.npz — run from the repository root:

    python tests/golden/make_golden.py

The fixtures are expected values for the reference's own test cases
(Greedy-cy/qwen2.5-jetson-inference tests/test_cuda.cpp; generators restated
in tests/refcases.py), computed here in float64 brute force with numpy, which
shares no code with the C oracle it is used to check.  Nothing from the
reference is imported or run.

Contents, per case key:
  <key>/sha256      SHA-256 of the generated input bytes (detects generator
                    drift between this script and the tests)
  <key>/tokens, <key>/rows   sampled output coordinates
  <key>/expected    float64 sum (+ bias) at those coordinates
  <key>/abs_sum     float64 sum of |terms| there (for error bounds)
  lm_tie/<i>/argmax expected argmax (the planted tie row with the lower index)
  bf16/in, bf16/out FP32 inputs and torch's float->bfloat16 words for them
                    (an independent implementation of RNE), plus the
                    reference self-test's known answers (export_model.py:
                    414-428, test_core.cpp:53,117-118).
"""
from __future__ import annotations

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))

import refcases as rc  # noqa: E402


def digest(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        if a is not None:
            h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def sample_coords(tokens: int, rows: int, seed: int):
    """All outputs for small cases, else rows {0, 1, N/2, N-1} plus 60 more
    drawn with Philox(seed), at tokens {0, M-1}."""
    if tokens * rows <= 4096:
        t, r = np.meshgrid(np.arange(tokens), np.arange(rows), indexing="ij")
        return t.ravel(), r.ravel()
    pick = {0, 1, rows // 2, rows - 1}
    pick.update(int(v) for v in rc.philox(seed).integers(0, rows, 60))
    rr = np.array(sorted(pick))
    tt = np.array(sorted({0, tokens - 1}))
    t, r = np.meshgrid(tt, rr, indexing="ij")
    return t.ravel(), r.ravel()


def w8a16_expected(q, s, x, b, t, r):
    k = q.shape[1]
    deq = q[r].astype(np.float64) * np.repeat(
        rc.bf16_values(s[r]).astype(np.float64), rc.GROUP, axis=1)[:, :k]
    xv = rc.bf16_values(x[t]).astype(np.float64)
    terms = deq * xv
    exp = terms.sum(axis=1)
    if b is not None:
        exp = exp + rc.bf16_values(b[r]).astype(np.float64)
    return exp, np.abs(terms).sum(axis=1)


def bf16_expected(w, x, b, t, r):
    terms = rc.bf16_values(w[r]).astype(np.float64) * rc.bf16_values(x[t]).astype(np.float64)
    exp = terms.sum(axis=1)
    if b is not None:
        exp = exp + rc.bf16_values(b[r]).astype(np.float64)
    return exp, np.abs(terms).sum(axis=1)


def main() -> None:
    out = {}
    seed = 100
    w8_cases = (rc.W8A16_TAIL_CASES + rc.W8A16_QWEN_CASES
                + rc.W8A16_PREFILL_CASES + rc.W8A16_ALIGNED_K_CASES)
    for (m, n, k, bias) in w8_cases:
        q, s, x, b = rc.w8a16_linear_case(m, n, k)
        bb = b if bias else None
        t, r = sample_coords(m, n, seed)
        seed += 1
        exp, mag = w8a16_expected(q, s, x, bb, t, r)
        key = f"w8a16/{m}x{n}x{k}x{int(bias)}"
        out[key + "/sha256"] = np.array(digest(q, s, x, bb))
        out[key + "/tokens"] = t.astype(np.int32)
        out[key + "/rows"] = r.astype(np.int32)
        out[key + "/expected"] = exp
        out[key + "/abs_sum"] = mag

    for (m, n, k, bias) in rc.BF16_LINEAR_CASES:
        w, x, b = rc.bf16_linear_case(m, n, k)
        bb = b if bias else None
        t, r = sample_coords(m, n, seed)
        seed += 1
        exp, mag = bf16_expected(w, x, bb, t, r)
        key = f"bf16/{m}x{n}x{k}x{int(bias)}"
        out[key + "/sha256"] = np.array(digest(w, x, bb))
        out[key + "/tokens"] = t.astype(np.int32)
        out[key + "/rows"] = r.astype(np.int32)
        out[key + "/expected"] = exp
        out[key + "/abs_sum"] = mag

    for (n, k, bias) in rc.BF16_GEMV_QWEN_CASES:
        w, x, b = rc.bf16_gemv_qwen_case(n, k)
        bb = b if bias else None
        t, r = sample_coords(1, n, seed)
        seed += 1
        exp, mag = bf16_expected(w, x.reshape(1, -1), bb, t, r)
        key = f"bf16gemv/{n}x{k}x{int(bias)}"
        out[key + "/sha256"] = np.array(digest(w, x, bb))
        out[key + "/tokens"] = t.astype(np.int32)
        out[key + "/rows"] = r.astype(np.int32)
        out[key + "/expected"] = exp
        out[key + "/abs_sum"] = mag

    for i, (v, k, ta, tb) in enumerate(rc.LM_HEAD_TIE_CASES):
        e, h = rc.lm_head_fused_case(v, k, ta, tb)
        full = rc.bf16_values(e).astype(np.float64) @ rc.bf16_values(h).astype(np.float64)
        key = f"lm_tie/{i}"
        out[key + "/sha256"] = np.array(digest(e, h))
        out[key + "/logits"] = full
        out[key + "/argmax"] = np.array(int(np.argmax(full)), dtype=np.int32)

    # BF16 RNE: the reference self-test's known answers, then torch's
    # conversion of special and random values.
    import torch

    tie = np.float32(1.0 + 1.0 / 256.0)
    above = np.nextafter(tie, np.float32(np.inf), dtype=np.float32)
    known_in = np.array([0.0, -0.0, 1.0, -2.5, np.inf, -np.inf, tie, above],
                        dtype=np.float32)
    known_out = np.array([0x0000, 0x8000, 0x3F80, 0xC020, 0x7F80, 0xFF80,
                          0x3F80, 0x3F81], dtype=np.uint16)
    rng = rc.philox(7)
    rand = np.concatenate([
        rng.normal(0, 1, 8000).astype(np.float32),
        rng.normal(0, 1e-3, 4000).astype(np.float32),
        (rng.integers(0, 2**32, 8000, dtype=np.uint64).astype(np.uint32)).view(np.float32),
    ])
    rand = rand[~np.isnan(rand)]
    conv = torch.from_numpy(rand.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    out["bf16/known_in"] = known_in
    out["bf16/known_out"] = known_out
    out["bf16/in"] = rand
    out["bf16/out"] = conv

    path = os.path.join(HERE, "linear_golden.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()
