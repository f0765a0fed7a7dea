"""Shared helpers for the GPU parity tests: uploads, downloads, tolerances."""
from __future__ import annotations

import numpy as np

import refcases as rc


def to_dev(a: np.ndarray, dev):
    """numpy int8 / uint16 (BF16 words) / float32 / int32 -> device tensor."""
    import torch
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        t = torch.from_numpy(a.view(np.int16)).view(torch.bfloat16)
    else:
        t = torch.from_numpy(a)
    return t.to(dev)


def bf16_out(shape, dev):
    import torch
    return torch.empty(shape, dtype=torch.bfloat16, device=dev)


def words(t) -> np.ndarray:
    """Device BF16 tensor -> numpy uint16 words (synchronises)."""
    import torch
    return t.detach().view(torch.int16).cpu().numpy().view(np.uint16)


def check_close(actual_words: np.ndarray, expected: np.ndarray, *, rel=1e-2,
                floor_frac=1e-3, what="output") -> dict:
    """The parity bar: per output |a - e| <= max(rel |e|, floor_frac rms(e)).

    `expected` is the oracle's FP32 (or float64) value before BF16 rounding.
    Returns statistics (max relative error, how many outputs used the floor,
    fraction of BF16 words identical to bf16(expected))."""
    a = rc.bf16_values(actual_words).astype(np.float64).ravel()
    e = np.asarray(expected, dtype=np.float64).ravel()
    assert a.shape == e.shape, (a.shape, e.shape)
    rms = float(np.sqrt(np.mean(e * e))) if e.size else 0.0
    floor = floor_frac * rms
    tol = np.maximum(rel * np.abs(e), floor)
    err = np.abs(a - e)
    bad = np.nonzero(err > tol)[0]
    assert bad.size == 0, (
        f"{what}: {bad.size}/{e.size} outside tolerance; first at {bad[0]}: "
        f"got {a[bad[0]]!r} expected {e[bad[0]]!r} (tol {tol[bad[0]]:.3g})")
    same = rc.bf16_words(e.astype(np.float32)) == np.asarray(actual_words).ravel()
    return {
        "max_rel": float(np.max(err / np.maximum(np.abs(e), 1e-30))) if e.size else 0.0,
        "floor_hits": int(np.sum(rel * np.abs(e) < floor)),
        "bit_identical": float(np.mean(same)) if e.size else 1.0,
    }


def ulp_distance_bf16(a_words, b_words) -> np.ndarray:
    """Distance in BF16 units in the last place between two word arrays."""
    def ordered(w):
        w = np.asarray(w, dtype=np.int32)
        return np.where(w & 0x8000, 0x8000 - (w & 0x7FFF), 0x8000 + w)
    return np.abs(ordered(a_words) - ordered(b_words))
