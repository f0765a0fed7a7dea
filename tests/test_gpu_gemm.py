"""GPU parity of the MFMA prefill GEMMs (W8A16 and BF16) through the C ABI.

Oracle: the CPU FP32 path (cpu_ops.cpp linear_fp32_batch, 108-123, restated
in oracle/) on the same bytes; for W8A16 on the exactly dequantised weights
q * s.  Bar, per output: |a - e| <= max(1e-2 |e|, 1e-3 rms(e)) (the BASELINE
north star) and at least 95 % of the BF16 words identical to bf16(e) (the
MFMA sums in FP32 like the oracle, in another order).  Dequantisation is
checked bitwise: with one-hot activation rows the GEMM returns
bf16(q[n, j] * s[n, j / 64]) exactly.
"""
import numpy as np
import pytest

import refcases as rc
from helpers import bf16_out, check_close, to_dev, words

pytestmark = pytest.mark.gpu

TILES = range(5)  # infer_hip_gemm_tile_count()
RAGGED = ((33, 100, 128), (130, 70, 192), (2, 128, 64), (200, 260, 1024), (65, 33, 4864))


def test_tile_count_matches(hip):
    assert hip.gemm_tile_count() == len(TILES) == len(hip.GEMM_TILES)


@pytest.mark.parametrize("m", (32, 128, 512))
@pytest.mark.parametrize("shape", rc.QWEN_LINEARS, ids=lambda s: s[0])
def test_config3_w8a16_gemm_synthetic(hip, orc, dev, m, shape):
    # Config 3: q ~ U{-127..127}, s = bf16(|N(0,.02)|/127), X = bf16(N(0,1)),
    # seed 3.
    name, n, k, _ = shape
    rng = rc.philox(3 + 100 * m + rc.QWEN_LINEARS.index(shape))
    q, s = rc.w8a16_synthetic(rng, n, k)
    x = rc.bf16_normal(rng, (m, k))
    exp = orc.linear_fp32_batch(orc.dequant_w8a16(q, s), None, rc.bf16_values(x))
    y = bf16_out((m, n), dev)
    hip.gemm_w8a16(to_dev(q, dev), to_dev(s, dev), 64, None, to_dev(x, dev), y, m, n, k)
    stats = check_close(words(y), exp, what=f"gemm_w8a16 {name} M={m}")
    assert stats["bit_identical"] > 0.95, stats


@pytest.mark.parametrize("m", (32, 128, 512))
@pytest.mark.parametrize("shape", rc.QWEN_LINEARS, ids=lambda s: s[0])
def test_config3_bf16_gemm_synthetic(hip, orc, dev, m, shape):
    # Config 3, W16A16 comparison: W = bf16(N(0, 0.02)), X = bf16(N(0,1)).
    name, n, k, _ = shape
    rng = rc.philox(3 + 100 * m + 10 * rc.QWEN_LINEARS.index(shape))
    w = rc.bf16_normal(rng, (n, k), 0.02)
    x = rc.bf16_normal(rng, (m, k))
    exp = orc.linear_fp32_batch(rc.bf16_values(w), None, rc.bf16_values(x))
    y = bf16_out((m, n), dev)
    hip.gemm_bf16(to_dev(w, dev), None, to_dev(x, dev), y, m, n, k)
    stats = check_close(words(y), exp, what=f"gemm_bf16 {name} M={m}")
    assert stats["bit_identical"] > 0.95, stats


@pytest.mark.parametrize("tile", TILES)
@pytest.mark.parametrize("mnk", RAGGED, ids=lambda c: "x".join(map(str, c)))
def test_every_tile_on_ragged_shapes(hip, orc, dev, tile, mnk):
    # M and N not multiples of any tile; bias on.
    m, n, k = mnk
    rng = rc.philox(70 + tile)
    q, s = rc.w8a16_synthetic(rng, n, k)
    x = rc.bf16_normal(rng, (m, k))
    b = rc.bf16_normal(rng, (n,))
    exp, _ = orc.w8a16_reference(q, s, 64, b, x)
    y = bf16_out((m, n), dev)
    hip.gemm_w8a16_tile(to_dev(q, dev), to_dev(s, dev), 64, to_dev(b, dev), to_dev(x, dev),
                        y, m, n, k, tile)
    check_close(words(y), exp, what=f"w8a16 tile {tile}")

    w = rc.bf16_normal(rng, (n, k), 0.02)
    expb = orc.bf16_linear_reference(w, b, x)
    yb = bf16_out((m, n), dev)
    hip.gemm_bf16_tile(to_dev(w, dev), to_dev(b, dev), to_dev(x, dev), yb, m, n, k, tile)
    check_close(words(yb), expb, what=f"bf16 tile {tile}")


@pytest.mark.parametrize("tile", TILES)
def test_gemm_dequant_is_bit_exact(hip, dev, tile):
    # Row i of X is e_{j_i}: Y[i, n] = bf16(q[n, j_i] * s[n, j_i / 64]) with
    # no rounding before the final BF16 one, for every chunk slot, group
    # edge and lane half of the staged columns.
    n, k = 160, 1216
    rng = rc.philox(90 + tile)
    q, s = rc.w8a16_synthetic(rng, n, k)
    q[0, :] = 127
    q[1, :] = -127
    cols = sorted({0, 1, 7, 8, 15, 16, 31, 32, 33, 63, 64, 65, 127, 128, 600, 1151, 1152,
                   1200, 1215})
    x = np.zeros((len(cols), k), np.uint16)
    for i, j in enumerate(cols):
        x[i, j] = 0x3F80  # BF16 1.0
    y = bf16_out((len(cols), n), dev)
    hip.gemm_w8a16_tile(to_dev(q, dev), to_dev(s, dev), 64, None, to_dev(x, dev), y,
                        len(cols), n, k, tile)
    got = words(y)
    for i, j in enumerate(cols):
        expect = rc.bf16_words((q[:, j].astype(np.float32)
                                * rc.bf16_values(s[:, j // 64])).astype(np.float32))
        np.testing.assert_array_equal(got[i], expect, err_msg=f"column {j}")


def test_gemm_row_matches_gemv(hip, orc, dev):
    # tools/linear_benchmark.cpp:533-542 / test_cuda.cpp:604-608: the GEMM's
    # row 0 agrees with the GEMV on the same row, within the reference bound.
    m, n, k = 128, 4864, 896
    rng = rc.philox(99)
    q, s = rc.w8a16_synthetic(rng, n, k)
    x = rc.bf16_normal(rng, (m, k))
    dq, ds, dx = to_dev(q, dev), to_dev(s, dev), to_dev(x, dev)
    y = bf16_out((m, n), dev)
    hip.gemm_w8a16(dq, ds, 64, None, dx, y, m, n, k)
    y1 = bf16_out((n,), dev)
    hip.gemv_w8a16(dq, ds, 64, None, to_dev(x[0], dev), y1, n, k)
    g, v = rc.bf16_values(words(y)[0]), rc.bf16_values(words(y1))
    assert np.all(np.abs(g - v) <= np.maximum(1.0 / 64, 0.01 * np.abs(v)))
