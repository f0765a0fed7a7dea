"""The random-init model writer (synthetic.py) against the reference
exporter's own self-tests (tools/export_model.py:414-522) and brute force."""
import numpy as np
import pytest

import synthetic as S


def test_bf16_known_answers():
    # export_model.py:414-427.
    exact = np.array([0.0, -0.0, 1.0, -2.5, np.inf, -np.inf], np.float32)
    np.testing.assert_array_equal(S.bf16_bits_to_float32(S.float32_to_bf16_bits(exact)), exact)
    tie = np.array([1.0 + 1.0 / 256.0], np.float32)
    assert int(S.float32_to_bf16_bits(tie)[0]) == 0x3F80
    assert int(S.float32_to_bf16_bits(np.nextafter(tie, np.float32(np.inf)))[0]) == 0x3F81
    assert np.isnan(S.bf16_bits_to_float32(S.float32_to_bf16_bits(np.array([np.nan],
                                                                          np.float32))))[0]
    assert S.float32_to_bf16_bits(np.array([-2.5], np.float32))[0] == 0xC020


def test_quantizer_exporter_fixture():
    # export_model.py:431-522: a [3, 70] q_proj from linspace(-0.75, 0.75)
    # with row 2's first group zeroed; scales [3, 2]; reconstruction error
    # with the stored BF16 scales <= 0.007.
    w = np.linspace(-0.75, 0.75, 210, dtype=np.float32).reshape(3, 70)
    w[2, :64] = 0.0
    q, s = S.quantize_groupwise(w, 64)
    assert q.shape == (3, 70) and s.shape == (3, 2)
    assert s[2, 0] == 1.0 and np.all(q[2, :64] == 0)
    stored = S.bf16_bits_to_float32(S.float32_to_bf16_bits(s))
    rec = np.concatenate([q[:, :64] * stored[:, :1], q[:, 64:] * stored[:, 1:]], 1)
    assert np.abs(rec - w).max() <= 0.007
    assert np.abs(q).max() == 127


def test_quantizer_brute_force():
    rng = np.random.default_rng(0)
    w = rng.normal(0, 0.02, (9, 200)).astype(np.float32)
    w[3, 64:128] = 0.0
    q, s = S.quantize_groupwise(w, 64)
    for r in range(9):
        for g in range(4):
            block = w[r, 64 * g:64 * g + 64]
            scale = np.float32(np.max(np.abs(block)) / np.float32(127.0))
            if scale == 0:
                scale = np.float32(1.0)
            assert s[r, g] == scale
            for j, v in enumerate(block):
                e = int(np.clip(np.rint(np.float32(v) / scale), -127, 127))
                assert q[r, 64 * g + j] == e


def test_random_model_layout_and_dequant():
    cfg = S.ModelConfig(hidden_size=128, intermediate_size=256, num_layers=2, num_heads=2,
                        num_kv_heads=1, vocab_size=64)
    t = S.random_model(cfg, "w8a16", seed=1)
    assert t["model.layers.1.self_attn.k_proj.weight"].shape == (64, 128)
    assert t["model.layers.1.self_attn.k_proj.weight"].dtype == np.int8
    assert t["model.layers.1.mlp.down_proj.weight.scale"].shape == (128, 4)
    assert "model.layers.0.self_attn.o_proj.bias" not in t
    f = S.dequantized_fp32(t, cfg)
    q = t["model.layers.1.mlp.down_proj.weight"].astype(np.float64)
    sc = S.bf16_bits_to_float32(t["model.layers.1.mlp.down_proj.weight.scale"]).astype(np.float64)
    exact = q * np.repeat(sc, 64, axis=1)  # the product is exact in FP32
    np.testing.assert_array_equal(f["wd"][1].astype(np.float64), exact)
    assert f["wq"].shape == (2, 128, 128) and f["bk"].shape == (2, 64)
    b = S.random_model(cfg, "w16a16", seed=1)
    assert b["model.layers.0.mlp.up_proj.weight"].dtype == np.uint16
    with pytest.raises(ValueError):
        S.random_model(cfg, "fp8")
