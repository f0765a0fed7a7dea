"""A model opened from a QWENBIN1 model directory (infer_hip_model_open, the
reference's Qwen2Model(model_directory, options), src/qwen2.cpp:30-78)
against the same weights handed over as tensors (infer_hip_model_create),
and against the CPU FP32 model oracle.

The archive is written by the library's own exporter from random FP32
checkpoint tensors; the weights read back from it feed the tensor path, so
both models compute with bit-identical weights and must agree bit for bit
(same kernels, same launch plans)."""
import json

import numpy as np
import pytest

import archive_hip
import model_hip
import synthetic as S

from test_gpu_model import TINY, check_step, oracle_model, prompt

pytestmark = pytest.mark.gpu


def _directory(tmp_path, cfg, precision, tied=True, seed=21):
    d = tmp_path / f"{precision}-{'tied' if tied else 'untied'}"
    d.mkdir()
    (d / "config.json").write_text(json.dumps({
        "model_type": "qwen2", "hidden_size": cfg.hidden_size,
        "intermediate_size": cfg.intermediate_size, "num_hidden_layers": cfg.num_layers,
        "num_attention_heads": cfg.num_heads, "num_key_value_heads": cfg.num_kv_heads,
        "vocab_size": cfg.vocab_size, "max_position_embeddings": 128,
        "rms_norm_eps": cfg.rms_norm_eps, "rope_theta": cfg.rope_theta,
        "tie_word_embeddings": tied}))
    source = S.random_checkpoint(cfg, seed=seed, std=0.15, tied=tied)
    archive_hip.export(source, d / f"model.{precision}.qbin", precision, 64,
                       source="random_checkpoint")
    with archive_hip.ModelArchive(d / f"model.{precision}.qbin") as a:
        tensors = {r.name: a.data(r.name) for r in a.records}
    return d, tensors


@pytest.mark.parametrize("precision", ["w8a16", "w16a16"])
@pytest.mark.parametrize("tied", [True, False], ids=["tied", "untied"])
def test_open_equals_create_from_tensors(dev, tmp_path, precision, tied):
    print(f"archive open {precision} tied={tied}", flush=True)
    d, tensors = _directory(tmp_path, TINY, precision, tied)
    opened = model_hip.Qwen2Model.open(d, precision, max_sequence_length=64, use_graph=True)
    assert opened.config.vocab_size == TINY.vocab_size
    given = model_hip.Qwen2Model(TINY, tensors, precision, max_sequence_length=64,
                                 use_graph=True)
    p = prompt(13, TINY.vocab_size, seed=2)
    a, b = opened.prefill(p), given.prefill(p)
    assert a == b
    np.testing.assert_array_equal(opened.last_logits_host(), given.last_logits_host())
    assert opened.decode_steps(20) == given.decode_steps(20)
    np.testing.assert_array_equal(opened.last_logits_host(), given.last_logits_host())
    opened.close()
    given.close()


def test_opened_model_matches_oracle(orc, dev, tmp_path):
    precision = "w8a16"
    d, tensors = _directory(tmp_path, TINY, precision, tied=True, seed=5)
    fp32 = S.dequantized_fp32(tensors, TINY)
    g = model_hip.Qwen2Model.open(d, precision, max_sequence_length=64, use_graph=False)
    o = oracle_model(orc, TINY, fp32, 64)
    p = prompt(9, TINY.vocab_size, seed=9)
    tok = g.prefill(p)
    ref_tok, ref_logits = o.prefill(p, logits=True)
    check_step(tok, g.last_logits_host(), ref_tok, ref_logits, 0.9999, "prefill")
    agree = 0
    for step in range(12):
        token = ref_tok
        tok = g.decode_next(token)
        ref_tok, ref_logits = o.decode(token, len(p) + step, logits=True)
        same, _ = check_step(tok, g.last_logits_host(), ref_tok, ref_logits, 0.9995,
                             f"step {step}")
        agree += same
    assert agree >= 10
    g.close()


def test_open_twice_and_reopen_after_close(dev, tmp_path):
    # The model owns its weight allocation: two models from one directory
    # are independent, and closing one leaves the other working.
    d, _ = _directory(tmp_path, TINY, "w8a16")
    first = model_hip.Qwen2Model.open(d, "w8a16", max_sequence_length=32)
    second = model_hip.Qwen2Model.open(d, "w8a16", max_sequence_length=32)
    p = prompt(5, TINY.vocab_size, seed=4)
    a = first.prefill(p)
    first.close()
    assert second.prefill(p) == a
    second.close()
    third = model_hip.Qwen2Model.open(d, "w8a16", max_sequence_length=32)
    assert third.prefill(p) == a
    third.close()
