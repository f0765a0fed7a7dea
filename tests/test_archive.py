"""QWENBIN1 archives on the host: the C++ reader, exporter and config loader
of the HIP library (include/infer_archive.h) against the numpy restatement
in oracle/archive_oracle.py, and the restatement against the reference's own
fixtures (tests/test_core.cpp:23-118 and the exporter self-tests,
tools/export_model.py:414-522).  No GPU is used."""
import hashlib
import json
import os
import struct

import numpy as np
import pytest

import archive_oracle as ao


@pytest.fixture(scope="module")
def arc(hip):
    import archive_hip
    archive_hip.load()
    return archive_hip


def _self_test_tensors():
    """export_model.py:433-454."""
    t = {
        "model.embed_tokens.weight": np.linspace(-0.25, 0.25, 20, dtype=np.float32).reshape(4, 5),
        "model.layers.0.self_attn.q_proj.weight":
            np.linspace(-0.75, 0.75, 210, dtype=np.float32).reshape(3, 70),
        "model.layers.0.self_attn.q_proj.bias": np.array([0.125, -0.25, 0.5], np.float32),
        "model.norm.weight": np.linspace(0.5, 1.5, 5, dtype=np.float32),
        "lm_head.weight": np.linspace(-0.125, 0.125, 20, dtype=np.float32).reshape(4, 5),
    }
    t["model.layers.0.self_attn.q_proj.weight"][2, :64] = 0.0
    return t


def _test_core_archive(path, values=(0x3F80, 0xC020), **overrides):
    """tests/test_core.cpp:23-63: data offset 512, one BF16 record "weight" [2]
    (the metadata as nlohmann::json dumps it: sorted keys, compact)."""
    meta = {"format": "QWENBIN1", "version": 1, "precision": "w16a16",
            "tensors": [{"name": "weight", "shape": [2], "dtype": "bfloat16", "offset": 0,
                         "nbytes": 4}]}
    meta["tensors"][0].update(overrides.pop("record", {}))
    encoded = json.dumps(meta, sort_keys=True, separators=(",", ":")).encode()
    header = dict(magic=b"QWENBIN1", version=1, json_size=len(encoded), data_offset=512)
    header.update(overrides)
    blob = bytearray(struct.pack("<8sIIQQ", header["magic"], header["version"],
                                 header["json_size"], header["data_offset"], 0))
    blob += encoded
    blob += b"\0" * (512 - len(blob))
    blob += struct.pack("<2H", *values)
    with open(path, "wb") as f:
        f.write(blob)
    return bytes(blob)


# ---------------------------------------------------------------- oracle --

def test_oracle_bf16_self_test_values():
    # export_model.py:414-428
    exact = np.array([0.0, -0.0, 1.0, -2.5, np.inf, -np.inf], np.float32)
    np.testing.assert_array_equal(ao.bfloat16_to_float32(ao.float32_to_bfloat16(exact)), exact)
    tie = np.array([1.0 + 1.0 / 256.0], np.float32)
    assert int(ao.float32_to_bfloat16(tie)[0]) == 0x3F80
    above = np.nextafter(tie, np.float32(np.inf))
    assert int(ao.float32_to_bfloat16(above)[0]) == 0x3F81
    assert np.isnan(ao.bfloat16_to_float32(ao.float32_to_bfloat16(np.array([np.nan],
                                                                         np.float32)))[0])


def test_oracle_bf16_matches_torch_rounding():
    # torch's float -> bfloat16 is round-to-nearest-even: an independent
    # implementation of the same rounding for every finite input.
    import torch
    rng = np.random.default_rng(11)
    bits = rng.integers(0, 2**32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    values = bits.view(np.float32)
    values = values[np.isfinite(values)]
    ours = ao.float32_to_bfloat16(values)
    theirs = torch.from_numpy(values.copy()).to(torch.bfloat16).view(torch.int16).numpy()
    np.testing.assert_array_equal(ours, theirs.view(np.uint16))


def test_oracle_quantizer_ties_round_half_to_even():
    # A group whose max is 127 has scale 1: w / s is w itself, and the halves
    # go to the even neighbour (np.rint), not away from zero.
    w = np.zeros((1, 64), np.float32)
    w[0, :6] = [127.0, 2.5, 3.5, -2.5, -0.5, 0.5]
    q, s = ao.quantize_groupwise(w, 64)
    assert s[0, 0] == 1.0
    assert q[0, :6].tolist() == [127, 2, 4, -2, 0, 0]


def test_oracle_quantizer_invariants():
    rng = np.random.default_rng(5)
    w = rng.standard_normal((37, 200)).astype(np.float32)
    w[3, 64:128] = 0.0
    q, s = ao.quantize_groupwise(w, 64)
    assert s.shape == (37, 4)
    assert s[3, 1] == 1.0 and not q[3, 64:128].any()
    assert np.abs(q.astype(np.int32)).max() <= 127
    for g in range(4):
        b, e = g * 64, min(200, (g + 1) * 64)
        rec = q[:, b:e].astype(np.float32) * s[:, g, None]
        assert np.all(np.abs(w[:, b:e] - rec) <= s[:, g, None] * 0.5 * (1 + 1e-6))
        nz = np.abs(w[:, b:e]).max(axis=1) > 0
        assert np.all(np.abs(q[nz, b:e].astype(np.int32)).max(axis=1) == 127)


def test_oracle_export_meets_w8a16_self_test():
    # export_model.py:466-521, applied to the restatement.
    tensors = _self_test_tensors()
    blob = ao.export(tensors, "w8a16", 64)
    recs = ao.read(blob)
    assert len(recs) == 6
    dtypes = [r["dtype"] for r, _ in recs.values()]
    assert dtypes.count("int8") == 1 and dtypes.count("bfloat16") == 5
    wname = "model.layers.0.self_attn.q_proj.weight"
    wrec, q = recs[wname]
    srec, sw = recs[wname + ".scale"]
    assert wrec["quant"] == {"scheme": "symmetric_group_w8a16", "group_size": 64, "axis": 1,
                             "scale_tensor": wname + ".scale", "scale_dtype": "bfloat16"}
    assert srec["shape"] == [3, 2]
    err = ao.groupwise_max_error(tensors[wname], q, ao.bfloat16_to_float32(sw).reshape(3, 2), 64)
    assert err <= 0.007
    assert ao.bfloat16_to_float32(sw)[2, 0] == 1.0  # the zero group
    for rec, data in recs.values():
        assert rec["offset"] % 256 == 0
        assert rec["sha256"] == hashlib.sha256(data.tobytes()).hexdigest()


def test_oracle_reads_test_core_fixture(tmp_path):
    blob = _test_core_archive(tmp_path / "a.qbin")
    rec, data = ao.read(blob)["weight"]
    assert rec["dtype"] == "bfloat16" and rec["shape"] == [2] and rec["nbytes"] == 4
    assert data.tolist() == [0x3F80, 0xC020]


# ---------------------------------------------------------------- reader --

def test_reader_loads_test_core_fixture(arc, tmp_path):
    # tests/test_core.cpp:104-118 (ModelArchive.LoadsBFloat16Tensor)
    path = tmp_path / "weight.qbin"
    _test_core_archive(path)
    with arc.ModelArchive(path) as a:
        assert len(a.records) == 1
        rec = a.record("weight")
        assert rec.dtype == "bfloat16" and rec.shape == (2,) and rec.nbytes == 4
        assert rec.quant is None
        assert a.data("weight").tolist() == [0x3F80, 0xC020]
        assert a.data_offset == 512
        assert a.mapped_bytes == 516
        assert a.precision == "w16a16"
        assert a.contains("weight") and not a.contains("other")


@pytest.mark.parametrize("case,message", [
    (dict(magic=b"QWENBIN2"), "bad archive magic"),
    (dict(version=2), "unsupported archive version"),
    (dict(json_size=10_000), "bad archive JSON size"),
    (dict(data_offset=516), "bad archive data offset"),
    (dict(record={"nbytes": 6}), "tensor size mismatch: weight"),
    (dict(record={"offset": 2}), "tensor lies outside archive: weight"),
    (dict(record={"dtype": "float16"}), "unsupported archive dtype: float16"),
    (dict(record={"shape": [3]}), "tensor size mismatch: weight"),
])
def test_reader_rejects_bad_archives(arc, tmp_path, case, message):
    # src/archive.cpp:58-99; the restatement raises the same message.
    path = tmp_path / "bad.qbin"
    blob = _test_core_archive(path, **case)
    with pytest.raises(arc.InferError) as err:
        arc.ModelArchive(path)
    assert message in str(err.value)
    if case.get("json_size") is None:
        with pytest.raises(ValueError, match=message):
            ao.read(blob)


def test_reader_rejects_duplicates_empty_and_truncated(arc, tmp_path):
    meta = {"tensors": [{"name": "w", "shape": [1], "dtype": "int8", "offset": 0, "nbytes": 1},
                        {"name": "w", "shape": [1], "dtype": "int8", "offset": 0, "nbytes": 1}]}
    enc = json.dumps(meta).encode()
    blob = struct.pack("<8sIIQQ", b"QWENBIN1", 1, len(enc), 256, 0) + enc
    blob += b"\0" * (256 - len(blob)) + b"\1"
    (tmp_path / "dup.qbin").write_bytes(blob)
    with pytest.raises(arc.InferError, match="duplicate tensor: w"):
        arc.ModelArchive(tmp_path / "dup.qbin")
    with pytest.raises(ValueError, match="duplicate tensor: w"):
        ao.read(blob)
    (tmp_path / "empty.qbin").write_bytes(b"")
    with pytest.raises(arc.InferError, match="cannot mmap archive"):
        arc.ModelArchive(tmp_path / "empty.qbin")
    (tmp_path / "short.qbin").write_bytes(b"QWENBIN1")
    with pytest.raises(arc.InferError, match="archive is truncated"):
        arc.ModelArchive(tmp_path / "short.qbin")
    with pytest.raises(arc.InferError, match="cannot open archive"):
        arc.ModelArchive(tmp_path / "missing.qbin")
    (tmp_path / "json.qbin").write_bytes(struct.pack("<8sIIQQ", b"QWENBIN1", 1, 3, 64, 0)
                                         + b"{x}" + b"\0" * 40)
    with pytest.raises(arc.InferError, match="archive metadata"):
        arc.ModelArchive(tmp_path / "json.qbin")


def test_reader_quant_axis_defaults_to_one(arc, tmp_path):
    meta = {"tensors": [{"name": "w", "shape": [1, 64], "dtype": "int8", "offset": 0,
                         "nbytes": 64, "quant": {"group_size": 64, "scale_tensor": "w.scale"}}]}
    enc = json.dumps(meta).encode()
    blob = struct.pack("<8sIIQQ", b"QWENBIN1", 1, len(enc), 256, 0) + enc
    blob += b"\0" * (256 - len(blob)) + bytes(range(64))
    (tmp_path / "q.qbin").write_bytes(blob)
    with arc.ModelArchive(tmp_path / "q.qbin") as a:
        assert a.record("w").quant == arc.QuantizationInfo(64, 1, "w.scale")
        assert a.data("w").tolist() == [list(range(64))]


# -------------------------------------------------------------- exporter --

def test_export_meets_w8a16_self_test(arc, tmp_path):
    # export_model.py:466-521 on the C++ exporter.
    tensors = _self_test_tensors()
    path = tmp_path / "model.w8a16.qbin"
    report = arc.export(tensors, path, "w8a16", 64)
    assert report["precision"] == "w8a16"
    assert report["quantized_tensor_count"] == 1
    assert report["tensor_count"] == 6
    assert report["dtype_counts"]["int8"] == 1
    assert report["dtype_counts"]["bfloat16"] == 5
    assert report["max_groupwise_abs_error"] <= 0.007
    with arc.ModelArchive(path) as a:
        a.verify()
        wname = "model.layers.0.self_attn.q_proj.weight"
        w = a.record(wname)
        assert w.dtype == "int8"
        assert w.quant == arc.QuantizationInfo(64, 1, wname + ".scale")
        s = a.record(wname + ".scale")
        assert s.dtype == "bfloat16" and s.shape == (3, 2)
        for name in ("model.embed_tokens.weight", "model.norm.weight", "lm_head.weight"):
            assert a.record(name).dtype == "bfloat16"
        scales = ao.bfloat16_to_float32(a.data(wname + ".scale")).reshape(3, 2)
        err = ao.groupwise_max_error(tensors[wname], a.data(wname), scales, 64)
        assert abs(err - report["max_groupwise_abs_error"]) < 1e-12
    blob = path.read_bytes()
    _, _, json_size, data_offset, _ = struct.unpack_from("<8sIIQQ", blob)
    meta = json.loads(blob[32:32 + json_size])
    assert meta["precision"] == "w8a16" and meta["group_size"] == 64
    assert data_offset == 1 << 20


@pytest.mark.parametrize("precision", ["w8a16", "w16a16", "fp32"])
def test_export_is_byte_identical_to_restatement(arc, tmp_path, precision):
    tensors = _self_test_tensors()
    path = tmp_path / "m.qbin"
    arc.export(tensors, path, precision, 64, source="/models/qwen-ü\n\t\"x\"")
    expected = ao.export(tensors, precision, 64, source="/models/qwen-ü\n\t\"x\"")
    assert path.read_bytes() == expected


def _random_tensors(seed=3):
    rng = np.random.default_rng(seed)
    t = {
        "model.embed_tokens.weight": rng.standard_normal((64, 96)).astype(np.float32),
        "model.layers.0.input_layernorm.weight": rng.standard_normal(96).astype(np.float32),
        "model.layers.0.mlp.down_proj.weight": rng.standard_normal((96, 200)).astype(np.float32),
        "model.layers.0.self_attn.k_proj.bias": rng.standard_normal(32).astype(np.float32),
        "model.layers.0.self_attn.k_proj.weight":
            (rng.standard_normal((32, 128)) * 1e-3).astype(np.float32),
        "scalar_like": np.array([3.0], np.float32),
        "three_d": rng.standard_normal((2, 3, 4)).astype(np.float32),
        "empty": np.zeros((0, 64), np.float32),
    }
    w = t["model.layers.0.mlp.down_proj.weight"]
    w[0, :] = 0.0                                  # zero groups -> scale 1
    w[1, :64] = np.arange(64) - 31.5               # exact halves after scaling
    w[2, 5] = np.float32(1e-30)                    # tiny scale
    w[3, 64:128] = np.float32(3.0e38)              # huge values
    w[4, 130] = -0.0
    return t


@pytest.mark.parametrize("precision", ["w8a16", "w16a16", "fp32"])
def test_export_random_tensors_byte_identical(arc, tmp_path, precision):
    tensors = _random_tensors()
    path = tmp_path / "r.qbin"
    report = arc.export(tensors, path, precision, 64, source="synthetic")
    expected = ao.export(tensors, precision, 64, source="synthetic")
    blob = path.read_bytes()
    assert blob == expected
    assert report["bytes"] == len(blob)
    with arc.ModelArchive(path) as a:
        a.verify()
        for rec in a.records:
            raw = a.data(rec.name).tobytes()
            assert rec.sha256 == hashlib.sha256(raw).hexdigest()


def test_export_matches_synthetic_quantizer(arc, tmp_path):
    # The random-init model builder quantises with its own numpy code; the
    # archive path must produce the same int8 words and BF16 scales.
    import synthetic
    tensors = _random_tensors(8)
    path = tmp_path / "s.qbin"
    arc.export(tensors, path, "w8a16", 64)
    with arc.ModelArchive(path) as a:
        for name in ("model.layers.0.mlp.down_proj.weight",
                     "model.layers.0.self_attn.k_proj.weight"):
            q, s = synthetic.quantize_groupwise(tensors[name], 64)
            np.testing.assert_array_equal(a.data(name), q)
            np.testing.assert_array_equal(a.data(name + ".scale"),
                                          synthetic.float32_to_bf16_bits(s))


def test_export_nan_and_inf_in_bf16(arc, tmp_path):
    t = {"x": np.array([np.nan, np.inf, -np.inf, 1.0, np.float32(3.4e38)], np.float32)}
    path = tmp_path / "n.qbin"
    report = arc.export(t, path, "w16a16")
    assert path.read_bytes() == ao.export(t, "w16a16")
    with arc.ModelArchive(path) as a:
        words = a.data("x")
    assert words[0] & 0x0040 and (words[0] & 0x7F80) == 0x7F80
    assert words.tolist()[1:4] == [0x7F80, 0xFF80, 0x3F80]
    assert report["max_bfloat16_abs_error"] == np.inf  # 3.4e38 rounds to inf


def test_export_verify_detects_corruption(arc, tmp_path):
    path = tmp_path / "c.qbin"
    arc.export(_self_test_tensors(), path, "w8a16")
    blob = bytearray(path.read_bytes())
    blob[(1 << 20) + 3] ^= 1
    path.write_bytes(bytes(blob))
    with arc.ModelArchive(path) as a:
        with pytest.raises(arc.InferError, match="SHA-256 mismatch"):
            a.verify()


def test_export_rejects_bad_arguments(arc, tmp_path):
    with pytest.raises(arc.InferError, match="group size 64"):
        arc.export(_self_test_tensors(), tmp_path / "g.qbin", "w8a16", 32)
    with pytest.raises(arc.InferError, match="unknown precision"):
        arc.export(_self_test_tensors(), tmp_path / "g.qbin", "int4", 64)
    with pytest.raises(arc.InferError, match="cannot create"):
        arc.export(_self_test_tensors(), tmp_path / "no" / "dir" / "g.qbin", "w16a16", 64)


def test_export_empty_archive(arc, tmp_path):
    path = tmp_path / "e.qbin"
    report = arc.export({}, path, "w16a16")
    assert path.read_bytes() == ao.export({}, "w16a16")
    assert report["bytes"] == 1 << 20 and report["tensor_count"] == 0


def _int8_archive(path, payload: bytes, sha256: str):
    meta = {"tensors": [{"name": "t", "shape": [len(payload)], "dtype": "int8", "offset": 0,
                         "nbytes": len(payload), "sha256": sha256}]}
    enc = json.dumps(meta).encode()
    blob = struct.pack("<8sIIQQ", b"QWENBIN1", 1, len(enc), 512, 0) + enc
    path.write_bytes(blob + b"\0" * (512 - len(blob)) + payload + b"\0")


@pytest.mark.parametrize("payload,digest", [
    # FIPS 180-4 / NIST example messages
    (b"abc", "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"),
    (b"", "e3b0c44298fc1c149afbf4c8996fb92427ae41e4649b934ca495991b7852b855"),
    (b"abcdbcdecdefdefgefghfghighijhijkijkljklmklmnlmnomnopnopq",
     "248d6a61d20638b8e5c026930c3e6039a33ce45964ff2167f6ecedd419db06c1"),
    (b"a" * 1000000, "cdc76e5c9914fb9281a1c7e284d73e67f1809a48a497200e046d39ccc7112cd0"),
])
def test_sha256_known_answers(arc, tmp_path, payload, digest):
    # verify() recomputes the digest with the library's SHA-256.
    assert hashlib.sha256(payload).hexdigest() == digest
    path = tmp_path / "h.qbin"
    _int8_archive(path, payload, digest)
    with arc.ModelArchive(path) as a:
        a.verify()
    _int8_archive(path, payload, digest[:-1] + ("0" if digest[-1] != "0" else "1"))
    with arc.ModelArchive(path) as a:
        with pytest.raises(arc.InferError, match="SHA-256 mismatch for t"):
            a.verify()


# ---------------------------------------------------------- config.json --

QWEN25_05B_CONFIG = {
    "architectures": ["Qwen2ForCausalLM"], "attention_dropout": 0.0, "bos_token_id": 151643,
    "eos_token_id": 151645, "hidden_act": "silu", "hidden_size": 896,
    "initializer_range": 0.02, "intermediate_size": 4864, "max_position_embeddings": 32768,
    "max_window_layers": 21, "model_type": "qwen2", "num_attention_heads": 14,
    "num_hidden_layers": 24, "num_key_value_heads": 2, "rms_norm_eps": 1e-06,
    "rope_scaling": None, "rope_theta": 1000000.0, "sliding_window": 32768,
    "tie_word_embeddings": True, "torch_dtype": "bfloat16", "transformers_version": "4.43.1",
    "use_cache": True, "use_sliding_window": False, "vocab_size": 151936,
}


def test_config_loads_qwen25_05b(arc, tmp_path):
    import synthetic
    path = tmp_path / "config.json"
    path.write_text(json.dumps(QWEN25_05B_CONFIG, indent=2))
    cfg, max_pos = arc.load_config(path)
    assert max_pos == 32768
    ref = synthetic.QWEN25_0_5B
    for field in ("hidden_size", "intermediate_size", "num_layers", "num_heads",
                  "num_kv_heads", "vocab_size", "eos_token_id"):
        assert getattr(cfg, field) == getattr(ref, field), field
    assert cfg.rms_norm_eps == pytest.approx(1e-6, rel=1e-7)
    assert cfg.rope_theta == 1e6


def test_config_defaults_and_errors(arc, tmp_path):
    base = {k: QWEN25_05B_CONFIG[k] for k in (
        "model_type", "hidden_size", "intermediate_size", "num_hidden_layers",
        "num_attention_heads", "num_key_value_heads", "vocab_size", "max_position_embeddings")}
    path = tmp_path / "config.json"
    path.write_text(json.dumps(base))
    cfg, _ = arc.load_config(path)
    assert cfg.eos_token_id == -1
    assert cfg.rms_norm_eps == pytest.approx(1e-6, rel=1e-7) and cfg.rope_theta == 1e6
    # model_config.cpp:19-20, 39-46
    for patch, message in (({"model_type": "llama"}, "only model_type=qwen2"),
                           ({"num_key_value_heads": 3}, "invalid GQA head counts"),
                           ({"hidden_size": 900}, "invalid attention head dimension"),
                           ({"num_hidden_layers": 0}, "invalid model dimensions"),
                           ({"vocab_size": 0}, "invalid vocabulary size")):
        path.write_text(json.dumps({**base, **patch}))
        with pytest.raises(arc.InferError, match=message):
            arc.load_config(path)
    del base["vocab_size"]
    path.write_text(json.dumps(base))
    with pytest.raises(arc.InferError, match="missing"):
        arc.load_config(path)
    with pytest.raises(arc.InferError, match="cannot open model config"):
        arc.load_config(tmp_path / "absent.json")


# ------------------------------------------ model open: host-side errors --

def _model_dir(tmp_path, tensors, precision, config=None):
    import archive_hip
    d = tmp_path / "model"
    d.mkdir(exist_ok=True)
    (d / "config.json").write_text(json.dumps(config or {
        "model_type": "qwen2", "hidden_size": 128, "intermediate_size": 256,
        "num_hidden_layers": 1, "num_attention_heads": 2, "num_key_value_heads": 1,
        "vocab_size": 64, "max_position_embeddings": 64}))
    archive_hip.export(tensors, d / f"model.{precision}.qbin", precision, 64)
    return d


def test_model_open_rejects_before_any_device_call(arc, tmp_path):
    # Every one of these fails on the host, before an allocation.
    import model_hip
    with pytest.raises(arc.InferError, match="cannot open model config"):
        model_hip.Qwen2Model.open(tmp_path / "nowhere")
    d = _model_dir(tmp_path, {"model.norm.weight": np.ones(128, np.float32)}, "w8a16")
    with pytest.raises(arc.InferError, match="max sequence length exceeds model limit"):
        model_hip.Qwen2Model.open(d, "w8a16", max_sequence_length=65)
    with pytest.raises(arc.InferError, match="cannot open archive"):
        model_hip.Qwen2Model.open(d, "w16a16", max_sequence_length=16)
    with pytest.raises(arc.InferError, match="missing tensor: model.embed_tokens.weight"):
        model_hip.Qwen2Model.open(d, "w8a16", max_sequence_length=16)
    emb = {"model.embed_tokens.weight": np.ones((64, 128), np.float32),
           "model.norm.weight": np.ones(96, np.float32)}
    d = _model_dir(tmp_path, emb, "w8a16")
    with pytest.raises(arc.InferError, match="model.norm.weight: unexpected dtype or shape"):
        model_hip.Qwen2Model.open(d, "w8a16", max_sequence_length=16)


# ------------------------------------------------------ C++17 boundary --

def test_cpp_archive_boundary(tmp_path):
    # tests/cpp/test_archive.cpp drives include/infer/archive_hip.hpp
    # (infer::ModelArchive, infer::ModelConfig, infer::export_archive) as the
    # reference's gtest suite drives its ModelArchive; host-only.
    import subprocess
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    binary = os.path.join(root, "tests", "cpp", "test_archive")
    if not os.path.exists(binary):
        subprocess.run(["make", "-C", os.path.join(root, "tests", "cpp"), "test_archive"],
                       check=True, capture_output=True)
    out = subprocess.run([binary, str(tmp_path)], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "PASSED" in out.stdout
