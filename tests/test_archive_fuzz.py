"""Hostile QWENBIN1 archives and config.json files (truncated, corrupted and
crafted) against the HIP library's C++ reader and config loader
(include/infer_archive.h) and their restatement (oracle/archive_oracle.py).

On every input the two accept or reject together.  A rejection carries the
same message where the reference has one (src/archive.cpp:58-99,
src/model_config.cpp:19-20, 39-46), and an "archive metadata: ..." /
"model config: ..." message on both sides otherwise.  An accepted archive
yields the same records and payload bytes on both sides, every one inside
the mapped file.  Host only; tests/test_sanitizers.py runs this file again
against the ASan/UBSan build of the library."""
import json
import random
import struct

import numpy as np
import pytest

import archive_oracle as ao

HEADER = struct.Struct("<8sIIQQ")
I32 = (-2 ** 31, 2 ** 31 - 1)


@pytest.fixture(scope="module")
def arc(hip):
    import archive_hip
    archive_hip.load()
    return archive_hip


# ------------------------------------------------------------- archives --

def _base_meta():
    """Three records: an int8 weight with its quant record, its BF16 group
    scales and an FP32 bias (the shapes of a W8A16 Linear, tools/
    export_model.py:229-246)."""
    return {"format": "QWENBIN1", "version": 1, "precision": "w8a16", "tensors": [
        {"name": "w", "shape": [3, 128], "dtype": "int8", "offset": 0, "nbytes": 384,
         "quant": {"group_size": 64, "axis": 1, "scale_tensor": "w.scale"},
         "sha256": "0" * 64},
        {"name": "w.scale", "shape": [3, 2], "dtype": "bfloat16", "offset": 384, "nbytes": 12},
        {"name": "b", "shape": [3], "dtype": "float32", "offset": 512, "nbytes": 12}]}


PAYLOAD = bytes(np.random.default_rng(7).integers(0, 256, 524, dtype=np.uint8))


def _blob(meta, payload=PAYLOAD, data_offset=1024, json_size=None, magic=b"QWENBIN1",
          version=1, reserved=0):
    text = meta if isinstance(meta, bytes) else json.dumps(
        meta, separators=(",", ":"), ensure_ascii=False).encode()
    size = len(text) if json_size is None else json_size
    head = HEADER.pack(magic, version, size, data_offset, reserved) + text
    assert len(head) <= 1024, "metadata larger than the fixture's data offset"
    return head + b"\0" * (1024 - len(head)) + payload


def _cpp(arc, path):
    try:
        with arc.ModelArchive(path) as a:
            mapped, base = a.mapped_bytes, a.data_offset
            out = []
            for r in a.records:
                assert base + r.offset + r.nbytes <= mapped, r
                out.append((r, a.data(r.name).tobytes()))
            return "ok", out
    except arc.InferError as e:
        return "err", str(e)


def _restated(blob):
    try:
        recs = ao.read(blob)
    except ValueError as e:
        return "err", str(e)
    return "ok", recs


def _same(arc, tmp_path, blob, tag="x"):
    """Opens `blob` with both readers and checks that they agree; returns
    the outcome ("ok" or "err", detail)."""
    path = tmp_path / f"{tag}.qbin"
    path.write_bytes(blob)
    got, want = _cpp(arc, path), _restated(blob)
    assert got[0] == want[0], (got, want)
    if got[0] == "err":
        if want[1].startswith("archive metadata:"):
            assert "archive metadata:" in got[1], (got, want)
        else:
            assert want[1] in got[1], (got, want)
        return got
    assert [r.name for r, _ in got[1]] == list(want[1]), (got, want)
    for r, payload in got[1]:
        item, data = want[1][r.name]
        assert list(r.shape) == list(item["shape"])
        assert (r.dtype, r.offset, r.nbytes) == (item["dtype"], item["offset"], item["nbytes"])
        sha = item.get("sha256")
        assert r.sha256 == (sha if isinstance(sha, str) else "")
        if "quant" in item:
            q = item["quant"]
            assert (r.quant.group_size, r.quant.axis, r.quant.scale_tensor) == (
                q["group_size"], q.get("axis", 1), q["scale_tensor"])
        else:
            assert r.quant is None
        assert payload == data.tobytes()
    return got


def test_base_fixture_is_accepted(arc, tmp_path):
    status, recs = _same(arc, tmp_path, _blob(_base_meta()))
    assert status == "ok" and [r.name for r, _ in recs] == ["w", "w.scale", "b"]


def test_every_truncation(arc, tmp_path):
    # Every prefix of the file: header, metadata and each payload cut short.
    blob = _blob(_base_meta())
    outcomes = set()
    for n in range(len(blob) + 1):
        status, detail = _same(arc, tmp_path, blob[:n])
        outcomes.add(detail.split(":")[0] if status == "err" else "ok")
    assert {"cannot mmap archive", "archive is truncated", "bad archive JSON size",
            "bad archive data offset", "tensor lies outside archive", "ok"} <= outcomes


def test_random_corruption(arc, tmp_path):
    # 1-3 bytes overwritten, mostly in the header and metadata.
    base = bytearray(_blob(_base_meta()))
    json_end = HEADER.size + HEADER.unpack_from(base)[2]
    special = b'"\\{}[],:09-+e.E \t\n\x00\x1f\x7f\x80\xbf\xc0\xc2\xe0\xed\xf0\xf4\xf5\xff'
    rng = random.Random(1234)
    outcomes = {"ok": 0, "err": 0}
    for case in range(2000):
        blob = bytearray(base)
        for _ in range(rng.randint(1, 3)):
            at = rng.randrange(json_end) if rng.random() < 0.85 else rng.randrange(len(blob))
            blob[at] = rng.choice(special) if rng.random() < 0.6 else rng.randrange(256)
        status, _ = _same(arc, tmp_path, bytes(blob), tag=f"c{case % 8}")
        outcomes[status] += 1
    assert outcomes["ok"] > 50 and outcomes["err"] > 500, outcomes


def _with(path, value):
    """The base metadata with one field replaced: path = (tensor index, key
    [, subkey]); value = raw JSON text spliced in as the field's value."""
    meta = _base_meta()
    marker = "@@MARK@@"
    target = meta["tensors"][path[0]]
    if len(path) == 3:
        target = target[path[1]]
    target[path[-1]] = marker
    return json.dumps(meta, separators=(",", ":")).replace(f'"{marker}"', value).encode()


# (raw JSON text, expected outcome): the expectation pins that each case
# means what it says; the two readers must also agree on it.
FIELD_CASES = [
    ((0, "nbytes"), "NaN", "archive metadata"),
    ((0, "nbytes"), "Infinity", "archive metadata"),
    ((0, "nbytes"), "-Infinity", "archive metadata"),
    ((0, "offset"), "00", "archive metadata"),
    ((0, "offset"), "+0", "archive metadata"),
    ((0, "offset"), ".0", "archive metadata"),
    ((0, "offset"), "0.", "archive metadata"),
    ((0, "offset"), "0.e1", "archive metadata"),
    ((0, "offset"), "0e", "archive metadata"),
    ((0, "offset"), "0x0", "archive metadata"),
    ((0, "offset"), "-0", "ok"),
    ((0, "offset"), "0.0", "archive metadata: bad offset or nbytes of w"),
    ((0, "nbytes"), "3.84e2", "archive metadata: bad offset or nbytes of w"),
    ((0, "nbytes"), "true", "archive metadata: bad offset or nbytes of w"),
    ((0, "nbytes"), "null", "archive metadata: bad offset or nbytes of w"),
    ((0, "nbytes"), '"384"', "archive metadata: bad offset or nbytes of w"),
    ((0, "offset"), "-1", "archive metadata: bad offset or nbytes of w"),
    ((0, "offset"), str(2 ** 63), "archive metadata: bad offset or nbytes of w"),
    ((0, "offset"), str(2 ** 63 - 1), "tensor lies outside archive: w"),
    ((0, "offset"), "1" * 400, "archive metadata: bad offset or nbytes of w"),
    ((0, "offset"), "1e400", "archive metadata: bad offset or nbytes of w"),
    ((0, "nbytes"), "385", "tensor size mismatch: w"),
    ((0, "offset"), "140", "ok"),
    ((0, "offset"), "141", "tensor lies outside archive: w"),
    ((0, "shape"), "[384]", "ok"),
    ((0, "shape"), "[384,1,1,1,1,1,1,1]", "ok"),
    ((0, "shape"), "[384,1,1,1,1,1,1,1,1]", "archive metadata: bad shape of w"),
    ((0, "shape"), "[-384]", "archive metadata: bad shape of w"),
    ((0, "shape"), "[384.0]", "archive metadata: bad shape of w"),
    ((0, "shape"), "[true]", "archive metadata: bad shape of w"),
    ((0, "shape"), '"384"', "archive metadata: bad shape of w"),
    ((0, "shape"), "{}", "archive metadata: bad shape of w"),
    ((0, "shape"), "[]", "tensor size mismatch: w"),
    # Shape products past 2^64: a wrapped product would match nbytes 0 or 384.
    ((0, "shape"), f"[{2 ** 32},{2 ** 32}]", "tensor size mismatch: w"),
    ((0, "shape"), f"[{2 ** 62},4]", "tensor size mismatch: w"),
    ((0, "shape"), f"[{2 ** 62 + 96},4]", "tensor size mismatch: w"),
    ((2, "shape"), f"[{2 ** 62 + 3}]", "tensor size mismatch: b"),
    ((0, "dtype"), '"float16"', "unsupported archive dtype: float16"),
    ((0, "dtype"), "8", "unsupported archive dtype: "),
    ((0, "dtype"), '"INT8"', "unsupported archive dtype: INT8"),
    ((0, "name"), "null", "archive metadata: tensor without a name"),
    ((0, "name"), "7", "archive metadata: tensor without a name"),
    ((0, "name"), '"b"', "duplicate tensor: b"),
    ((0, "name"), '"\\u00e9"', "ok"),
    ((0, "name"), '"é中"', "ok"),
    ((0, "name"), '"\\ud83d\\ude00"', "ok"),
    ((0, "name"), '"\\ud83d"', "archive metadata"),
    ((0, "name"), '"\\ude00"', "archive metadata"),
    ((0, "name"), '"\\ud83d\\u0041"', "archive metadata"),
    ((0, "name"), '"\\ud83dx"', "archive metadata"),
    ((0, "name"), '"\\u12"', "archive metadata"),
    ((0, "name"), '"\\u12G4"', "archive metadata"),
    ((0, "name"), '"\\a"', "archive metadata"),
    ((0, "name"), '"\\/\\b\\f\\n\\r\\t\\"\\\\"', "ok"),
    ((0, "name"), '"tab\there"', "archive metadata"),
    ((0, "name"), '"del\x7f"', "ok"),
    ((0, "sha256"), "5", "ok"),
    ((0, "quant", "group_size"), "0", "archive metadata: bad quant record of w"),
    ((0, "quant", "group_size"), "-64", "archive metadata: bad quant record of w"),
    ((0, "quant", "group_size"), str(2 ** 31), "archive metadata: bad quant record of w"),
    ((0, "quant", "group_size"), str(2 ** 31 - 1), "ok"),
    ((0, "quant", "group_size"), '"64"', "archive metadata: bad quant record of w"),
    ((0, "quant", "group_size"), "64.0", "archive metadata: bad quant record of w"),
    ((0, "quant", "scale_tensor"), "5", "archive metadata: bad quant record of w"),
    ((0, "quant", "axis"), "null", "archive metadata: bad quant axis of w"),
    ((0, "quant", "axis"), "1.5", "archive metadata: bad quant axis of w"),
    ((0, "quant", "axis"), str(-2 ** 31 - 1), "archive metadata: bad quant axis of w"),
    ((0, "quant", "axis"), "0", "ok"),
    ((0, "quant"), "null", "archive metadata: bad quant record of w"),
    ((0, "quant"), "[]", "archive metadata: bad quant record of w"),
    ((0, "quant"), "{}", "archive metadata: bad quant record of w"),
]


@pytest.mark.parametrize("path,value,expect", FIELD_CASES)
def test_crafted_fields(arc, tmp_path, path, value, expect):
    status, detail = _same(arc, tmp_path, _blob(_with(path, value)))
    if expect == "ok":
        assert status == "ok", detail
    else:
        assert status == "err" and expect in detail, detail


def _raw_utf8_name(raw: bytes):
    meta = json.dumps(_base_meta(), separators=(",", ":")).encode()
    return meta.replace(b'"name":"w"', b'"name":"' + raw + b'"', 1)


@pytest.mark.parametrize("raw,ok", [
    (b"\xc3\xa9", True),                 # U+00E9
    (b"\xf0\x9f\x98\x80", True),         # U+1F600
    (b"\xf4\x8f\xbf\xbf", True),         # U+10FFFF
    (b"\xc0\x80", False),                # overlong NUL
    (b"\xc1\xbf", False),                # overlong
    (b"\xe0\x80\xaf", False),            # overlong '/'
    (b"\xed\xa0\x80", False),            # encoded surrogate
    (b"\xf4\x90\x80\x80", False),        # past U+10FFFF
    (b"\xf5\x80\x80\x80", False),
    (b"\x80", False),                    # stray continuation
    (b"\xc2", False),                    # cut by the closing quote
    (b"\xe2\x82", False),
    (b"\xff", False),
])
def test_utf8_in_strings(arc, tmp_path, raw, ok):
    status, detail = _same(arc, tmp_path, _blob(_raw_utf8_name(raw)))
    assert (status == "ok") == ok, detail


def _meta_text(**extra):
    meta = _base_meta()
    meta.update(extra)
    return json.dumps(meta, separators=(",", ":")).encode()


def _nested(depth):
    return "[" * depth + "]" * depth


DOCUMENT_CASES = [
    # a repeated key keeps its last value (nlohmann::json and Python json)
    (_meta_text()[:-1] + b',"tensors":[]}', "ok"),
    (b'{"tensors":[],' + _meta_text()[1:], "ok"),
    (_meta_text().replace(b'"name":"w",', b'"name":"x","name":"w",'), "ok"),
    (b"[]", "archive metadata: no tensors array"),
    (b"null", "archive metadata: no tensors array"),
    (b'{"tensors":{}}', "archive metadata: no tensors array"),
    (b'{"tensors":[1]}', "archive metadata: tensor without a name"),
    (b'{"tensors":[]}', "ok"),
    (b' \t\r\n{"tensors":[]} \n', "ok"),
    (b'\x0c{"tensors":[]}', "archive metadata"),
    (b'\xc2\xa0{"tensors":[]}', "archive metadata"),
    (b'\xef\xbb\xbf{"tensors":[]}', "archive metadata"),
    (b'{"tensors":[]} x', "archive metadata"),
    (b'{"tensors":[]}\x00', "archive metadata"),
    (b'{"tensors":[]}{}', "archive metadata"),
    (b'{"tensors":[],}', "archive metadata"),
    (b'{"tensors":[,]}', "archive metadata"),
    (b'{"tensors" []}', "archive metadata"),
    (b"{'tensors':[]}", "archive metadata"),
    (b'{"tensors":[]', "archive metadata"),
    (b'{"tensors":tru}', "archive metadata"),
    (b'{"tensors":[],"x":nul}', "archive metadata"),
    (b'{"tensors":[],"x":[true,false,null,-1.5e-3,1E+2,0,"\\u0000"]}', "ok"),
    (b"", "archive metadata"),
    (b" ", "archive metadata"),
    # nesting: values down to depth 64 are read, deeper ones are not
    ('{"tensors":[],"x":%s}' % _nested(64), "ok"),
    ('{"tensors":[],"x":%s}' % _nested(65), "archive metadata"),
    (_nested(65), "archive metadata: no tensors array"),
    (_nested(66), "archive metadata"),
    (_nested(5000), "archive metadata"),
]


@pytest.mark.parametrize("text,expect", DOCUMENT_CASES)
def test_crafted_documents(arc, tmp_path, text, expect):
    text = text.encode() if isinstance(text, str) else text
    if len(text) > 900:  # deeper than the fixture's 1 KiB header region
        blob = HEADER.pack(b"QWENBIN1", 1, len(text), HEADER.size + len(text), 0) + text + b"\0"
    else:
        blob = _blob(text)
    status, detail = _same(arc, tmp_path, blob)
    if expect == "ok":
        assert status == "ok", detail
    else:
        assert status == "err" and expect in detail, detail


@pytest.mark.parametrize("kw,expect", [
    (dict(magic=b"QWENBIN2"), "bad archive magic"),
    (dict(magic=b"qwenbin1"), "bad archive magic"),
    (dict(version=0), "unsupported archive version"),
    (dict(version=2 ** 32 - 1), "unsupported archive version"),
    (dict(json_size=0), "archive metadata"),
    (dict(json_size=2 ** 32 - 1), "bad archive JSON size"),
    (dict(data_offset=1024 + 524), "bad archive data offset"),
    (dict(data_offset=2 ** 64 - 1), "bad archive data offset"),
    (dict(data_offset=1024 + 523), "tensor lies outside archive: w"),
    (dict(data_offset=1000), "ok"),
    (dict(data_offset=0), "ok"),
    (dict(reserved=2 ** 64 - 1), "ok"),
])
def test_crafted_headers(arc, tmp_path, kw, expect):
    status, detail = _same(arc, tmp_path, _blob(_base_meta(), **kw))
    if expect == "ok":
        assert status == "ok", detail
    else:
        assert status == "err" and expect in detail, detail


def test_json_size_at_every_length(arc, tmp_path):
    # json_size cut short or run into the zero padding and the payload.
    blob = bytearray(_blob(_base_meta()))
    n = HEADER.unpack_from(blob)[2]
    for size in list(range(0, n + 3)) + [1000, 1023 - HEADER.size, 1024 - HEADER.size,
                                         len(blob) - HEADER.size,
                                         len(blob) - HEADER.size + 1]:
        struct.pack_into("<I", blob, 12, size)
        _same(arc, tmp_path, bytes(blob), tag=f"s{size % 4}")


def test_record_wraparound_is_outside(arc, tmp_path):
    # data_offset + offset + nbytes past 2^64 must not wrap into the file.
    meta = {"tensors": [{"name": "big", "shape": [2 ** 63 - 1], "dtype": "int8",
                         "offset": 2 ** 63 - 1, "nbytes": 2 ** 63 - 1}]}
    status, detail = _same(arc, tmp_path, _blob(meta))
    assert status == "err" and "tensor lies outside archive: big" in detail


# --------------------------------------------------------- config.json --

CONFIG = {"architectures": ["Qwen2ForCausalLM"], "bos_token_id": 151643,
          "eos_token_id": 151643, "hidden_size": 896, "intermediate_size": 4864,
          "max_position_embeddings": 32768, "model_type": "qwen2", "num_attention_heads": 14,
          "num_hidden_layers": 24, "num_key_value_heads": 2, "rms_norm_eps": 1e-06,
          "rope_theta": 1000000.0, "tie_word_embeddings": True, "torch_dtype": "bfloat16",
          "vocab_size": 151936}
INT_FIELDS = ("hidden_size", "intermediate_size", "num_hidden_layers", "num_attention_heads",
              "num_key_value_heads", "vocab_size", "max_position_embeddings")


def _int32(v):
    return isinstance(v, int) and not isinstance(v, bool) and I32[0] <= v <= I32[1]


def _number(v):
    return isinstance(v, (int, float)) and not isinstance(v, bool)


def _config_restated(raw: bytes):
    """ModelConfig::load and validate (src/model_config.cpp:15-46) with the
    C++ loader's type rules: the seven sizes are JSON integers in int32
    range, optional fields take their default only when absent."""
    j = ao.parse_json(raw)
    if not isinstance(j, dict) or j.get("model_type") != "qwen2":
        raise ValueError("only model_type=qwen2 is supported")
    if not all(_int32(j.get(k)) for k in INT_FIELDS):
        raise ValueError("model config: missing or non-integer field")
    for key in ("eos_token_id", "bos_token_id"):
        if key in j and not _int32(j[key]):
            raise ValueError("model config: bad " + key)
    for key in ("rms_norm_eps", "rope_theta"):
        if key in j and not _number(j[key]):
            raise ValueError("model config: bad " + key)
    if "tie_word_embeddings" in j and not isinstance(j["tie_word_embeddings"], bool):
        raise ValueError("model config: bad tie_word_embeddings")
    hidden, inter, layers, heads, kv, vocab, max_pos = (j[k] for k in INT_FIELDS)
    if hidden <= 0 or inter <= 0 or layers <= 0:
        raise ValueError("invalid model dimensions")
    if heads <= 0 or kv <= 0 or heads % kv != 0:
        raise ValueError("invalid GQA head counts")
    if hidden % heads != 0:
        raise ValueError("invalid attention head dimension")
    if vocab <= 0:
        raise ValueError("invalid vocabulary size")

    def f32(v):  # the C++ loader's static_cast<float>(strtod(token))
        return float(np.float32(float(str(v))))

    return (hidden, inter, layers, heads, kv, vocab, j.get("eos_token_id", -1),
            f32(j.get("rms_norm_eps", 1e-6)), f32(j.get("rope_theta", 1e6)), max_pos)


def _config_same(arc, tmp_path, raw: bytes, tag="c"):
    path = tmp_path / f"{tag}.json"
    path.write_bytes(raw)
    try:
        ao.parse_json(raw)
    except ValueError:
        want = ("err", None)  # a JSON error: "model config: <parser detail>"
    else:
        try:
            want = ("ok", _config_restated(raw))
        except ValueError as e:
            want = ("err", str(e))
    try:
        cfg, max_pos = arc.load_config(path)
        got = ("ok", (cfg.hidden_size, cfg.intermediate_size, cfg.num_layers, cfg.num_heads,
                      cfg.num_kv_heads, cfg.vocab_size, cfg.eos_token_id,
                      float(np.float32(cfg.rms_norm_eps)), float(np.float32(cfg.rope_theta)),
                      max_pos))
    except arc.InferError as e:
        got = ("err", str(e))
    assert got[0] == want[0], (raw, got, want)
    if got[0] == "ok":
        assert got[1] == want[1], (raw, got, want)
    elif want[1] is None:
        assert "model config:" in got[1], (raw, got, want)
    else:
        assert want[1] in got[1], (raw, got, want)
    return got


def test_config_base_is_accepted(arc, tmp_path):
    status, values = _config_same(arc, tmp_path, json.dumps(CONFIG, indent=2).encode())
    assert status == "ok" and values[:6] == (896, 4864, 24, 14, 2, 151936)


@pytest.mark.parametrize("patch,expect", [
    ({"eos_token_id": None}, "model config: bad eos_token_id"),
    ({"eos_token_id": [151645, 151643]}, "model config: bad eos_token_id"),
    ({"bos_token_id": "x"}, "model config: bad bos_token_id"),
    ({"rms_norm_eps": "1e-6"}, "model config: bad rms_norm_eps"),
    ({"rms_norm_eps": None}, "model config: bad rms_norm_eps"),
    ({"rope_theta": True}, "model config: bad rope_theta"),
    ({"rope_theta": 10000}, "ok"),
    ({"tie_word_embeddings": 1}, "model config: bad tie_word_embeddings"),
    ({"tie_word_embeddings": False}, "ok"),
    ({"hidden_size": 896.0}, "model config: missing or non-integer field"),
    ({"hidden_size": True}, "model config: missing or non-integer field"),
    ({"hidden_size": 2 ** 31}, "model config: missing or non-integer field"),
    ({"hidden_size": -896}, "invalid model dimensions"),
    ({"num_key_value_heads": 0}, "invalid GQA head counts"),
    ({"num_attention_heads": -14}, "invalid GQA head counts"),
    ({"num_attention_heads": 2 ** 31 - 1, "num_key_value_heads": 1},
     "invalid attention head dimension"),
    ({"model_type": 2}, "only model_type=qwen2 is supported"),
    ({"model_type": "Qwen2"}, "only model_type=qwen2 is supported"),
])
def test_config_crafted_fields(arc, tmp_path, patch, expect):
    raw = json.dumps({**CONFIG, **patch}).encode()
    status, detail = _config_same(arc, tmp_path, raw)
    if expect == "ok":
        assert status == "ok", detail
    else:
        assert status == "err" and expect in detail, detail


def test_config_random_corruption(arc, tmp_path):
    base = json.dumps(CONFIG, separators=(",", ":")).encode()
    special = b'"\\{}[],:0129-+e.E \t\n\x00\x7f\x80\xc2\xed\xff'
    rng = random.Random(99)
    outcomes = {"ok": 0, "err": 0}
    for case in range(1200):
        blob = bytearray(base)
        for _ in range(rng.randint(1, 3)):
            at = rng.randrange(len(blob))
            blob[at] = rng.choice(special) if rng.random() < 0.6 else rng.randrange(256)
        if rng.random() < 0.1:
            blob = blob[:rng.randrange(len(blob) + 1)]
        status, _ = _config_same(arc, tmp_path, bytes(blob), tag=f"c{case % 8}")
        outcomes[status] += 1
    assert outcomes["ok"] > 30 and outcomes["err"] > 300, outcomes
