"""QWENBIN1 archive restated in numpy — TEST INFRASTRUCTURE ONLY.

A byte-level restatement of the reference's exporter and reader
(Greedy-cy/qwen2.5-jetson-inference tools/export_model.py and
src/archive.cpp), used by ``tests/`` as the checker of the C++ archive code
in the HIP library.  Only ``tests/`` may import this module; the product
never does.

Pinning (each function below is checked by ``tests/test_archive.py``):
  - ``float32_to_bfloat16``: the exporter's own self_test values
    (export_model.py:414-428: exact values, the 1 + 2^-8 tie -> 0x3F80 and
    the next float -> 0x3F81, NaN stays NaN) and an exhaustive comparison
    with torch's float -> bfloat16 conversion over finite sampled inputs;
  - ``quantize_groupwise``: the W8A16 self-test fixture's assertions
    (export_model.py:431-522: counts, scale shape [3, 2], max reconstruction
    error <= 0.007, a zero group takes scale 1), half-to-even ties at known
    points, and the invariants |q| <= 127, |w - q s| <= s / 2 and
    max |q| = 127 per non-zero group;
  - ``export``: hashlib's SHA-256 of every payload, ``json.loads`` of the
    metadata, the W8A16 self-test's structural assertions, and the reader
    of the reference's test_core fixture (tests/test_core.cpp:23-118).
"""
from __future__ import annotations

import hashlib
import json
import struct

import numpy as np

# export_model.py:25-29
MAGIC = b"QWENBIN1"
VERSION = 1
FILE_HEADER = struct.Struct("<8sIIQQ")
DATA_OFFSET = 1024 * 1024
ALIGNMENT = 256
DTYPE_BYTES = {"float32": 4, "bfloat16": 2, "int8": 1}


def float32_to_bfloat16(array) -> np.ndarray:
    """export_model.py:123-131: (bits + 0x7FFF + lsb) >> 16; NaN keeps its
    high half with the quiet bit set."""
    v = np.ascontiguousarray(array, dtype=np.float32)
    bits = v.view(np.uint32).astype(np.uint64)
    out = ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(v)
    if np.any(nan):
        out[nan] = ((bits[nan] >> 16) | 0x0040).astype(np.uint16)
    return out


def bfloat16_to_float32(words) -> np.ndarray:
    """export_model.py:134-136."""
    return (np.ascontiguousarray(words, dtype="<u2").astype(np.uint32) << 16).view(np.float32)


def should_quantize(name: str, array: np.ndarray) -> bool:
    """export_model.py:220-223."""
    return array.ndim == 2 and name not in ("model.embed_tokens.weight", "lm_head.weight")


def quantize_groupwise(weight: np.ndarray, group_size: int):
    """export_model.py:226-247: per row, per group of `group_size` columns,
    scale = max|w| / 127 in float32 (1 for an all-zero group) and
    q = clip(rint(w / scale), -127, 127).  Returns (q, float32 scales)."""
    w = np.ascontiguousarray(weight, dtype=np.float32)
    rows, cols = w.shape
    groups = (cols + group_size - 1) // group_size
    q = np.empty((rows, cols), np.int8)
    scales = np.empty((rows, groups), np.float32)
    for g in range(groups):
        b, e = g * group_size, min(cols, (g + 1) * group_size)
        block = w[:, b:e]
        s = (np.max(np.abs(block), axis=1) / np.float32(127.0)).astype(np.float32)
        s = np.where(s == 0.0, np.float32(1.0), s).astype(np.float32)
        q[:, b:e] = np.clip(np.rint(block / s[:, None]), -127, 127).astype(np.int8)
        scales[:, g] = s
    return q, scales


def groupwise_max_error(weight, q, scales, group_size: int) -> float:
    """export_model.py:250-270 (max part) in float32."""
    w = np.asarray(weight, np.float32)
    cols = w.shape[1]
    worst = 0.0
    for g in range(scales.shape[1]):
        b, e = g * group_size, min(cols, (g + 1) * group_size)
        err = np.abs(w[:, b:e] - q[:, b:e].astype(np.float32) * scales[:, g, None])
        worst = max(worst, float(err.max(initial=0.0)))
    return worst


def export(tensors: dict, precision: str, group_size: int = 64, source: str = "") -> bytes:
    """export_model.py:273-368 over in-memory FP32 arrays: the whole file."""
    if precision == "w8a16" and group_size != 64:
        raise ValueError("w8a16 currently requires group size 64")
    payload = bytearray()
    records = []

    def put(name, array, dtype, quant=None):
        pad = (-len(payload)) % ALIGNMENT           # align_file, :103-108
        payload.extend(b"\0" * pad)
        raw = np.ascontiguousarray(array).tobytes()
        record = {"name": name, "shape": list(array.shape), "dtype": dtype,
                  "offset": len(payload), "nbytes": len(raw),
                  "sha256": hashlib.sha256(raw).hexdigest()}
        if quant is not None:
            record["quant"] = quant
        records.append(record)
        payload.extend(raw)

    for name, value in tensors.items():
        array = np.ascontiguousarray(value, dtype=np.float32)
        if precision == "w8a16" and should_quantize(name, array):
            q, scales = quantize_groupwise(array, group_size)
            put(name, q, "int8", {"scheme": "symmetric_group_w8a16", "group_size": group_size,
                                  "axis": 1, "scale_tensor": name + ".scale",
                                  "scale_dtype": "bfloat16"})
            put(name + ".scale", float32_to_bfloat16(scales).astype("<u2"), "bfloat16")
        elif precision in ("w16a16", "w8a16"):
            put(name, float32_to_bfloat16(array).astype("<u2"), "bfloat16")
        else:
            put(name, array.astype("<f4"), "float32")
    metadata = {"format": "QWENBIN1", "version": VERSION, "source": source,
                "precision": precision,
                "group_size": group_size if precision == "w8a16" else None,
                "tensors": records}
    encoded = json.dumps(metadata, ensure_ascii=False, separators=(",", ":")).encode("utf-8")
    if FILE_HEADER.size + len(encoded) > DATA_OFFSET:
        raise RuntimeError("archive JSON exceeds reserved header region")
    head = FILE_HEADER.pack(MAGIC, VERSION, len(encoded), DATA_OFFSET, 0) + encoded
    # output.truncate(DATA_OFFSET): the reserved region is zero and the file
    # is at least DATA_OFFSET bytes long.
    return head + b"\0" * (DATA_OFFSET - len(head)) + bytes(payload)


MAX_DEPTH = 64   # deepest value of the metadata JSON (the top level is 0)
MAX_DIMS = 8     # infer_hip_tensor_record's shape capacity (infer_archive.h)
_I64 = (-2 ** 63, 2 ** 63 - 1)
_I32 = (-2 ** 31, 2 ** 31 - 1)


class _Pairs(list):
    """An object's (key, value) pairs in file order, before duplicates fold."""


def _reject_constant(name):
    raise ValueError("bad number: " + name)


def parse_json(raw: bytes):
    """JSON text as strictly as nlohmann::json::parse reads it (the
    reference's metadata and config.json parser): RFC 8259 numbers and
    literals only (no NaN or Infinity), UTF-8 checked, \\u escapes only as
    characters or whole surrogate pairs; a repeated key keeps its last value.
    The C++ parser also bounds the nesting at MAX_DEPTH.  Raises ValueError."""
    try:
        tree = json.loads(raw.decode("utf-8"), parse_constant=_reject_constant,
                          object_pairs_hook=_Pairs)
    except (UnicodeDecodeError, ValueError, RecursionError) as e:
        raise ValueError(str(e)) from None

    def fold(v, depth):
        if depth > MAX_DEPTH:
            raise ValueError("metadata nested too deeply")
        if isinstance(v, str):
            try:
                v.encode("utf-8")
            except UnicodeEncodeError:
                raise ValueError("bad surrogate pair") from None
            return v
        if isinstance(v, _Pairs):
            out = {}
            for k, x in v:
                fold(k, depth + 1)
                out[k] = fold(x, depth + 1)
            return out
        if isinstance(v, list):
            return [fold(x, depth + 1) for x in v]
        return v

    return fold(tree, 0)


def parse_metadata(raw: bytes):
    """parse_json for the archive metadata: raises ValueError("archive
    metadata: ...")."""
    try:
        return parse_json(raw)
    except ValueError as e:
        raise ValueError("archive metadata: " + str(e)) from None


def _integer(v, bounds):
    """A JSON integer token within bounds (bool and float tokens are not)."""
    return isinstance(v, int) and not isinstance(v, bool) and bounds[0] <= v <= bounds[1]


def read(blob: bytes) -> dict:
    """ModelArchive::open (src/archive.cpp:49-102) over bytes: name ->
    (record, numpy payload); raises ValueError with the reference's message.

    Field checks run in the reference's order: name, shape, dtype, offset
    and nbytes, the size and bounds checks, the quant record, duplicates.
    A missing key or a value of the wrong JSON type raises there (nlohmann's
    at() and get<T>()); it raises "archive metadata: ..." here.  Where the
    reference's conversions would truncate a fractional size or wrap a
    negative one, both readers here reject the value, and shape products are
    exact (no 64-bit wrap)."""
    if len(blob) == 0:
        raise ValueError("cannot mmap archive")
    if len(blob) < FILE_HEADER.size:
        raise ValueError("archive is truncated")
    magic, version, json_size, data_offset, _ = FILE_HEADER.unpack_from(blob, 0)
    if magic != MAGIC:
        raise ValueError("bad archive magic")
    if version != 1:
        raise ValueError("unsupported archive version")
    if FILE_HEADER.size + json_size > len(blob):
        raise ValueError("bad archive JSON size")
    if data_offset >= len(blob):
        raise ValueError("bad archive data offset")
    meta = parse_metadata(blob[FILE_HEADER.size:FILE_HEADER.size + json_size])
    tensors = meta.get("tensors") if isinstance(meta, dict) else None
    if not isinstance(tensors, list):
        raise ValueError("archive metadata: no tensors array")
    out = {}
    np_types = {"float32": "<f4", "bfloat16": "<u2", "int8": "i1"}
    for item in tensors:
        item = item if isinstance(item, dict) else {}
        name = item.get("name")
        if not isinstance(name, str):
            raise ValueError("archive metadata: tensor without a name")
        shape = item.get("shape")
        if (not isinstance(shape, list) or len(shape) > MAX_DIMS
                or not all(_integer(d, (0, _I64[1])) for d in shape)):
            raise ValueError("archive metadata: bad shape of " + name)
        dtype = item.get("dtype")
        dtype = dtype if isinstance(dtype, str) else ""
        if dtype not in DTYPE_BYTES:
            raise ValueError("unsupported archive dtype: " + dtype)
        offset, nbytes = item.get("offset"), item.get("nbytes")
        if not (_integer(offset, (0, _I64[1])) and _integer(nbytes, (0, _I64[1]))):
            raise ValueError("archive metadata: bad offset or nbytes of " + name)
        numel = 1
        for d in shape:
            numel *= d
        if nbytes != numel * DTYPE_BYTES[dtype]:
            raise ValueError("tensor size mismatch: " + name)
        begin = data_offset + offset
        if begin + nbytes > len(blob):
            raise ValueError("tensor lies outside archive: " + name)
        if "quant" in item:
            q = item["quant"] if isinstance(item["quant"], dict) else {}
            group = q.get("group_size")
            if (not _integer(group, _I32) or group <= 0
                    or not isinstance(q.get("scale_tensor"), str)):
                raise ValueError("archive metadata: bad quant record of " + name)
            if "axis" in q and not _integer(q["axis"], _I32):
                raise ValueError("archive metadata: bad quant axis of " + name)
        if name in out:
            raise ValueError("duplicate tensor: " + name)
        data = np.frombuffer(blob, dtype=np_types[dtype], count=numel, offset=begin)
        out[name] = (item, data.reshape(shape))
    return out
