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


def read(blob: bytes) -> dict:
    """ModelArchive::open (src/archive.cpp:49-102) over bytes: name ->
    (record, numpy payload); raises ValueError with the reference's message."""
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
    meta = json.loads(blob[FILE_HEADER.size:FILE_HEADER.size + json_size])
    out = {}
    np_types = {"float32": "<f4", "bfloat16": "<u2", "int8": "i1"}
    for item in meta["tensors"]:
        dtype = item["dtype"]
        if dtype not in DTYPE_BYTES:
            raise ValueError("unsupported archive dtype: " + dtype)
        numel = int(np.prod(item["shape"], dtype=np.int64))
        if item["nbytes"] != numel * DTYPE_BYTES[dtype]:
            raise ValueError("tensor size mismatch: " + item["name"])
        begin = data_offset + item["offset"]
        if begin + item["nbytes"] > len(blob):
            raise ValueError("tensor lies outside archive: " + item["name"])
        if item["name"] in out:
            raise ValueError("duplicate tensor: " + item["name"])
        data = np.frombuffer(blob, dtype=np_types[dtype], count=numel, offset=begin)
        out[item["name"]] = (item, data.reshape(item["shape"]))
    return out
