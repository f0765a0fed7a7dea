"""Python binding of the QWENBIN1 archive C ABI (include/infer_archive.h).

:class:`ModelArchive` mirrors the reference's ``infer::ModelArchive``
(include/infer/archive.hpp:22-52, src/archive.cpp:49-124): ``records``,
``record``, ``contains``, ``data``, ``data_offset``, ``mapped_bytes`` and
``path`` keep their meaning, and a bad file raises
:class:`linear_hip.InferError` with the reference's message where it throws
``infer::Error``.  :func:`export` is ``export()`` of the reference's
tools/export_model.py:273-396 over in-memory FP32 tensors (the safetensors
reading stays with the caller), and :func:`load_config` is
``ModelConfig::load`` (src/model_config.cpp:15-37).  All of it runs on the
host, in the C++ library.
"""
from __future__ import annotations

import ctypes
import dataclasses
import os

import numpy as np

import linear_hip
from linear_hip import InferError, _check
from synthetic import ModelConfig

MAX_DIMS = 8
DTYPES = {0: "float32", 1: "bfloat16", 2: "int8"}
NUMPY_DTYPES = {"float32": np.float32, "bfloat16": np.uint16, "int8": np.int8}

EXPORTED_SYMBOLS = (
    "infer_hip_archive_open",
    "infer_hip_archive_close",
    "infer_hip_archive_tensor_count",
    "infer_hip_archive_record",
    "infer_hip_archive_find",
    "infer_hip_archive_data",
    "infer_hip_archive_data_offset",
    "infer_hip_archive_mapped_bytes",
    "infer_hip_archive_verify",
    "infer_hip_archive_precision",
    "infer_hip_archive_export",
    "infer_hip_model_config_load",
    "infer_hip_model_open",
)


class _Record(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("ndim", ctypes.c_int),
                ("shape", ctypes.c_int64 * MAX_DIMS), ("dtype", ctypes.c_int),
                ("offset", ctypes.c_uint64), ("nbytes", ctypes.c_uint64),
                ("quant_group_size", ctypes.c_int), ("quant_axis", ctypes.c_int),
                ("scale_tensor", ctypes.c_char_p), ("sha256", ctypes.c_char_p)]


class _ExportTensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("ndim", ctypes.c_int),
                ("shape", ctypes.POINTER(ctypes.c_int64)),
                ("data", ctypes.POINTER(ctypes.c_float))]


class _Report(ctypes.Structure):
    _fields_ = [("tensor_count", ctypes.c_int), ("quantized_count", ctypes.c_int),
                ("int8_count", ctypes.c_int), ("bfloat16_count", ctypes.c_int),
                ("float32_count", ctypes.c_int), ("max_groupwise_abs_error", ctypes.c_double),
                ("max_bfloat16_abs_error", ctypes.c_double), ("bytes", ctypes.c_uint64)]


class _Config(ctypes.Structure):
    _fields_ = [("hidden_size", ctypes.c_int), ("intermediate_size", ctypes.c_int),
                ("num_layers", ctypes.c_int), ("num_heads", ctypes.c_int),
                ("num_kv_heads", ctypes.c_int), ("vocab_size", ctypes.c_int),
                ("eos_token_id", ctypes.c_int), ("rms_norm_eps", ctypes.c_float),
                ("rope_theta", ctypes.c_float)]


_bound = False


def load():
    global _bound
    lib = linear_hip.load()
    if _bound:
        return lib
    p, i, cp = ctypes.c_void_p, ctypes.c_int, ctypes.c_char_p
    sigs = {
        "infer_hip_archive_open": ([cp, ctypes.POINTER(p)], i),
        "infer_hip_archive_close": ([p], i),
        "infer_hip_archive_tensor_count": ([p], i),
        "infer_hip_archive_record": ([p, i, ctypes.POINTER(_Record)], i),
        "infer_hip_archive_find": ([p, cp], i),
        "infer_hip_archive_data": ([p, i], p),
        "infer_hip_archive_data_offset": ([p], ctypes.c_uint64),
        "infer_hip_archive_mapped_bytes": ([p], ctypes.c_size_t),
        "infer_hip_archive_verify": ([p], i),
        "infer_hip_archive_precision": ([p], cp),
        "infer_hip_archive_export": ([cp, cp, i, ctypes.POINTER(_ExportTensor), i, cp,
                                      ctypes.POINTER(_Report)], i),
        "infer_hip_model_config_load": ([cp, ctypes.POINTER(_Config),
                                         ctypes.POINTER(ctypes.c_int)], i),
    }
    for name, (args, res) in sigs.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    _bound = True
    return lib


@dataclasses.dataclass(frozen=True)
class QuantizationInfo:
    """include/infer/archive.hpp:7-11."""
    group_size: int
    axis: int
    scale_tensor: str


@dataclasses.dataclass(frozen=True)
class TensorRecord:
    """include/infer/archive.hpp:13-20 (plus the recorded SHA-256)."""
    name: str
    shape: tuple
    dtype: str
    offset: int
    nbytes: int
    quant: QuantizationInfo | None
    sha256: str


def _path(path) -> bytes:
    return os.fsencode(os.fspath(path))


class ModelArchive:
    """A mapped QWENBIN1 file (the reference's ``infer::ModelArchive``)."""

    def __init__(self, path):
        lib = load()
        self._lib = lib
        self._h = ctypes.c_void_p()
        self.path = os.fspath(path)
        _check(lib.infer_hip_archive_open(_path(path), ctypes.byref(self._h)))
        self.records = []
        for k in range(lib.infer_hip_archive_tensor_count(self._h)):
            r = _Record()
            _check(lib.infer_hip_archive_record(self._h, k, ctypes.byref(r)))
            quant = None
            if r.quant_group_size:
                quant = QuantizationInfo(r.quant_group_size, r.quant_axis,
                                         r.scale_tensor.decode())
            self.records.append(TensorRecord(
                r.name.decode(), tuple(r.shape[d] for d in range(r.ndim)), DTYPES[r.dtype],
                r.offset, r.nbytes, quant, r.sha256.decode()))
        self._index = {rec.name: k for k, rec in enumerate(self.records)}

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.infer_hip_archive_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _handle(self):
        if not self._h:
            raise InferError(linear_hip.INVALID_ARGUMENT, "archive is closed")
        return self._h

    def contains(self, name: str) -> bool:
        return name in self._index

    def record(self, name: str) -> TensorRecord:
        if name not in self._index:
            raise InferError(linear_hip.INVALID_ARGUMENT, "missing tensor: " + name)
        return self.records[self._index[name]]

    def data(self, name: str) -> np.ndarray:
        """The payload as a numpy array of the record's shape (BF16 as uint16
        words), copied out of the mapping."""
        rec = self.record(name)
        ptr = self._lib.infer_hip_archive_data(self._handle(), self._index[name])
        raw = (ctypes.c_uint8 * rec.nbytes).from_address(ptr) if rec.nbytes else b""
        arr = np.frombuffer(bytearray(raw), dtype=NUMPY_DTYPES[rec.dtype])
        return arr.reshape(rec.shape)

    @property
    def data_offset(self) -> int:
        return self._lib.infer_hip_archive_data_offset(self._handle())

    @property
    def mapped_bytes(self) -> int:
        return self._lib.infer_hip_archive_mapped_bytes(self._handle())

    @property
    def precision(self) -> str:
        return self._lib.infer_hip_archive_precision(self._handle()).decode()

    def verify(self) -> None:
        """verify_archive (tools/export_model.py:148-199): alignment and the
        SHA-256 of every payload; raises InferError on a mismatch."""
        _check(self._lib.infer_hip_archive_verify(self._handle()))


def export(tensors, destination, precision: str, group_size: int = 64,
           source: str = "") -> dict:
    """Write a QWENBIN1 archive of `tensors` (name -> FP32 array, in file
    order) at `destination`; returns the report's counts and errors."""
    lib = load()
    items = list(tensors.items())
    arrays, shapes = [], []
    table = (_ExportTensor * max(1, len(items)))()
    for k, (name, value) in enumerate(items):
        a = np.ascontiguousarray(value, dtype=np.float32)
        shape = (ctypes.c_int64 * max(1, a.ndim))(*a.shape)
        arrays.append(a)
        shapes.append(shape)
        table[k] = _ExportTensor(name.encode(), a.ndim, shape,
                                 a.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
    report = _Report()
    _check(lib.infer_hip_archive_export(_path(destination), precision.encode(), group_size,
                                        table, len(items), source.encode(),
                                        ctypes.byref(report)))
    return {
        "precision": precision,
        "bytes": report.bytes,
        "tensor_count": report.tensor_count,
        "quantized_tensor_count": report.quantized_count,
        "dtype_counts": {"int8": report.int8_count, "bfloat16": report.bfloat16_count,
                         "float32": report.float32_count},
        "bfloat16_tensor_count": report.bfloat16_count,
        "max_groupwise_abs_error": report.max_groupwise_abs_error,
        "max_bfloat16_abs_error": report.max_bfloat16_abs_error,
    }


def load_config(path) -> tuple[ModelConfig, int]:
    """ModelConfig::load: (config, max_position_embeddings)."""
    lib = load()
    c = _Config()
    max_pos = ctypes.c_int()
    _check(lib.infer_hip_model_config_load(_path(path), ctypes.byref(c), ctypes.byref(max_pos)))
    cfg = ModelConfig(c.hidden_size, c.intermediate_size, c.num_layers, c.num_heads,
                      c.num_kv_heads, c.vocab_size, c.eos_token_id, c.rms_norm_eps,
                      c.rope_theta)
    return cfg, max_pos.value
