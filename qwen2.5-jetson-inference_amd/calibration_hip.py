"""ctypes bindings of libinfer_calib.so, the measurement aids bench.py uses
next to the Linear library: a read-only streaming kernel, an empty kernel and
the compute-unit probes (csrc/calibration.hip).  Not part of the Linear ABI.  There is no fallback:
if the library is missing, load() raises."""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libinfer_calib.so")
EXPORTED_SYMBOLS = ("infer_calib_stream_read", "infer_calib_empty", "infer_calib_cu_probe")
_lib = None


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built (run __graft_entry__.build())")
        lib = ctypes.CDLL(LIB_PATH)
        lib.infer_calib_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
                                                ctypes.c_int, ctypes.c_void_p]
        lib.infer_calib_stream_read.restype = ctypes.c_int
        lib.infer_calib_empty.argtypes = [ctypes.c_int, ctypes.c_void_p]
        lib.infer_calib_empty.restype = ctypes.c_int
        lib.infer_calib_cu_probe.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                             ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                             ctypes.c_void_p, ctypes.c_void_p]
        lib.infer_calib_cu_probe.restype = ctypes.c_int
        _lib = lib
    return _lib


def _stream(stream):
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    return stream if isinstance(stream, int) else stream.cuda_stream


def stream_read(data, sink, blocks: int, nbytes: int | None = None, stream=None) -> None:
    """Reads the first `nbytes` (default: all) of the contiguous device tensor
    `data` with `blocks` workgroups; `sink` is a device tensor of at least
    one int32 that is never written for an equal-word fill."""
    nbytes = data.numel() * data.element_size() if nbytes is None else nbytes
    if not data.is_contiguous() or nbytes > data.numel() * data.element_size() or sink.numel() < 1:
        raise ValueError("stream_read: contiguous data of at least nbytes and a sink are needed")
    rc = load().infer_calib_stream_read(data.data_ptr(), nbytes, sink.data_ptr(), blocks,
                                        _stream(stream))
    if rc != 0:
        raise ValueError(f"infer_calib_stream_read: status {rc}")


def empty(blocks: int, stream=None) -> None:
    rc = load().infer_calib_empty(blocks, _stream(stream))
    if rc != 0:
        raise ValueError(f"infer_calib_empty: status {rc}")


# Compute-unit probe kinds (csrc/calibration.hip) and, per wave and loop
# iteration, the LDS bytes they move and the MFMAs and FMAs they issue.
CU_PROBES = {
    "lds_read": (0, 8192, 0, 0),
    "lds_write": (1, 8192, 0, 0),
    "mfma": (2, 0, 16, 0),
    "mfma_fold": (3, 0, 16, 64),
    "mfma_beside_lds_read": (4, 8192, 8, 0),
    "mfma_fold_4_partials": (5, 0, 16, 64),
    "mfma_fold_interleaved": (6, 0, 16, 64),
    "fill_direct_to_lds": (7, 8192, 0, 0),
    "fill_through_registers": (8, 8192, 0, 0),
    "lds_write_b64": (9, 4096, 0, 0),
}


def cu_probe(name: str, blocks: int, threads: int, iters: int, cycles, sink, src=None,
             stream=None) -> None:
    """Runs probe `name` on `blocks` workgroups of `threads`; `cycles` is an
    int64 device tensor of 2 * blocks entries that receives each block's
    shader-clock and 100 MHz-clock deltas; the fill probes read `src`, a
    device tensor of at least 1 MiB."""
    if cycles.numel() < 2 * blocks or cycles.element_size() != 8 or sink.numel() < 1:
        raise ValueError("cu_probe: cycles needs 2 * blocks int64 entries and a sink")
    if src is not None and src.numel() * src.element_size() < (1 << 20):
        raise ValueError("cu_probe: src must hold at least 1 MiB")
    rc = load().infer_calib_cu_probe(CU_PROBES[name][0], blocks, threads, iters,
                                     src.data_ptr() if src is not None else None,
                                     cycles.data_ptr(), sink.data_ptr(), _stream(stream))
    if rc != 0:
        raise ValueError(f"infer_calib_cu_probe: status {rc}")
