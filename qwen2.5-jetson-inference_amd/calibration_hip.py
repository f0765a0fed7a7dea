"""ctypes bindings of libinfer_calib.so, the measurement aids bench.py uses
next to the Linear library: a read-only streaming kernel and an empty kernel
(csrc/calibration.hip).  Not part of the Linear ABI.  There is no fallback:
if the library is missing, load() raises."""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libinfer_calib.so")
EXPORTED_SYMBOLS = ("infer_calib_stream_read", "infer_calib_empty")
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
