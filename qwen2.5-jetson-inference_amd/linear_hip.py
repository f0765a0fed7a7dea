"""Python binding of the MI355X Linear hot path (``libinfer_linear.so``).

The functions mirror the reference's operator boundary,
``include/infer/cuda_ops.hpp`` (Greedy-cy/qwen2.5-jetson-inference):
same names, same argument order and meaning, raw device pointers plus a
stream.  Each argument may be a device pointer (``int``) or a contiguous
``torch`` CUDA tensor; ``None`` is a null pointer.  A nonzero status from
the C ABI raises :class:`InferError` (the reference throws ``infer::Error``,
``include/infer/common.hpp:66-82``).

There is no fallback: if the library is missing, :func:`load` raises.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
# INFER_HIP_LIBRARY names another build of the same library (the host-only
# sanitizer build the CPU tests load); by default the in-tree build.
LIB_PATH = os.environ.get("INFER_HIP_LIBRARY") or os.path.join(_HERE, "libinfer_linear.so")

OK = 0
INVALID_ARGUMENT = 1
LAUNCH_FAILED = 2
RUNTIME_ERROR = 3

# Every symbol include/infer_linear.h declares.
EXPORTED_SYMBOLS = (
    "infer_hip_last_error",
    "infer_hip_abi_version",
    "infer_hip_gemv_bf16",
    "infer_hip_gemm_bf16",
    "infer_hip_lm_head_bf16",
    "infer_hip_lm_head_bf16_noalloc",
    "infer_hip_lm_head_workspace_entries",
    "infer_hip_gemv_w8a16",
    "infer_hip_gemm_w8a16",
    "infer_hip_gemm_tile_count",
    "infer_hip_gemm_w8a16_tile",
    "infer_hip_gemm_bf16_tile",
    "infer_hip_gemm_workspace_bytes",
    "infer_hip_gemm_w8a16_ws",
    "infer_hip_gemm_bf16_ws",
    "infer_hip_w8a16_gemv_plan_create",
    "infer_hip_w8a16_gemv_plan_launch",
    "infer_hip_w8a16_gemv_plan_bytes",
    "infer_hip_w8a16_gemv_plan_destroy",
    "infer_hip_gemm_plan_create",
    "infer_hip_gemm_plan_launch",
    "infer_hip_gemm_plan_flops",
    "infer_hip_gemm_plan_destroy",
    "infer_hip_gemm_plan_timeline",
)


class W8A16GemvDesc(ctypes.Structure):
    """infer_hip_w8a16_gemv_desc: the arguments of one gemv_w8a16 call."""
    _fields_ = [
        ("weight", ctypes.c_void_p),
        ("scales", ctypes.c_void_p),
        ("group_size", ctypes.c_int),
        ("bias", ctypes.c_void_p),
        ("input", ctypes.c_void_p),
        ("output", ctypes.c_void_p),
        ("out_features", ctypes.c_int),
        ("in_features", ctypes.c_int),
    ]


class GemmDesc(ctypes.Structure):
    """infer_hip_gemm_desc: the arguments of one gemm_w8a16 / gemm_bf16 call."""
    _fields_ = [
        ("w8a16", ctypes.c_int),
        ("weight", ctypes.c_void_p),
        ("scales", ctypes.c_void_p),
        ("group_size", ctypes.c_int),
        ("bias", ctypes.c_void_p),
        ("input", ctypes.c_void_p),
        ("output", ctypes.c_void_p),
        ("tokens", ctypes.c_int),
        ("out_features", ctypes.c_int),
        ("in_features", ctypes.c_int),
    ]


class InferError(RuntimeError):
    """A nonzero status from the C ABI, with the library's message."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


_lib = None


def _hip_runtimes_mapped():
    try:
        with open("/proc/self/maps") as f:
            return sorted({line.split()[-1] for line in f
                           if "libamdhip64" in line and "/" in line})
    except OSError:
        return []


def load() -> ctypes.CDLL:
    """Load the HIP library (raises if it has not been built).

    torch (when installed) is imported first: its wheel ships its own HIP
    runtime, whose soname (libamdhip64.so.7) the library's dependency then
    resolves to, so the process holds one HIP runtime.  Two runtimes in one
    process cannot share the GPU; that case raises instead of running."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise InferError(RUNTIME_ERROR,
                         f"{LIB_PATH} is missing: run __graft_entry__.build()")
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(LIB_PATH)
    runtimes = _hip_runtimes_mapped()
    if len(runtimes) > 1:
        raise InferError(RUNTIME_ERROR,
                         "two HIP runtimes are loaded in this process: " + ", ".join(runtimes))
    p, i = ctypes.c_void_p, ctypes.c_int
    lib.infer_hip_last_error.restype = ctypes.c_char_p
    lib.infer_hip_abi_version.restype = i
    sigs = {
        "infer_hip_gemv_bf16": [p, p, p, p, i, i, p],
        "infer_hip_gemm_bf16": [p, p, p, p, i, i, i, p],
        "infer_hip_lm_head_bf16": [p, p, p, p, p, p, p, i, i, p],
        "infer_hip_lm_head_bf16_noalloc": [p, p, p, p, p, i, i, p],
        "infer_hip_gemv_w8a16": [p, p, i, p, p, p, i, i, p],
        "infer_hip_gemm_w8a16": [p, p, i, p, p, p, i, i, i, p],
        "infer_hip_gemm_w8a16_tile": [p, p, i, p, p, p, i, i, i, i, p],
        "infer_hip_gemm_bf16_tile": [p, p, p, p, i, i, i, i, p],
        "infer_hip_gemm_w8a16_ws": [p, p, i, p, p, p, i, i, i, p, ctypes.c_size_t, p],
        "infer_hip_gemm_bf16_ws": [p, p, p, p, i, i, i, p, ctypes.c_size_t, p],
    }
    for name, args in sigs.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = i
    lib.infer_hip_gemm_tile_count.argtypes = []
    lib.infer_hip_gemm_tile_count.restype = i
    lib.infer_hip_gemm_workspace_bytes.argtypes = [i, i, i]
    lib.infer_hip_gemm_workspace_bytes.restype = ctypes.c_size_t
    lib.infer_hip_lm_head_workspace_entries.argtypes = [i, i]
    lib.infer_hip_lm_head_workspace_entries.restype = ctypes.c_size_t
    lib.infer_hip_w8a16_gemv_plan_create.argtypes = [p, i, ctypes.POINTER(p)]
    lib.infer_hip_w8a16_gemv_plan_create.restype = i
    lib.infer_hip_w8a16_gemv_plan_launch.argtypes = [p, p]
    lib.infer_hip_w8a16_gemv_plan_launch.restype = i
    lib.infer_hip_w8a16_gemv_plan_bytes.argtypes = [p]
    lib.infer_hip_w8a16_gemv_plan_bytes.restype = ctypes.c_double
    lib.infer_hip_w8a16_gemv_plan_destroy.argtypes = [p]
    lib.infer_hip_w8a16_gemv_plan_destroy.restype = i
    lib.infer_hip_gemm_plan_create.argtypes = [p, i, ctypes.POINTER(p)]
    lib.infer_hip_gemm_plan_create.restype = i
    lib.infer_hip_gemm_plan_launch.argtypes = [p, p]
    lib.infer_hip_gemm_plan_launch.restype = i
    lib.infer_hip_gemm_plan_flops.argtypes = [p]
    lib.infer_hip_gemm_plan_flops.restype = ctypes.c_double
    lib.infer_hip_gemm_plan_destroy.argtypes = [p]
    lib.infer_hip_gemm_plan_destroy.restype = i
    lib.infer_hip_gemm_plan_timeline.argtypes = [p, p, i, ctypes.POINTER(i), p]
    lib.infer_hip_gemm_plan_timeline.restype = i
    _lib = lib
    return lib


def _ptr(t):
    if t is None:
        return None
    if isinstance(t, int):
        return t
    if not t.is_cuda:
        raise InferError(INVALID_ARGUMENT, "tensor must live on the GPU")
    if not t.is_contiguous():
        raise InferError(INVALID_ARGUMENT, "tensor must be contiguous")
    return t.data_ptr()


def _stream(stream):
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


def _check(status: int) -> None:
    if status != OK:
        msg = load().infer_hip_last_error().decode("utf-8", "replace")
        raise InferError(status, msg)


def gemv_bf16(weight, bias, input, output, out_features, in_features,
              stream=None):
    """cuda_ops.hpp:24-26."""
    _check(load().infer_hip_gemv_bf16(_ptr(weight), _ptr(bias), _ptr(input),
                                      _ptr(output), out_features, in_features,
                                      _stream(stream)))


def gemm_bf16(weight, bias, input, output, tokens, out_features, in_features,
              stream=None):
    """cuda_ops.hpp:32-35."""
    _check(load().infer_hip_gemm_bf16(_ptr(weight), _ptr(bias), _ptr(input),
                                      _ptr(output), tokens, out_features,
                                      in_features, _stream(stream)))


def lm_head_workspace_entries(vocab: int, in_features: int) -> int:
    return int(load().infer_hip_lm_head_workspace_entries(vocab, in_features))


def lm_head_bf16(weight, bias, input, logits, block_max_value,
                 block_max_index, argmax, vocab, in_features, stream=None):
    """cuda_ops.hpp:42-45 (argmax over FP32 sums, ties to the lowest index)."""
    _check(load().infer_hip_lm_head_bf16(
        _ptr(weight), _ptr(bias), _ptr(input), _ptr(logits),
        _ptr(block_max_value), _ptr(block_max_index), _ptr(argmax), vocab,
        in_features, _stream(stream)))


def lm_head_bf16_noalloc(weight, bias, input, logits, argmax, vocab, in_features,
                         stream=None):
    """lm_head_bf16 with the library's static device scratch instead of a
    workspace (infer_hip_lm_head_bf16_noalloc; vocab <= 1048576)."""
    _check(load().infer_hip_lm_head_bf16_noalloc(
        _ptr(weight), _ptr(bias), _ptr(input), _ptr(logits), _ptr(argmax), vocab,
        in_features, _stream(stream)))


def gemv_w8a16(weight, scales, group_size, bias, input, output, out_features,
               in_features, stream=None):
    """cuda_ops.hpp:47-50."""
    _check(load().infer_hip_gemv_w8a16(_ptr(weight), _ptr(scales), group_size,
                                       _ptr(bias), _ptr(input), _ptr(output),
                                       out_features, in_features,
                                       _stream(stream)))


def gemm_w8a16(weight, scales, group_size, bias, input, output, tokens,
               out_features, in_features, stream=None):
    """cuda_ops.hpp:51-55."""
    _check(load().infer_hip_gemm_w8a16(_ptr(weight), _ptr(scales), group_size,
                                       _ptr(bias), _ptr(input), _ptr(output),
                                       tokens, out_features, in_features,
                                       _stream(stream)))


# MFMA workgroup tiles (rows x columns of Y) of the explicit-tile entries.
GEMM_TILES = ("128x128", "128x64", "64x128", "64x64", "32x128", "256x128")


def gemm_tile_count() -> int:
    return int(load().infer_hip_gemm_tile_count())


def gemm_w8a16_tile(weight, scales, group_size, bias, input, output, tokens,
                    out_features, in_features, tile, stream=None):
    """gemm_w8a16 with the MFMA workgroup tile named (-1 = automatic)."""
    _check(load().infer_hip_gemm_w8a16_tile(_ptr(weight), _ptr(scales), group_size,
                                            _ptr(bias), _ptr(input), _ptr(output),
                                            tokens, out_features, in_features, tile,
                                            _stream(stream)))


def gemm_bf16_tile(weight, bias, input, output, tokens, out_features,
                   in_features, tile, stream=None):
    """gemm_bf16 with the MFMA workgroup tile named (-1 = automatic)."""
    _check(load().infer_hip_gemm_bf16_tile(_ptr(weight), _ptr(bias), _ptr(input),
                                           _ptr(output), tokens, out_features,
                                           in_features, tile, _stream(stream)))


def gemm_workspace_bytes(max_tokens, out_features, in_features) -> int:
    """Workspace bytes of gemm_*_ws for every token count up to max_tokens
    (0: no such call splits K)."""
    return int(load().infer_hip_gemm_workspace_bytes(max_tokens, out_features, in_features))


def _ws_args(workspace):
    """(pointer, bytes) of a workspace tensor (or None)."""
    if workspace is None:
        return None, 0
    return _ptr(workspace), workspace.numel() * workspace.element_size()


def gemm_w8a16_ws(weight, scales, group_size, bias, input, output, tokens, out_features,
                  in_features, workspace, stream=None):
    """gemm_w8a16 with a caller workspace (a zeroed device tensor of at
    least gemm_workspace_bytes bytes): long-K calls split over K."""
    wp, wb = _ws_args(workspace)
    _check(load().infer_hip_gemm_w8a16_ws(_ptr(weight), _ptr(scales), group_size, _ptr(bias),
                                          _ptr(input), _ptr(output), tokens, out_features,
                                          in_features, wp, wb, _stream(stream)))


def gemm_bf16_ws(weight, bias, input, output, tokens, out_features, in_features, workspace,
                 stream=None):
    """gemm_bf16 with a caller workspace (see gemm_w8a16_ws)."""
    wp, wb = _ws_args(workspace)
    _check(load().infer_hip_gemm_bf16_ws(_ptr(weight), _ptr(bias), _ptr(input), _ptr(output),
                                         tokens, out_features, in_features, wp, wb,
                                         _stream(stream)))


class W8A16GemvPlan:
    """A grouped W8A16 GEMV plan: ``calls`` is a sequence of
    ``(weight, scales, group_size, bias, input, output, out_features,
    in_features)`` tuples, each the arguments of one independent
    :func:`gemv_w8a16` call.  The tensors must outlive the plan."""

    def __init__(self, calls):
        calls = list(calls)
        arr = (W8A16GemvDesc * len(calls))()
        for d, c in zip(arr, calls):
            w, s, g, b, x, y, n, k = c
            d.weight, d.scales, d.group_size = _ptr(w), _ptr(s), g
            d.bias, d.input, d.output = _ptr(b), _ptr(x), _ptr(y)
            d.out_features, d.in_features = n, k
        handle = ctypes.c_void_p()
        _check(load().infer_hip_w8a16_gemv_plan_create(
            ctypes.cast(arr, ctypes.c_void_p) if calls else None, len(calls),
            ctypes.byref(handle)))
        self._handle = handle
        self.count = len(calls)

    @property
    def bytes(self) -> float:
        """Compulsory bytes one launch moves."""
        return float(load().infer_hip_w8a16_gemv_plan_bytes(self._handle))

    def launch(self, stream=None) -> None:
        _check(load().infer_hip_w8a16_gemv_plan_launch(self._handle, _stream(stream)))

    def close(self) -> None:
        if self._handle:
            _check(load().infer_hip_w8a16_gemv_plan_destroy(self._handle))
            self._handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class GemmPlan:
    """A grouped GEMM plan: ``calls`` is a sequence of W8A16 tuples
    ``(weight, scales, group_size, bias, input, output, tokens,
    out_features, in_features)`` (the arguments of :func:`gemm_w8a16`) or of
    BF16 tuples ``(weight, bias, input, output, tokens, out_features,
    in_features)`` (:func:`gemm_bf16`); all of one kind.  The tensors must
    outlive the plan."""

    def __init__(self, calls):
        calls = list(calls)
        arr = (GemmDesc * len(calls))()
        for d, c in zip(arr, calls):
            if len(c) == 9:
                w, s, g, b, x, y, m, n, k = c
                d.w8a16, d.scales, d.group_size = 1, _ptr(s), g
            else:
                w, b, x, y, m, n, k = c
                d.w8a16, d.scales, d.group_size = 0, None, 0
            d.weight, d.bias, d.input, d.output = _ptr(w), _ptr(b), _ptr(x), _ptr(y)
            d.tokens, d.out_features, d.in_features = m, n, k
        handle = ctypes.c_void_p()
        _check(load().infer_hip_gemm_plan_create(
            ctypes.cast(arr, ctypes.c_void_p) if calls else None, len(calls),
            ctypes.byref(handle)))
        self._handle = handle
        self.count = len(calls)

    @property
    def flops(self) -> float:
        return float(load().infer_hip_gemm_plan_flops(self._handle))

    def launch(self, stream=None) -> None:
        _check(load().infer_hip_gemm_plan_launch(self._handle, _stream(stream)))

    def workgroups(self) -> int:
        """Workgroups of a wide-tile plan's GEMM launch (raises on other plans)."""
        n = ctypes.c_int(0)
        _check(load().infer_hip_gemm_plan_timeline(self._handle, None, 0, ctypes.byref(n), None))
        return n.value

    TIMELINE_WORDS = 16

    def launch_timeline(self, stamps, stream=None) -> None:
        """One launch that also writes each workgroup's 16 timeline words
        (int64 device tensor of 16 * workgroups() entries, zeroed)."""
        n = ctypes.c_int(0)
        _check(load().infer_hip_gemm_plan_timeline(
            self._handle, _ptr(stamps), stamps.numel() // self.TIMELINE_WORDS, ctypes.byref(n),
            _stream(stream)))

    def close(self) -> None:
        if self._handle:
            _check(load().infer_hip_gemm_plan_destroy(self._handle))
            self._handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
