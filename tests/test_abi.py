"""The C ABI without a GPU: the library loads, exports exactly what
include/infer_linear.h declares, and rejects bad arguments on the host before
any HIP call (the reference throws infer::Error for these,
tests/test_cuda.cpp:887-890)."""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_symbols():
    text = open(os.path.join(ROOT, "include", "infer_linear.h")).read()
    return sorted(set(re.findall(r"\b(infer_hip_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol(hip):
    lib = hip.load()
    declared = _declared_symbols()
    assert declared, "no declarations found"
    for name in declared:
        assert hasattr(lib, name), name
    assert sorted(hip.EXPORTED_SYMBOLS) == declared


def test_abi_version(hip):
    assert hip.load().infer_hip_abi_version() == 1


def test_group_size_other_than_64_is_rejected(hip):
    # test_cuda.cpp:887-890: gemv_w8a16 with group 32 throws.
    with pytest.raises(hip.InferError) as err:
        hip.gemv_w8a16(None, None, 32, None, None, None, 1, 1, stream=0)
    assert err.value.status == hip.INVALID_ARGUMENT
    assert "group size must be 64" in str(err.value)
    with pytest.raises(hip.InferError):
        hip.gemm_w8a16(None, None, 128, None, None, None, 2, 1, 1, stream=0)


@pytest.mark.parametrize("n,k", [(0, 64), (-1, 64), (8, -1)])
def test_bad_shapes_are_rejected(hip, n, k):
    with pytest.raises(hip.InferError) as err:
        hip.gemv_bf16(16, None, 16, 16, n, k, stream=0)
    assert err.value.status == hip.INVALID_ARGUMENT
    with pytest.raises(hip.InferError):
        hip.gemv_w8a16(16, 16, 64, None, 16, 16, n, k, stream=0)
    with pytest.raises(hip.InferError):
        hip.lm_head_bf16(16, None, 16, 16, 16, 16, 16, n, k, stream=0)


def test_zero_tokens_rejected(hip):
    with pytest.raises(hip.InferError):
        hip.gemm_bf16(16, None, 16, 16, 0, 8, 8, stream=0)
    with pytest.raises(hip.InferError):
        hip.gemm_w8a16(16, 16, 64, None, 16, 16, 0, 8, 64, stream=0)


def test_null_required_pointers_rejected(hip):
    with pytest.raises(hip.InferError):
        hip.gemv_bf16(None, None, 16, 16, 8, 8, stream=0)
    with pytest.raises(hip.InferError):
        hip.gemv_w8a16(16, None, 64, None, 16, 16, 8, 64, stream=0)
    with pytest.raises(hip.InferError):
        hip.lm_head_bf16(16, None, 16, 16, None, 16, 16, 8, 8, stream=0)
    with pytest.raises(hip.InferError):
        hip.gemm_w8a16(16, 16, 64, None, None, 16, 2, 8, 64, stream=0)


def test_last_error_is_per_call(hip):
    with pytest.raises(hip.InferError):
        hip.gemv_bf16(None, None, None, None, 8, 8, stream=0)
    assert hip.load().infer_hip_last_error()


@pytest.mark.parametrize("vocab,k", [(151936, 896), (512, 64), (1002, 64), (200, 10),
                                     (8, 4), (64, 896), (1, 1), (7, 8), (100000, 4096)])
def test_lm_head_workspace_never_exceeds_reference_sizing(hip, vocab, k):
    # src/qwen2.cpp:193-198 allocates ceil(V / 8) entries.
    entries = hip.lm_head_workspace_entries(vocab, k)
    assert 1 <= entries <= (vocab + 7) // 8


def test_lm_head_workspace_invalid_shape(hip):
    assert hip.lm_head_workspace_entries(0, 896) == 0
