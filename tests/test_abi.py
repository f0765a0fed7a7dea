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


# ------------------------------------------------------ model runtime ABI --

def _declared_model_symbols():
    text = open(os.path.join(ROOT, "include", "infer_model.h")).read()
    return sorted(set(re.findall(r"\b(infer_hip_\w+)\s*\(", text)))


def test_library_exports_every_model_symbol(hip):
    import model_hip
    lib = model_hip.load()
    declared = _declared_model_symbols()
    assert declared
    for name in declared:
        assert hasattr(lib, name), name
    assert sorted(model_hip.EXPORTED_SYMBOLS) == declared


def test_library_exports_every_archive_symbol(hip):
    import archive_hip
    lib = archive_hip.load()
    text = open(os.path.join(ROOT, "include", "infer_archive.h")).read()
    declared = sorted(set(re.findall(r"\b(infer_hip_\w+)\s*\(", text)))
    assert declared
    for name in declared:
        assert hasattr(lib, name), name
    assert sorted(archive_hip.EXPORTED_SYMBOLS) == declared


def _create(cfg_fields, precision=2, max_seq=16, layers=None):
    import ctypes
    import model_hip
    lib = model_hip.load()
    cfg = model_hip._Config(*cfg_fields)
    lay = layers if layers is not None else (model_hip._Layer * max(1, cfg_fields[2]))()
    w = model_hip._Weights(None, None, None, lay)
    opts = model_hip._Options(precision, max_seq, 0)
    h = ctypes.c_void_p()
    return lib.infer_hip_model_create(ctypes.byref(cfg), ctypes.byref(w), ctypes.byref(opts),
                                      ctypes.byref(h)), h


@pytest.mark.parametrize("fields,why", [
    ((896, 4864, 0, 14, 2, 151936, -1, 1e-6, 1e6), "invalid model dimensions"),
    ((896, 4864, 24, 14, 3, 151936, -1, 1e-6, 1e6), "invalid GQA head counts"),
    ((900, 4864, 24, 14, 2, 151936, -1, 1e-6, 1e6), "invalid attention head dimension"),
    ((128, 256, 1, 4, 1, 64, -1, 1e-6, 1e6), "head_dim 32"),
    ((2560, 256, 1, 40, 8, 64, -1, 1e-6, 1e6), "40 attention heads"),
    ((896, 4864, 24, 14, 2, 151936, -1, 1e-6, 0.0), "rope_theta"),
])
def test_model_create_rejects_bad_config_on_host(hip, fields, why):
    # model_config.cpp:42-48 plus the shapes the HIP kernels support; all
    # rejected before any HIP call.
    rc, h = _create(fields)
    assert rc == hip.INVALID_ARGUMENT and not h.value
    assert why in hip.load().infer_hip_last_error().decode()


def test_model_create_rejects_precision_and_missing_weights(hip):
    fields = (128, 256, 1, 2, 1, 64, -1, 1e-6, 1e6)
    rc, _ = _create(fields, precision=0)
    assert rc == hip.INVALID_ARGUMENT
    assert "precision" in hip.load().infer_hip_last_error().decode()
    rc, _ = _create(fields, max_seq=0)
    assert rc == hip.INVALID_ARGUMENT
    rc, _ = _create(fields)
    assert rc == hip.INVALID_ARGUMENT
    assert "null embedding" in hip.load().infer_hip_last_error().decode()


def test_model_null_handles_are_rejected(hip):
    import ctypes
    import model_hip
    lib = model_hip.load()
    out = ctypes.c_int()
    assert lib.infer_hip_model_prefill(None, None, 0, ctypes.byref(out)) == hip.INVALID_ARGUMENT
    assert lib.infer_hip_model_decode_next(None, 0, ctypes.byref(out)) == hip.INVALID_ARGUMENT
    assert lib.infer_hip_model_decode_steps(None, 1, None) == hip.INVALID_ARGUMENT
    assert lib.infer_hip_model_rewind(None, 1, 1) == hip.INVALID_ARGUMENT
    assert lib.infer_hip_model_position(None) == -1
    assert lib.infer_hip_model_destroy(None) == hip.OK


def test_attention_prefill_rejects_bad_arguments_on_host(hip):
    import model_hip
    lib = model_hip.load()
    f = lib.infer_hip_attention_prefill_bf16
    assert f(None, 16, 16, 16, 4, 2, 1, 64, 8, None) == hip.INVALID_ARGUMENT
    assert f(16, 16, 16, 16, 4, 2, 1, 32, 8, None) == hip.INVALID_ARGUMENT
    assert "head_dim 32" in lib.infer_hip_last_error().decode()
    assert f(16, 16, 16, 16, 9, 2, 1, 64, 8, None) == hip.INVALID_ARGUMENT
    assert f(16, 16, 16, 16, 4, 3, 2, 64, 8, None) == hip.INVALID_ARGUMENT
    assert f(16, 16, 16, 16, 0, 2, 1, 64, 8, None) == hip.INVALID_ARGUMENT


def test_library_exports_every_decode_symbol(hip):
    import decode_hip
    lib = decode_hip.load()
    text = open(os.path.join(ROOT, "include", "infer_decode.h")).read()
    declared = sorted(set(re.findall(r"\b(infer_hip_\w+)\s*\(", text)))
    assert declared
    for name in declared:
        assert hasattr(lib, name), name
    assert sorted(decode_hip.EXPORTED_SYMBOLS) == declared


def test_decode_ops_reject_bad_arguments_on_host(hip):
    # Every check runs before any HIP call; fake 16-byte aligned addresses
    # are never dereferenced.
    import ctypes
    import decode_hip
    lib = decode_hip.load()
    bad = hip.INVALID_ARGUMENT
    err = lambda: lib.infer_hip_last_error().decode()  # noqa: E731
    g = (decode_hip.NormGemv * 1)(decode_hip.NormGemv(4096, 4096, None, 4096, 896))
    f = lib.infer_hip_rms_norm_gemv_w8a16
    assert f(None, 4096, 1e-6, 896, g, 1, None) == bad
    assert f(4104, 4096, 1e-6, 896, g, 1, None) == bad and "aligned" in err()
    assert f(4096, 4096, 1e-6, 900, g, 1, None) == bad and "multiple of 64" in err()
    assert f(4096, 4096, 1e-6, 8192, g, 1, None) == bad
    assert f(4096, 4096, 1e-6, 896, g, 0, None) == bad and "count" in err()
    assert f(4096, 4096, 1e-6, 896, g, 4, None) == bad
    g[0].weight = 4097
    assert f(4096, 4096, 1e-6, 896, g, 1, None) == bad and "weight" in err()
    g[0].weight, g[0].out_features = 4096, 0
    assert f(4096, 4096, 1e-6, 896, g, 1, None) == bad
    f = lib.infer_hip_rms_norm_gate_up_silu_w8a16
    assert f(4096, 4096, 1e-6, 896, 4096, None, 4096, 4096, 4096, 4864, None) == bad
    assert f(4096, 4096, 1e-6, 896, 4096, 4096, 4096, 4096, 4096, -1, None) == bad
    f = lib.infer_hip_gemv_w8a16_rows
    assert f(4096, 4096, None, 4096, 4096, 896, 8256, None) == bad and "8192" in err()
    assert f(4096, 4096, None, 4098, 4096, 896, 4864, None) == bad
    assert f(4096, 4096, None, None, 4096, 896, 4864, None) == bad
    f = lib.infer_hip_attention_merge_o_proj
    assert f(4096, 4096, 14, 64, 128, 8, 1024, 4096, 4096, 4096, 896, None) == bad
    assert "span" in err()
    assert f(4096, 4096, 14, 32, 128, 8, 1024, 4096, 4096, 4096, 896, None) == bad
    assert f(4096, 4096, 33, 64, 256, 8, 2048, 4096, 4096, 4096, 896, None) == bad
    assert f(4096, None, 14, 64, 256, 8, 2048, 4096, 4096, 4096, 896, None) == bad
    assert f(4096, 4096, 14, 64, 256, 8, 2048, 4104, 4096, 4096, 896, None) == bad
    f = lib.infer_hip_rms_norm_lm_head_argmax
    assert f(4096, 4096, 1e-6, 4096, 151936, 900, 4096, 4096, 4096, None) == bad
    assert f(4096, 4096, 1e-6, 4096, 0, 896, 4096, 4096, 4096, None) == bad
    assert f(4096, 4096, 1e-6, 4096, 151936, 896, 4096, 4100, 4096, None) == bad
    assert f(4096, 4096, 1e-6, 4096, 151936, 896, 4096, 4096, None, None) == bad
    assert lib.infer_hip_lm_head_decode_workspace_bytes(0) == 0
    assert lib.infer_hip_lm_head_decode_workspace_bytes(151936) >= 256 + 8


def test_attention_decode_span_closed_form(hip):
    # head_dim 64 with up to 1024 positions of capacity: one span of 1024
    # (the whole-context form); otherwise the smallest multiple of 128 that
    # covers max_seq in at most 8 splits.
    import decode_hip
    for max_seq in (1, 7, 128, 129, 1000, 1024):
        assert decode_hip.attention_decode_span(max_seq, 64) == 1024
        assert decode_hip.attention_decode_splits(max_seq, 64) == 1
    for max_seq, hd in [(m, 64) for m in (1025, 1500, 2048, 2049, 4096, 32768)] + \
                       [(m, 128) for m in (1, 7, 128, 129, 1000, 1024, 1025, 4096)]:
        span = decode_hip.attention_decode_span(max_seq, hd)
        splits = decode_hip.attention_decode_splits(max_seq, hd)
        assert span % 128 == 0 and 1 <= splits <= 8, (max_seq, span, splits)
        assert span * (splits - 1) < max_seq <= span * splits
        assert span == 128 or (span - 128) * 8 < max_seq  # the smallest that fits 8 splits
    assert decode_hip.attention_decode_span(2048, 64) == 256
    assert decode_hip.attention_decode_span(1024, 128) == 128
    assert decode_hip.attention_decode_span(0, 64) == 0
    assert decode_hip.attention_decode_span(1024, 32) == 0


@pytest.mark.parametrize("theta,head_dim", [(1e6, 64), (1e4, 128), (1e6, 2)])
def test_rope_row_equals_the_oracle_rotation(hip, orc, theta, head_dim):
    # Rotating the unit vector e_i (dims i and i + half = 1, 0) by the
    # oracle's rope (cpu_ops.cpp:33-56 restated) yields exactly (cos, sin)
    # of pair i: the library's row must equal it bit for bit.
    import numpy as np
    import decode_hip
    half = head_dim // 2
    for position in (0, 1, 7, 100, 1023, 32767):
        row = decode_hip.rope_row(theta, head_dim, position)
        q = np.zeros((half, head_dim), np.float32)
        q[np.arange(half), np.arange(half)] = 1.0
        rq, _ = orc.rope(q.reshape(-1), np.zeros(head_dim, np.float32), half, 1, head_dim,
                         position, theta)
        rq = rq.reshape(half, head_dim)
        np.testing.assert_array_equal(row[:, 0], rq[np.arange(half), np.arange(half)])
        np.testing.assert_array_equal(row[:, 1], rq[np.arange(half), np.arange(half) + half])
        if position == 0:
            assert np.all(row[:, 0] == 1.0) and np.all(row[:, 1] == 0.0)


def test_rope_row_and_new_decode_ops_reject_bad_arguments(hip):
    import ctypes
    import decode_hip
    lib = decode_hip.load()
    bad = hip.INVALID_ARGUMENT
    buf = (ctypes.c_float * 64)()
    assert lib.infer_hip_rope_row(1e6, 63, 0, buf) == bad
    assert lib.infer_hip_rope_row(1e6, 64, -1, buf) == bad
    assert lib.infer_hip_rope_row(1e6, 64, 0, None) == bad
    f = lib.infer_hip_attention_decode_bf16
    assert f(4096, 4096, 4096, 4096, 4096, 14, 2, 64, 2048, None) == bad  # split form only
    assert "1024" in lib.infer_hip_last_error().decode()
    assert f(4096, 4096, 4096, 4096, 4096, 14, 2, 128, 512, None) == bad
    assert f(4096, 4096, 4096, 4096, 4096, 14, 3, 64, 512, None) == bad
    assert f(4104, 4096, 4096, 4096, 4096, 14, 2, 64, 512, None) == bad
    assert f(4096, 4096, None, 4096, 4096, 14, 2, 64, 512, None) == bad
    w = decode_hip.W8A16Weight(4096, 4096, None)
    g = lib.infer_hip_rms_norm_qkv_rope_w8a16
    args = [4096, 4096, 1e-6, 896, ctypes.byref(w), ctypes.byref(w), ctypes.byref(w), 4096, 4096,
            4096, 4096, 4096, 14, 2, 64, 1024, None]
    for i, v in ((3, 900), (12, 0), (13, 3), (14, 63), (15, 0), (11, None), (4, None)):
        a = list(args)
        a[i] = v
        assert g(*a) == bad, (i, v)


def test_halves_attention_ops_reject_bad_arguments(hip):
    import decode_hip
    lib = decode_hip.load()
    bad = hip.INVALID_ARGUMENT
    f = lib.infer_hip_attention_decode_halves_bf16
    assert f(4096, 4096, 4096, 4096, 4096, 14, 2, 64, 2048, None) == bad  # at most 1024
    assert f(4096, 4096, 4096, 4096, 4096, 14, 2, 128, 512, None) == bad  # head_dim 64
    assert f(4096, 4096, 4096, 4096, 4096, 14, 3, 64, 512, None) == bad  # GQA
    assert f(4096, 4096, 4096, 4096, 4100, 14, 2, 64, 512, None) == bad  # records aligned
    assert f(4096, 4096, 4096, None, 4096, 14, 2, 64, 512, None) == bad
    g = lib.infer_hip_attention_halves_o_proj_w8a16
    assert g(4096, 4096, 65, 1024, 4096, 4096, 4096, 896, None) == bad   # 65 x 64 > 4096
    assert g(4096, 4096, 14, 1025, 4096, 4096, 4096, 896, None) == bad   # max_seq
    assert g(4096, 4096, 14, 1024, 4096, 4096, 4096, 0, None) == bad     # no outputs
    assert g(4100, 4096, 14, 1024, 4096, 4096, 4096, 896, None) == bad   # records aligned
    assert g(4096, 4096, 14, 1024, 4104, 4096, 4096, 896, None) == bad   # weight aligned
    assert g(4096, None, 14, 1024, 4096, 4096, 4096, 896, None) == bad


def test_parts_attention_ops_reject_bad_arguments(hip):
    """The parts forms: num_parts 2 or 4 only, then the halves' checks."""
    import decode_hip
    lib = decode_hip.load()
    bad = hip.INVALID_ARGUMENT
    err = lambda: lib.infer_hip_last_error().decode()  # noqa: E731
    f = lib.infer_hip_attention_decode_parts_bf16
    for parts in (0, 1, 3, 8):
        assert f(4096, 4096, 4096, 4096, 4096, 14, 2, 64, 1024, parts, None) == bad
        assert "num_parts" in err()
    assert f(4096, 4096, 4096, 4096, 4096, 14, 2, 64, 2048, 4, None) == bad  # at most 1024
    assert f(4096, 4096, 4096, 4096, 4096, 14, 3, 64, 512, 4, None) == bad   # GQA
    assert f(4096, 4096, 4096, 4096, 4100, 14, 2, 64, 512, 4, None) == bad   # records aligned
    g = lib.infer_hip_attention_parts_o_proj_w8a16
    for parts in (1, 3):
        assert g(4096, 4096, 14, 1024, parts, 4096, 4096, 4096, 896, None) == bad
        assert "num_parts" in err()
    assert g(4096, 4096, 65, 1024, 4, 4096, 4096, 4096, 896, None) == bad   # 65 x 64 > 4096
    assert g(4096, 4096, 14, 1025, 4, 4096, 4096, 4096, 896, None) == bad   # max_seq
    assert g(4096, 4096, 14, 1024, 4, 4096, None, 4096, 896, None) == bad   # scales
    o = lib.infer_hip_attention_parts_o_proj_bf16
    assert o(4096, 4096, 14, 1024, 3, 4096, 4096, 896, None) == bad
    assert o(4096, 4096, 33, 1024, 4, 4096, 4096, 896, None) == bad         # 33 x 64 > 2048
    assert o(4096, 4096, 14, 1024, 4, 4104, 4096, 896, None) == bad         # weight aligned


def test_attention_spans_rejects_bad_arguments(hip):
    """infer_hip_attention_decode_spans_bf16: shapes, nulls and alignment are
    checked on the host; nothing is launched."""
    import decode_hip
    lib = decode_hip.load()
    bad = hip.INVALID_ARGUMENT
    f = lib.infer_hip_attention_decode_spans_bf16
    assert f(4096, 4096, 4096, 4096, 4096, 14, 2, 96, 2048, None) == bad   # head_dim
    assert f(4096, 4096, 4096, 4096, 4096, 14, 3, 64, 2048, None) == bad   # GQA
    assert f(4096, 4096, 4096, 4096, 4096, 14, 2, 64, 0, None) == bad      # capacity
    assert f(4096, 4100, 4096, 4096, 4096, 14, 2, 64, 2048, None) == bad   # cache aligned
    assert f(4096, 4096, 4096, None, 4096, 14, 2, 64, 2048, None) == bad
    assert f(4096, 4096, 4096, 4096, None, 14, 2, 64, 2048, None) == bad


def test_bf16_decode_ops_reject_bad_arguments(hip):
    """The BF16 siblings of the fused decode operators: K limits half the
    W8A16 ones (8 BF16 weights per 16-byte chunk), no scales needed; checked
    on the host, nothing launched."""
    import ctypes
    import decode_hip
    lib = decode_hip.load()
    bad = hip.INVALID_ARGUMENT
    err = lambda: lib.infer_hip_last_error().decode()  # noqa: E731
    g = (decode_hip.NormGemvBf16 * 1)(decode_hip.NormGemvBf16(4096, None, 4096, 896))
    f = lib.infer_hip_rms_norm_gemv_bf16
    assert f(4096, 4096, 1e-6, 2112, g, 1, None) == bad and "2048" in err()
    assert f(4096, 4096, 1e-6, 900, g, 1, None) == bad and "multiple of 64" in err()
    assert f(4096, 4096, 1e-6, 896, None, 1, None) == bad
    assert f(4096, 4096, 1e-6, 896, g, 0, None) == bad and "count" in err()
    g[0].weight = 4104
    assert f(4096, 4096, 1e-6, 896, g, 1, None) == bad and "aligned" in err()
    f = lib.infer_hip_rms_norm_gate_up_silu_bf16
    assert f(4096, 4096, 1e-6, 2112, 4096, 4096, 4096, 4864, None) == bad
    assert f(4096, 4096, 1e-6, 896, 4096, None, 4096, 4864, None) == bad
    assert f(4096, 4096, 1e-6, 896, 4096, 4096, 4096, 0, None) == bad
    w = decode_hip.Bf16Weight(4096, None)
    q = lib.infer_hip_rms_norm_qkv_rope_bf16
    args = [4096, 4096, 1e-6, 896, ctypes.byref(w), ctypes.byref(w), ctypes.byref(w), 4096, 4096,
            4096, 4096, 4096, 14, 2, 64, 1024, None]
    for i, v in ((3, 2112), (3, 900), (12, 0), (13, 3), (14, 63), (11, None), (4, None)):
        a = list(args)
        a[i] = v
        assert q(*a) == bad, (i, v)
    o = lib.infer_hip_attention_halves_o_proj_bf16
    assert o(4096, 4096, 33, 1024, 4096, 4096, 896, None) == bad   # 33 x 64 > 2048
    assert o(4096, 4096, 14, 1025, 4096, 4096, 896, None) == bad   # max_seq
    assert o(4096, 4096, 14, 1024, 4104, 4096, 896, None) == bad   # weight aligned
    assert o(4096, 4096, 14, 1024, None, 4096, 896, None) == bad
    r = lib.infer_hip_gemv_bf16_rows
    assert r(4096, None, 4096, 4096, 896, 5184, None) == bad and "5120" in err()
    assert r(4096, None, 4098, 4096, 896, 4864, None) == bad
    assert r(4096, None, 4096, 4096, 0, 4864, None) == bad


def test_gate_up_silu_rejects_bad_arguments(hip):
    """infer_hip_gemm_gate_up_silu_*: the group size, shapes, null pointers,
    K % 64 and alignment are checked on the host; nothing is launched."""
    import model_hip
    a = 256  # a 16-byte aligned stand-in address (never dereferenced)

    def w8(**kw):
        args = dict(gate_w=a, gate_s=a, gate_b=None, up_w=a, up_s=a, up_b=None, group_size=64,
                    x=a, y=a, tokens=4, intermediate=128, hidden=128)
        args.update(kw)
        model_hip.gemm_gate_up_silu_w8a16(**args, stream=0)

    def bf16(**kw):
        args = dict(gate_w=a, gate_b=None, up_w=a, up_b=None, x=a, y=a, tokens=4,
                    intermediate=128, hidden=128)
        args.update(kw)
        model_hip.gemm_gate_up_silu_bf16(**args, stream=0)

    cases = [(w8, dict(group_size=32), "group size must be 64"),
             (w8, dict(tokens=0), "bad shape"), (w8, dict(intermediate=-1), "bad shape"),
             (w8, dict(hidden=0), "bad shape"), (w8, dict(gate_s=None), "null"),
             (w8, dict(up_w=None), "null"), (w8, dict(y=None), "null"),
             (w8, dict(hidden=96), "hidden % 64"), (w8, dict(up_w=a + 8), "aligned"),
             (w8, dict(x=a + 2), "aligned"),
             (w8, dict(tokens=1 << 21, hidden=1024), "2 GiB"),
             (bf16, dict(tokens=-3), "bad shape"), (bf16, dict(gate_w=None), "null"),
             (bf16, dict(hidden=100), "hidden % 64"), (bf16, dict(gate_w=a + 4), "aligned")]
    for fn, kw, text in cases:
        with pytest.raises(hip.InferError) as err:
            fn(**kw)
        assert err.value.status == hip.INVALID_ARGUMENT, kw
        assert text in str(err.value), (kw, str(err.value))


def test_calibration_library_exports_its_symbols():
    """libinfer_calib.so, bench.py's measurement aids (a streaming read, an
    empty kernel and the compute-unit probes): built by build() and
    exporting every entry point, whose argument checks run on the host
    before any launch."""
    import ctypes
    import calibration_hip as cal
    lib = cal.load()
    for name in cal.EXPORTED_SYMBOLS:
        assert hasattr(lib, name), name
    # rejected before launching: null, misaligned or ragged reads, bad grids
    assert lib.infer_calib_stream_read(None, 16, ctypes.c_void_p(16), 1, None) == 1
    assert lib.infer_calib_stream_read(ctypes.c_void_p(32), 16, None, 1, None) == 1
    assert lib.infer_calib_stream_read(ctypes.c_void_p(36), 16, ctypes.c_void_p(16), 1, None) == 1
    assert lib.infer_calib_stream_read(ctypes.c_void_p(32), 24, ctypes.c_void_p(16), 1, None) == 1
    assert lib.infer_calib_stream_read(ctypes.c_void_p(32), 16, ctypes.c_void_p(16), 0, None) == 1
    assert lib.infer_calib_empty(0, None) == 1
    assert lib.infer_calib_empty(65537, None) == 1
    # compute-unit probes: unknown kind, thread counts off the wave grid, no
    # cycle buffer, a fill probe without (or with a misaligned) source
    buf = ctypes.c_void_p(256)
    assert lib.infer_calib_cu_probe(-1, 1, 256, 1, None, buf, buf, None) == 1
    assert lib.infer_calib_cu_probe(len(cal.CU_PROBES), 1, 256, 1, None, buf, buf, None) == 1
    assert lib.infer_calib_cu_probe(0, 1, 96, 1, None, buf, buf, None) == 1
    assert lib.infer_calib_cu_probe(0, 1, 2048, 1, None, buf, buf, None) == 1
    assert lib.infer_calib_cu_probe(0, 1, 256, 0, None, buf, buf, None) == 1
    assert lib.infer_calib_cu_probe(0, 1, 256, 1, None, None, buf, None) == 1
    assert lib.infer_calib_cu_probe(7, 1, 256, 1, None, buf, buf, None) == 1
    assert lib.infer_calib_cu_probe(7, 1, 256, 1, ctypes.c_void_p(264), buf, buf, None) == 1

