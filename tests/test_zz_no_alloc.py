"""infer_hip_lm_head_bf16_noalloc (static device scratch) against
infer_hip_lm_head_bf16 (caller workspace): identical logits and argmax, on
two calls in a row, the second smaller, both through the C ABI."""
import numpy as np
import pytest

import refcases as rc
from helpers import bf16_out, to_dev, words

pytestmark = pytest.mark.gpu


def _with_workspace(hip, dev, e, h, vocab, k):
    import torch
    n = hip.lm_head_workspace_entries(vocab, k)
    bv = torch.empty(n, dtype=torch.float32, device=dev)
    bi = torch.empty(n, dtype=torch.int32, device=dev)
    logits = bf16_out((vocab,), dev)
    am = torch.full((1,), -7, dtype=torch.int32, device=dev)
    hip.lm_head_bf16(e, None, h, logits, bv, bi, am, vocab, k)
    return words(logits), int(am.cpu().item())


def _no_alloc(hip, dev, e, h, vocab, k):
    import torch
    logits = bf16_out((vocab,), dev)
    am = torch.full((1,), -7, dtype=torch.int32, device=dev)
    hip.lm_head_bf16_noalloc(e, None, h, logits, am, vocab, k)
    return words(logits), int(am.cpu().item())


def test_no_alloc_lm_head_matches_workspace_entry_point(hip, orc, dev):
    # Call 1: config 2's full vocabulary; call 2: smaller (fewer first-stage
    # blocks, so the second call reads only what it wrote); call 3: the
    # reference's tie case on the unaligned generic kernel.
    rng = rc.philox(2)
    cases = [(rc.VOCAB, rc.HIDDEN, 0.02), (5000, 896, 0.05)]
    for vocab, k, std in cases:
        e = rc.bf16_normal(rng, (vocab, k), std)
        h = rc.bf16_normal(rng, (k,))
        de, dh = to_dev(e, dev), to_dev(h, dev)
        lw, aw = _with_workspace(hip, dev, de, dh, vocab, k)
        ln, an = _no_alloc(hip, dev, de, dh, vocab, k)
        np.testing.assert_array_equal(ln, lw)
        assert an == aw
        _, _, idx = orc.lm_head(e, h)
        assert an == idx, (vocab, an, idx)
    vocab, k, ta, tb = 1002, 64, 7, 71
    e, h = rc.lm_head_fused_case(vocab, k, ta, tb)
    import torch
    raw = torch.empty(vocab * k * 2 + 2, dtype=torch.uint8, device=dev)
    de = raw[2:].view(torch.bfloat16)          # 2-byte offset: the generic kernel
    de.copy_(to_dev(e, dev).view(-1))
    dh = to_dev(h, dev)
    ln, an = _no_alloc(hip, dev, de, dh, vocab, k)
    lw, aw = _with_workspace(hip, dev, de, dh, vocab, k)
    np.testing.assert_array_equal(ln, lw)
    assert an == aw == ta


def test_no_alloc_lm_head_rejects_vocab_beyond_its_scratch(hip, dev):
    import torch
    vocab, k = 1_100_000, 8   # 68750 first-stage blocks > 65536
    assert hip.lm_head_workspace_entries(vocab, k) > 65536
    e = torch.zeros((vocab, k), dtype=torch.bfloat16, device=dev)
    h = torch.zeros((k,), dtype=torch.bfloat16, device=dev)
    logits = bf16_out((vocab,), dev)
    am = torch.zeros((1,), dtype=torch.int32, device=dev)
    with pytest.raises(hip.InferError, match="scratch"):
        hip.lm_head_bf16_noalloc(e, None, h, logits, am, vocab, k)
