"""infer_hip_gemm_gate_up_silu_{w8a16,bf16}: gate_proj and up_proj of one
input plus SiLU-mul in one launch of gate|up pair tiles (the model's prefill
runs it for prompts over 256 tokens), or for at most 32 tokens of the skinny
kernel's pair form (each workgroup streams 32 gate rows and 32 up rows).

The reference computes the same thing as two GEMM calls and silu_mul_bf16
(src/qwen2.cpp:560-568).  So does this test, on the device: both GEMMs
through infer_hip_gemm_* (the 64 x 64 tiles, whose per-element arithmetic
is the pair tile's: the same per-group MFMA partials folded in group order),
then bf16(g / (1 + exp(-g)) * u) on their BF16 outputs.  The GEMM parts must
agree exactly; the SiLU is torch's exp and division here and the kernel's
hardware 2^x and reciprocal there (a few FP32 ulps apart), so an output may
differ by one BF16 unit in the last place, on at most 0.5 % of the outputs.  The GEMMs themselves are checked against the FP32 oracle
elsewhere (tests/test_gpu_gemm.py); the pair tile's layout (rows of gate in
columns 0-63, up in 64-127, 64-column steps, tails) is what this file pins.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _case(torch, dev, tokens, inter, hidden, w8, bias, seed):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    x = torch.randn((tokens, hidden), device=dev, generator=g).to(torch.bfloat16)
    mats = []
    for _ in range(2):
        if w8:
            q = torch.randint(-127, 128, (inter, hidden), dtype=torch.int8, device=dev,
                              generator=g)
            s = ((torch.randn((inter, hidden // 64), device=dev, generator=g) * 0.02).abs_()
                 / 127.0 + 1e-4).to(torch.bfloat16)
        else:
            q = (torch.randn((inter, hidden), device=dev, generator=g) * 0.05).to(torch.bfloat16)
            s = None
        b = ((torch.randn((inter,), device=dev, generator=g) * 0.5).to(torch.bfloat16)
             if bias else None)
        mats.append((q, s, b))
    return x, mats


@pytest.mark.parametrize("w8", [True, False], ids=["w8a16", "bf16"])
@pytest.mark.parametrize("tokens, inter, hidden, bias", [
    (512, 4864, 896, False),   # the Qwen2.5-0.5B prefill at 512 tokens
    (300, 4864, 896, False),   # a partly filled second row of tiles
    (257, 200, 128, True),     # a 64-column tail (200 = 3 x 64 + 8) and biases
    (64, 64, 64, True),        # one tile, mostly empty rows
    (2, 136, 192, False),      # two tokens; K of 3 groups (the skinny pair, up to 32)
    (32, 4864, 896, False),    # config 0's 32-token prompt: skinny pair, 4 waves
    (17, 200, 128, True),      # skinny pair: ragged rows, biases
])
def test_gate_up_silu_matches_separate_ops(hip, dev, w8, tokens, inter, hidden, bias):
    import model_hip
    import torch
    linear_hip = hip
    print(f"gate|up silu w8={w8} tokens={tokens} inter={inter} hidden={hidden} bias={bias}",
          flush=True)
    x, ((gw, gs, gb), (uw, us, ub)) = _case(torch, dev, tokens, inter, hidden, w8, bias,
                                           seed=tokens + inter + hidden)
    gate = torch.empty((tokens, inter), dtype=torch.bfloat16, device=dev)
    up = torch.empty_like(gate)
    fused = torch.full((tokens, inter), float("nan"), dtype=torch.bfloat16, device=dev)
    if w8:
        for (w, s, b), y in (((gw, gs, gb), gate), ((uw, us, ub), up)):
            linear_hip.gemm_w8a16(w, s, 64, b, x, y, tokens, inter, hidden)
        model_hip.gemm_gate_up_silu_w8a16(gw, gs, gb, uw, us, ub, 64, x, fused, tokens, inter,
                                          hidden)
    else:
        for (w, _, b), y in (((gw, gs, gb), gate), ((uw, us, ub), up)):
            linear_hip.gemm_bf16(w, b, x, y, tokens, inter, hidden)
        model_hip.gemm_gate_up_silu_bf16(gw, gb, uw, ub, x, fused, tokens, inter, hidden)
    torch.cuda.synchronize()
    gf, uf = gate.float(), up.float()
    ref = (gf / (1.0 + torch.exp(-gf)) * uf).to(torch.bfloat16)
    got_w = fused.view(torch.int16).cpu().numpy().astype(np.int32)
    ref_w = ref.view(torch.int16).cpu().numpy().astype(np.int32)
    assert np.all(np.isfinite(fused.float().cpu().numpy())), "unwritten or non-finite outputs"
    ulps = np.abs(got_w - ref_w)
    worst = np.unravel_index(np.argmax(ulps), ulps.shape)
    assert ulps.max() <= 1, (f"{ulps.max()} BF16 ulps at {worst}: fused "
                             f"{fused[worst].item()} vs {ref[worst].item()}")
    assert np.mean(ulps != 0) <= 5e-3, f"{np.mean(ulps != 0):.4%} outputs differ"
