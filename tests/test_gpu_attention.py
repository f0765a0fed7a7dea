"""The prefill attention kernel on its own (infer_hip_attention_prefill_bf16,
the reference's attention_prefill_bf16, include/infer/cuda_ops.hpp:92-97)
against the CPU FP32 oracle's attention, as the reference's
CudaBFloat16.RopeKvAndAttentionMatchFp32 test checks its kernel against a
causal FP32 reference (tests/test_cuda.cpp:249-296, 385-393).

The expected row of token t is the oracle's decode attention over positions
0 .. t (cpu_ops.cpp:58-91), the same definition the reference test uses.
Bar: the output within BF16 rounding of the FP32 result plus a few FP32
ulps of the value scale, |a - e| <= 2^-8 |e| + 2^-16 max|v| (the
probabilities enter the MFMA product as BF16 hi + lo parts, about 16 bits;
BF16 probabilities alone miss this bound by an order of magnitude), and on
the reference test's own input pattern (magnitudes below 0.5) its absolute
tolerance 0.004 too.  The random cases draw q, k and v from N(0, 1)."""
import numpy as np
import pytest

import model_hip
import refcases as R

pytestmark = pytest.mark.gpu


def _case(t, heads, kv_heads, hd, max_seq, seed, pattern=False):
    rng = np.random.default_rng(seed)
    if pattern:
        # tests/test_cuda.cpp:318-326: q = (i % 11 - 5) 0.08, k = (i % 7 - 3)
        # 0.07, v = (i % 9 - 4) 0.06 over the flat index
        q = ((np.arange(t * heads * hd) % 11) - 5).astype(np.float32) * np.float32(0.08)
        kv = np.arange(max_seq * kv_heads * hd)
        k = ((kv % 7) - 3).astype(np.float32) * np.float32(0.07)
        v = ((kv % 9) - 4).astype(np.float32) * np.float32(0.06)
    else:
        q = rng.standard_normal(t * heads * hd).astype(np.float32)
        k = rng.standard_normal(max_seq * kv_heads * hd).astype(np.float32)
        v = rng.standard_normal(max_seq * kv_heads * hd).astype(np.float32)
    qw = R.bf16_words(q).reshape(t, heads, hd)
    kw = R.bf16_words(k).reshape(kv_heads, max_seq, hd)
    vw = R.bf16_words(v).reshape(kv_heads, max_seq, hd)
    # positions past the prompt hold NaN: the kernel must neither read them
    # into a result (masked keys, zeroed values) nor fault on them
    kw[:, t:, :] = 0x7FC0
    vw[:, t:, :] = 0x7FC0
    return qw, kw, vw


def _expected(orc, qw, kw, vw, heads, kv_heads, hd, max_seq):
    t = qw.shape[0]
    qf, kf, vf = R.bf16_values(qw), R.bf16_values(kw), R.bf16_values(vw)
    out = np.empty((t, heads * hd), np.float32)
    for tok in range(t):
        out[tok] = orc.attention_decode(qf[tok].reshape(-1), kf, vf, heads, kv_heads, hd,
                                        tok + 1, max_seq)
    return out


def _run(dev, qw, kw, vw, heads, kv_heads, hd, max_seq, offset=0):
    import torch
    t = qw.shape[0]

    def put(a):
        flat = torch.from_numpy(a.reshape(-1).view(np.int16).copy())
        buf = torch.zeros(flat.numel() + offset, dtype=torch.int16, device=dev)
        buf[offset:] = flat.to(dev)
        return buf, buf[offset:]

    qb, q = put(qw)
    kb, k = put(kw)
    vb, v = put(vw)
    ob = torch.zeros(t * heads * hd + offset, dtype=torch.int16, device=dev)
    o = ob[offset:]
    model_hip.attention_prefill_bf16(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), t,
                                     heads, kv_heads, hd, max_seq, stream=0)
    torch.cuda.synchronize()
    return R.bf16_values(o.cpu().numpy().view(np.uint16)).reshape(t, heads * hd)


def _check(got, exp, vw, what, absolute=None):
    assert np.all(np.isfinite(got)), what
    err = np.abs(got - exp)
    if absolute is not None:
        assert err.max() <= absolute, f"{what}: max abs error {err.max():.3g}"
    vals = R.bf16_values(vw)
    vmax = float(np.abs(vals[np.isfinite(vals)]).max())
    bound = 2.0 ** -8 * np.abs(exp) + 2.0 ** -16 * vmax
    worst = np.argmax(err - bound)
    assert np.all(err <= bound), (f"{what}: {got.flat[worst]} vs {exp.flat[worst]} "
                                  f"(error {err.flat[worst]:.3g})")


CASES = [
    # (tokens, heads, kv_heads, head_dim, max_seq)
    (3, 4, 2, 64, 5),          # the reference test's counts at head_dim 64
    (1, 14, 2, 64, 1024),
    (31, 14, 2, 64, 64),
    (33, 14, 2, 64, 64),
    (250, 14, 2, 64, 256),
    (512, 14, 2, 64, 1024),    # config 4's prompt
    (100, 8, 1, 128, 128),
    (70, 32, 4, 128, 97),      # max_seq not a multiple of 32
    (1024, 14, 2, 64, 1024),
]


@pytest.mark.parametrize("t,heads,kv_heads,hd,max_seq", CASES)
def test_prefill_attention_matches_oracle(orc, dev, t, heads, kv_heads, hd, max_seq):
    print(f"attention prefill t={t} heads={heads}/{kv_heads} hd={hd} max_seq={max_seq}",
          flush=True)
    qw, kw, vw = _case(t, heads, kv_heads, hd, max_seq, seed=t + hd)
    exp = _expected(orc, qw, kw, vw, heads, kv_heads, hd, max_seq)
    got = _run(dev, qw, kw, vw, heads, kv_heads, hd, max_seq)
    _check(got, exp, vw, f"t={t}")


@pytest.mark.parametrize("slope", [0.0375, 0.005])
def test_prefill_attention_rising_scores(orc, dev, slope):
    """Scores that rise along the keys (key p scores about 8 slope p nats
    above key 0 at head_dim 64) keep moving each query's softmax maximum:
    by about 14 base-2 units per 32-key block at slope 0.0375, past the
    kernel's rescale slack (8) every block, and by about 1.8 at 0.005, where
    the probabilities grow up to 2^8 between rescales."""
    t, heads, kv_heads, hd, max_seq = 300, 4, 2, 64, 320
    print(f"attention prefill rising scores slope={slope}", flush=True)
    rng = np.random.default_rng(11)
    q = (1.0 + 0.1 * rng.standard_normal(t * heads * hd)).astype(np.float32)
    ramp = slope * np.arange(max_seq, dtype=np.float32)[None, :, None]
    k = (ramp + 0.1 * rng.standard_normal((kv_heads, max_seq, hd))).astype(np.float32)
    v = rng.standard_normal((kv_heads, max_seq, hd)).astype(np.float32)
    qw = R.bf16_words(q).reshape(t, heads, hd)
    kw = R.bf16_words(k.reshape(-1)).reshape(kv_heads, max_seq, hd)
    vw = R.bf16_words(v.reshape(-1)).reshape(kv_heads, max_seq, hd)
    kw[:, t:, :] = 0x7FC0
    vw[:, t:, :] = 0x7FC0
    exp = _expected(orc, qw, kw, vw, heads, kv_heads, hd, max_seq)
    _check(_run(dev, qw, kw, vw, heads, kv_heads, hd, max_seq), exp, vw, f"slope={slope}")


def test_prefill_attention_reference_pattern(orc, dev):
    qw, kw, vw = _case(40, 4, 2, 64, 48, seed=0, pattern=True)
    exp = _expected(orc, qw, kw, vw, 4, 2, 64, 48)
    _check(_run(dev, qw, kw, vw, 4, 2, 64, 48), exp, vw, "pattern", absolute=0.004)


@pytest.mark.parametrize("hd", [64, 128])
def test_unaligned_operands_take_the_exact_path(orc, dev, hd):
    # 2-byte offsets: the MFMA kernel needs 16-byte alignment; the scalar
    # kernel takes over with the same results
    qw, kw, vw = _case(45, 4, 1, hd, 64, seed=7)
    exp = _expected(orc, qw, kw, vw, 4, 1, hd, 64)
    _check(_run(dev, qw, kw, vw, 4, 1, hd, 64, offset=1), exp, vw, "unaligned")


def test_prefill_attention_is_deterministic(dev):
    qw, kw, vw = _case(300, 14, 2, 64, 512, seed=3)
    a = _run(dev, qw, kw, vw, 14, 2, 64, 512)
    b = _run(dev, qw, kw, vw, 14, 2, 64, 512)
    assert np.array_equal(a, b)
