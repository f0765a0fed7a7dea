"""The CPU model oracle (oracle/model_oracle.c) pinned against closed forms,
float64 brute force and an independent float64 model on tiny shapes.

These run without a GPU.  The reference's own op tests restated here:
test_ops.cpp:5-12 (RMSNorm closed form) and 47-55 (RoPE at position 0 is
the identity); its qwen2 tests check a prefill against step-by-step decode
(test_qwen2.cpp:450-488), as test_prefill_equals_decode_steps does.
"""
import numpy as np
import pytest

import oracle
import refcases as rc


def test_rms_norm_closed_form():
    # test_ops.cpp:5-12.
    out = oracle.rms_norm(np.array([1, 2, 3, 4], np.float32), np.ones(4, np.float32), 0.0)
    np.testing.assert_allclose(out, np.array([1, 2, 3, 4]) / np.sqrt(7.5), atol=1e-6)


def test_rms_norm_float64_brute_force():
    rng = rc.philox(5)
    x = rng.normal(0, 3, 896).astype(np.float32)
    w = rng.normal(1, 0.1, 896).astype(np.float32)
    out = oracle.rms_norm(x, w, 1e-6)
    x64 = x.astype(np.float64)
    exp = x64 / np.sqrt(np.mean(x64 * x64) + 1e-6) * w
    np.testing.assert_allclose(out, exp, rtol=2e-6, atol=1e-7)


def test_rope_position_zero_is_identity():
    # test_ops.cpp:47-55.
    q, k = oracle.rope([1, 2, 3, 4], [5, 6, 7, 8], 1, 1, 4, 0, 10000.0)
    np.testing.assert_array_equal(q, [1, 2, 3, 4])
    np.testing.assert_array_equal(k, [5, 6, 7, 8])


@pytest.mark.parametrize("position", [1, 7, 511, 1023])
def test_rope_rotate_half_float64(position):
    rng = rc.philox(6 + position)
    heads, kv_heads, hd, theta = 14, 2, 64, 1e6
    q = rng.normal(0, 1, heads * hd).astype(np.float32)
    k = rng.normal(0, 1, kv_heads * hd).astype(np.float32)
    qo, ko = oracle.rope(q, k, heads, kv_heads, hd, position, theta)

    def ref(x, n):
        x = x.astype(np.float64).reshape(n, hd)
        i = np.arange(hd // 2)
        ang = position * theta ** (-2.0 * i / hd)
        a, b = x[:, :hd // 2], x[:, hd // 2:]
        return np.concatenate([a * np.cos(ang) - b * np.sin(ang),
                               b * np.cos(ang) + a * np.sin(ang)], 1).ravel()
    # float32 angles of large positions carry ~1e-4 relative phase error.
    np.testing.assert_allclose(qo, ref(q, heads), atol=2e-3 * (1 + position / 512))
    np.testing.assert_allclose(ko, ref(k, kv_heads), atol=2e-3 * (1 + position / 512))
    # each rotated pair keeps its length
    pq = qo.reshape(heads, 2, hd // 2)
    p0 = q.reshape(heads, 2, hd // 2)
    np.testing.assert_allclose((pq ** 2).sum(1), (p0 ** 2).sum(1), rtol=1e-5)


def _attention64(q, kc, vc, heads, kv_heads, hd, seq):
    out = np.zeros((heads, hd))
    for h in range(heads):
        g = h // (heads // kv_heads)
        s = kc[g, :seq].astype(np.float64) @ q[h * hd:(h + 1) * hd] / np.sqrt(hd)
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ vc[g, :seq]
    return out.ravel()


def test_attention_single_position_returns_value_row():
    heads, kv_heads, hd, max_seq = 4, 2, 8, 5
    rng = rc.philox(7)
    kc = rng.normal(0, 1, (kv_heads, max_seq, hd)).astype(np.float32)
    vc = rng.normal(0, 1, (kv_heads, max_seq, hd)).astype(np.float32)
    q = rng.normal(0, 1, heads * hd).astype(np.float32)
    out = oracle.attention_decode(q, kc, vc, heads, kv_heads, hd, 1, max_seq).reshape(heads, hd)
    for h in range(heads):
        np.testing.assert_array_equal(out[h], vc[h // 2, 0])


def test_attention_gqa_mapping_and_brute_force():
    heads, kv_heads, hd, max_seq, seq = 14, 2, 64, 40, 33
    rng = rc.philox(8)
    kc = rng.normal(0, 1, (kv_heads, max_seq, hd)).astype(np.float32)
    vc = rng.normal(0, 1, (kv_heads, max_seq, hd)).astype(np.float32)
    # equal keys: every head returns the mean of its kv head's values
    flat = np.repeat(kc[:, :1], max_seq, 1)
    q = rng.normal(0, 1, heads * hd).astype(np.float32)
    out = oracle.attention_decode(q, flat, vc, heads, kv_heads, hd, seq, max_seq)
    for h in range(heads):
        np.testing.assert_allclose(out[h * hd:(h + 1) * hd], vc[h // 7, :seq].mean(0),
                                   atol=1e-5)
    out = oracle.attention_decode(q, kc, vc, heads, kv_heads, hd, seq, max_seq)
    np.testing.assert_allclose(out, _attention64(q, kc, vc, heads, kv_heads, hd, seq),
                               atol=2e-5)


def test_silu_mul_closed_form():
    g = np.array([-8, -1, -0.5, 0, 0.25, 1, 3, 20], np.float32)
    u = np.array([1, 2, -1, 5, 0.5, -3, 1, 1], np.float32)
    out = oracle.silu_mul(g, u)
    g64 = g.astype(np.float64)
    np.testing.assert_allclose(out, g64 / (1 + np.exp(-g64)) * u, rtol=1e-6, atol=1e-7)
    assert out[3] == 0.0
    assert abs(out[-1] - 20.0) < 1e-6


# --------------------------------------------------------- whole model --

TINY = dict(layers=2, hidden=64, heads=4, kv_heads=2, inter=96, vocab=50, max_seq=16)


def tiny_weights(seed=9, **dims):
    d = dict(TINY, **dims)
    rng = rc.philox(seed)
    L, H, I, V = d["layers"], d["hidden"], d["inter"], d["vocab"]
    kv = d["kv_heads"] * H // d["heads"]

    def n(*shape, std=0.1):
        return rng.normal(0, std, shape).astype(np.float32)
    return d, {
        "embed": n(V, H, std=1.0), "final_norm": 1 + n(H), "in_norm": 1 + n(L, H),
        "post_norm": 1 + n(L, H), "wq": n(L, H, H), "bq": n(L, H), "wk": n(L, kv, H),
        "bk": n(L, kv), "wv": n(L, kv, H), "bv": n(L, kv), "wo": n(L, H, H),
        "wg": n(L, I, H), "wu": n(L, I, H), "wd": n(L, H, I),
    }


def model64_step(w, d, tokens, theta=1e6, eps=1e-6):
    """An independent float64 forward of the whole sequence (causal), the
    reference's op order: pre-norm attention and MLP blocks with residuals,
    rotate-half RoPE, GQA, SiLU gate, tied LM head.  Returns the logits of
    every position."""
    H, heads, kvh = d["hidden"], d["heads"], d["kv_heads"]
    hd = H // heads
    T = len(tokens)
    f = {k: v.astype(np.float64) for k, v in w.items()}
    x = f["embed"][tokens]

    def norm(v, g):
        return v / np.sqrt(np.mean(v * v, -1, keepdims=True) + eps) * g

    pos = np.arange(T)[:, None]
    ang = pos * theta ** (-2.0 * np.arange(hd // 2) / hd)

    def rope(m, nh):
        m = m.reshape(T, nh, hd)
        a, b = m[..., :hd // 2], m[..., hd // 2:]
        c, s = np.cos(ang)[:, None], np.sin(ang)[:, None]
        return np.concatenate([a * c - b * s, b * c + a * s], -1)
    mask = np.tril(np.ones((T, T), bool))
    for layer in range(d["layers"]):
        h = norm(x, f["in_norm"][layer])
        q = rope(h @ f["wq"][layer].T + f["bq"][layer], heads)
        k = rope(h @ f["wk"][layer].T + f["bk"][layer], kvh)
        v = (h @ f["wv"][layer].T + f["bv"][layer]).reshape(T, kvh, hd)
        att = np.zeros((T, heads, hd))
        for head in range(heads):
            g = head // (heads // kvh)
            s = q[:, head] @ k[:, g].T / np.sqrt(hd)
            s = np.where(mask, s, -np.inf)
            p = np.exp(s - s.max(1, keepdims=True))
            att[:, head] = (p / p.sum(1, keepdims=True)) @ v[:, g]
        x = x + att.reshape(T, H) @ f["wo"][layer].T
        h = norm(x, f["post_norm"][layer])
        gate, up = h @ f["wg"][layer].T, h @ f["wu"][layer].T
        x = x + (gate / (1 + np.exp(-gate)) * up) @ f["wd"][layer].T
    return norm(x, f["final_norm"]) @ f["embed"].T


def test_model_matches_float64_forward():
    d, w = tiny_weights()
    m = oracle.Model(w, **d)
    tokens = [3, 17, 42, 0, 49, 8]
    ref = model64_step(w, d, tokens)
    idx, logits = m.prefill(tokens[:1], logits=True)
    np.testing.assert_allclose(logits, ref[0], rtol=1e-4, atol=1e-4)
    for t in range(1, len(tokens)):
        idx, logits = m.decode(tokens[t], t, logits=True)
        np.testing.assert_allclose(logits, ref[t], rtol=1e-4, atol=1e-4)
        assert idx == int(np.argmax(ref[t]))


def test_prefill_equals_decode_steps():
    d, w = tiny_weights(seed=10)
    tokens = [5, 1, 44, 30, 12, 9, 9, 2]
    a = oracle.Model(w, **d)
    b = oracle.Model(w, **d)
    ia, la = a.prefill(tokens, logits=True)
    ib, lb = b.prefill(tokens[:1], logits=True)
    for t in range(1, len(tokens)):
        ib, lb = b.decode(tokens[t], t, logits=True)
    assert ia == ib
    np.testing.assert_allclose(la, lb, rtol=1e-5, atol=1e-5)


def test_model_rejects_bad_input():
    d, w = tiny_weights()
    m = oracle.Model(w, **d)
    with pytest.raises(ValueError):
        m.prefill([d["vocab"]])
    with pytest.raises(ValueError):
        m.decode(0, d["max_seq"])
    with pytest.raises(ValueError):
        oracle.Model(w, **dict(d, heads=3))
