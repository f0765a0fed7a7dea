"""The fused decode-step kernels one by one (include/infer_decode.h), the
launches the headline decode step runs, against exact host results.

Bit-exact design.  The weights are random int8 with power-of-two group
scales that differ per (row, group); the activations after the RMSNorm
(or, without a norm, the inputs) are 0 except for one element per 16-value
chunk, which is +-1 or +-2.  Every product q * s * x then has at most 16
significant bits on a grid of 2^-9 and every partial sum fits in FP32's 24
bits, so the kernel's FP32 sum is exact in any order and its BF16 output
must equal bf16(exact) bit for bit.  Rotating the nonzero element over the
16 slots of a chunk across launches puts every (row, column) weight byte
into some output, so the int8 unpacking, the group-scale indexing
(row * K/64 + k/64), the row -> output mapping and the bias indexing are
all checked exactly (the north star's "bit-exact" requirement), at the
decode step's shapes, the R = 2 row tails, the three-descriptor q|k|v
launch and K at the 1/2/4/5/8-slab boundaries.

The SiLU-mul output (expf on the GPU), the split-attention merge with real
softmax weights and the full-vocabulary LM head are then checked against
float64 with the error bound their arithmetic allows; the LM head's argmax
must be exact wherever the top-two margin exceeds that bound, and planted
ties (tests/test_cuda.cpp:790-880) resolve to the lowest index.
"""
import numpy as np
import pytest

import refcases as rc
from helpers import bf16_out, to_dev, words

pytestmark = pytest.mark.gpu

EPS = 1e-6


@pytest.fixture(scope="module")
def dec():
    import decode_hip
    decode_hip.load()
    return decode_hip


def f32(v):
    return np.asarray(v, dtype=np.float32)


def bf16(v):
    """Exact float64/float32 values -> BF16 words (RNE)."""
    return rc.bf16_words(np.asarray(v, dtype=np.float64).astype(np.float32))


def pow2_scales(n, k, salt=0):
    """BF16 scales 2^-(2 .. 6), different for neighbouring rows and groups."""
    r = np.arange(n)[:, None]
    g = np.arange(k // 64)[None, :]
    return bf16(2.0 ** -(2 + (3 * r + g + salt) % 5))


def sparse_positions(k, t):
    c = np.arange(k // 16)
    return 16 * c + (c + t) % 16


def exact_gemv(q, s_words, xv, bias_words=None, grid_bits=9):
    """sum_k q s x (+ bias) in float64, asserting the design keeps it exact
    in FP32 (every partial sum on the grid of 2^-grid_bits within 24 bits)."""
    s = rc.bf16_values(s_words).astype(np.float64)
    n, k = q.shape
    deq = q.astype(np.float64) * np.repeat(s, 64, axis=1)[:, :k]
    terms = deq * xv.astype(np.float64)[None, :]
    assert np.all(np.abs(terms).sum(axis=1) * 2 ** grid_bits < 2 ** 24), "design not exact"
    y = terms.sum(axis=1)
    if bias_words is not None:
        y = y + rc.bf16_values(bias_words).astype(np.float64)
    return y


def norm_input(k, t, rng):
    """x (BF16) and norm weight whose BF16-rounded RMSNorm is exactly
    +-1 / +-2 at one element per chunk and 0 elsewhere; returns
    (x words, norm words, xn float64)."""
    pos = sparse_positions(k, t)
    x = np.zeros(k, np.float32)
    x[pos] = rng.choice([-1.0, 1.0], size=pos.size)
    nw = rc.bf16_values(rc.bf16_normal(rng, (k,)))
    nw[pos] = rng.choice([0.25, 0.5], size=pos.size)
    # The kernel's arithmetic (FP32): scale = 1 / sqrt(sum(x^2) / k + eps),
    # xn = bf16((x * scale) * w).
    ss = f32(pos.size)
    scale = f32(1.0) / np.sqrt(ss / f32(k) + f32(EPS))
    v = (f32(x) * scale) * f32(nw)
    xn = rc.bf16_values(rc.bf16_words(v)).astype(np.float64)
    assert set(np.unique(np.abs(xn[pos]))) <= {1.0, 2.0}
    assert np.all(xn[np.setdiff1d(np.arange(k), pos)] == 0)
    # |v| is within 1e-4 of 1 or 2: far from a BF16 rounding boundary, so an
    # ulp of difference in the GPU's sqrt or division cannot change xn.
    assert np.all(np.abs(np.abs(v[pos]) / np.abs(xn[pos]) - 1) < 1e-4)
    return rc.bf16_words(x), rc.bf16_words(nw), xn


def w8_rows(rng, n, k):
    return rng.integers(-127, 128, size=(n, k), dtype=np.int8)


def dyadic_bias(rng, n):
    return bf16(rng.integers(-128, 129, size=n) / 64.0)


# ------------------------------------------------ RMSNorm + q|k|v GEMVs --

NORM_GEMV_SHAPES = [
    # (K, (n per GEMV)), K at 1, 2 and 4 slabs of 1024
    (896, (896, 128, 128)),    # the decode step's q|k|v
    (64, (3, 5, 130)),         # one chunk per lane, R = 2 tails
    (1024, (1, 897)),
    (1088, (257,)),            # two slabs, the second mostly past K
    (2048, (64, 2, 33)),
    (4096, (130,)),
]


@pytest.mark.parametrize("shape", NORM_GEMV_SHAPES, ids=lambda s: f"k{s[0]}_n{'-'.join(map(str, s[1]))}")
def test_rms_norm_gemv_bit_exact(dec, dev, shape):
    k, ns = shape
    rng = rc.philox(100 + k)
    ws = [w8_rows(rng, n, k) for n in ns]
    ss = [pow2_scales(n, k, salt=i) for i, n in enumerate(ns)]
    bs = [dyadic_bias(rng, n) if i != 1 else None for i, n in enumerate(ns)]
    dws, dss = [to_dev(w, dev) for w in ws], [to_dev(s, dev) for s in ss]
    dbs = [to_dev(b, dev) if b is not None else None for b in bs]
    slots = range(16) if k in (896, 64) else (0, 7, 15)
    for t in slots:
        xw, nw, xn = norm_input(k, t, rng)
        outs = [bf16_out((n,), dev) for n in ns]
        dec.rms_norm_gemv_w8a16(to_dev(xw, dev), to_dev(nw, dev), EPS, k,
                                [(dws[i], dss[i], dbs[i], outs[i], n) for i, n in enumerate(ns)])
        for i, n in enumerate(ns):
            exp = bf16(exact_gemv(ws[i], ss[i], xn, bs[i]))
            got = words(outs[i])
            bad = np.nonzero(got != exp)[0]
            assert bad.size == 0, (f"K={k} gemv {i} slot {t}: {bad.size}/{n} rows differ, "
                                   f"first row {bad[0]}: {got[bad[0]]:#06x} vs {exp[bad[0]]:#06x}")


def test_rms_norm_gemv_matches_oracle_on_real_inputs(dec, orc, dev):
    # Config-1 style operands (random BF16 scales and activations): the
    # fused launch against the oracle's rms_norm + linear on the same
    # BF16-rounded normalised input, within the parity bar.
    from helpers import check_close
    rng = rc.philox(7)
    k = 896
    x = rc.bf16_normal(rng, (k,))
    nw = rc.bf16_normal(rng, (k,), 0.5)
    xn = rc.bf16_values(rc.bf16_words(orc.rms_norm(rc.bf16_values(x), rc.bf16_values(nw), EPS)))
    calls, exps = [], []
    for n in (896, 128, 128):
        q, s = rc.w8a16_synthetic(rng, n, k)
        b = rc.bf16_normal(rng, (n,), 0.1)
        exps.append(orc.linear_fp32(orc.dequant_w8a16(q, s), rc.bf16_values(b), xn))
        calls.append((to_dev(q, dev), to_dev(s, dev), to_dev(b, dev), bf16_out((n,), dev), n))
    dec.rms_norm_gemv_w8a16(to_dev(x, dev), to_dev(nw, dev), EPS, k, calls)
    for (_, _, _, y, n), e in zip(calls, exps):
        stats = check_close(words(y), e, what=f"q|k|v n={n}")
        assert stats["bit_identical"] > 0.95, stats


# ------------------------------------------ RMSNorm + gate|up + SiLU-mul --

def silu_mul_expected(g_words, u_words):
    """Two candidate BF16 words for bf16(silu(g) * u), g and u BF16: from
    float64 and from FP32 arithmetic.  They differ only where the value sits
    within FP32 rounding (expf, the division, the product) of a BF16
    rounding boundary, or where FP32's expf overflows; the kernel may give
    either there, and must give the common word everywhere else."""
    g = rc.bf16_values(g_words).astype(np.float64)
    u = rc.bf16_values(u_words).astype(np.float64)
    with np.errstate(over="ignore"):
        v64 = g / (1.0 + np.exp(-g)) * u
        g32 = g.astype(np.float32)
        v32 = (g32 / (np.float32(1) + np.exp(-g32))) * u.astype(np.float32)
    a, b = bf16(v64), rc.bf16_words(v32)
    return a, b


@pytest.mark.parametrize("k,n", [(896, 4864), (64, 5), (1024, 33), (2048, 130)])
def test_rms_norm_gate_up_silu(dec, dev, k, n):
    rng = rc.philox(200 + k)
    wg, wu = w8_rows(rng, n, k), w8_rows(rng, n, k)
    # smaller scales keep |gate| well inside expf's range
    sg, su = pow2_scales(n, k, 0), pow2_scales(n, k, 2)
    sg = bf16(rc.bf16_values(sg) / 16.0)
    su = bf16(rc.bf16_values(su) / 16.0)
    dwg, dwu, dsg, dsu = (to_dev(a, dev) for a in (wg, wu, sg, su))
    ambiguous = 0
    for t in (range(16) if n == 4864 else (0, 9)):
        xw, nw, xn = norm_input(k, t, rng)
        g = bf16(exact_gemv(wg, sg, xn, grid_bits=10))  # exact sums, one BF16 rounding
        u = bf16(exact_gemv(wu, su, xn, grid_bits=10))
        a, b = silu_mul_expected(g, u)
        out = bf16_out((n,), dev)
        dec.rms_norm_gate_up_silu_w8a16(to_dev(xw, dev), to_dev(nw, dev), EPS, k, dwg, dsg, dwu,
                                        dsu, out, n)
        got = words(out)
        ok = (got == a) | (got == b)
        assert ok.all(), (f"K={k} slot {t}: {np.sum(~ok)} rows differ, first "
                          f"{np.nonzero(~ok)[0][0]}")
        ambiguous += int(np.sum(a != b))
    assert ambiguous <= max(2, n // 100), ambiguous


# ------------------------------------------- down GEMV + residual (rows) --

@pytest.mark.parametrize("k,n", [(4864, 896), (64, 3), (896, 897), (1024, 4), (1088, 65),
                                 (4096, 33), (5120, 7), (8192, 130)])
@pytest.mark.parametrize("bias", ["none", "separate", "residual"])
def test_gemv_w8a16_rows_bit_exact(dec, dev, k, n, bias):
    rng = rc.philox(300 + k + n)
    q = w8_rows(rng, n, k)
    s = pow2_scales(n, k, 1)
    dq, ds = to_dev(q, dev), to_dev(s, dev)
    b = dyadic_bias(rng, n) if bias != "none" else None
    for t in ((0, 3, 8, 15) if k == 4864 else (0, 11)):
        pos = sparse_positions(k, t)
        xv = np.zeros(k, np.float64)
        xv[pos] = rng.choice([-2.0, -1.0, 1.0, 2.0], size=pos.size)
        y = bf16_out((n,), dev)
        if bias == "residual":
            import torch
            y.copy_(to_dev(b, dev))   # the output holds the residual and is updated in place
            dec.gemv_w8a16_rows(dq, ds, y, to_dev(bf16(xv), dev), y, n, k)
        else:
            dec.gemv_w8a16_rows(dq, ds, to_dev(b, dev) if b is not None else None,
                                to_dev(bf16(xv), dev), y, n, k)
        exp = bf16(exact_gemv(q, s, xv, b))
        got = words(y)
        bad = np.nonzero(got != exp)[0]
        assert bad.size == 0, (f"K={k} n={n} slot {t}: {bad.size} rows differ, first {bad[0]}: "
                               f"{got[bad[0]]:#06x} vs {exp[bad[0]]:#06x}")


# --------------------------- split-attention merge + o GEMV + residual --

# At max_seq 2048 the split attention has 8 spans of 256 positions: these
# positions give 1 to 8 splits, their edges, and one past the capacity
# (clamped to 2047).  At max_seq 1024 the split form has 8 spans of 128 at
# head_dim 128; at head_dim 64 the decode step uses the whole-context
# attention there, and the merge entry point normalises a single record.
MERGE_POSITIONS = {2048: (0, 1, 255, 256, 511, 512, 1023, 1024, 1200, 1535, 1536, 1791, 1792,
                          2046, 2047, 3000),
                   1024: (0, 1, 127, 128, 511, 600, 895, 896, 1023, 1500)}


def merge_case(heads, hd, max_seq, rng, exact):
    import decode_hip
    span = decode_hip.attention_decode_span(max_seq, hd)
    splits = decode_hip.attention_decode_splits(max_seq, hd)
    rec = hd + 2
    part = np.full((heads, splits, rec), np.nan, np.float32)  # unused records: NaN
    if exact:
        # m = 0 everywhere and l = (1, 0, 0, ...): every used split has weight
        # exactly 1, so attn = sum of the used splits' acc (multiples of 1/8).
        part[:, :, :hd] = rng.integers(-1, 2, size=(heads, splits, hd)) / 8.0
        part[:, :, hd] = 0.0
        part[:, :, hd + 1] = 0.0
        part[:, 0, hd + 1] = 1.0
    else:
        part[:, :, :hd] = rng.normal(0, 3, size=(heads, splits, hd))
        part[:, :, hd] = rng.normal(0, 2, size=(heads, splits))
        part[:, :, hd + 1] = rng.uniform(1, 60, size=(heads, splits))
    return part, span, splits


def merge_expected(part, pos, span, max_seq, hd):
    """The merged attention output per head, float64, then rounded to BF16."""
    used = min(pos, max_seq - 1) // span + 1
    p = part[:, :used].astype(np.float64)
    m = p[:, :, hd]
    big = m.max(axis=1, keepdims=True)
    e = np.exp(m - big)
    a = (p[:, :, :hd] * e[:, :, None]).sum(axis=1) / (p[:, :, hd + 1] * e).sum(axis=1)[:, None]
    return a.reshape(-1)


@pytest.mark.parametrize("max_seq", [2048, 1024])
@pytest.mark.parametrize("heads,hd,n,w8", [(14, 64, 896, True), (14, 64, 896, False),
                                           (2, 128, 130, True), (32, 64, 64, True),
                                           (4, 128, 9, False)])
def test_attention_merge_o_proj_bit_exact(dec, dev, heads, hd, n, w8, max_seq):
    import torch
    rng = rc.philox(400 + heads * hd + n)
    k = heads * hd
    if w8:
        wq = w8_rows(rng, n, k)
        s = pow2_scales(n, k, 3)
        deq = wq.astype(np.float64) * np.repeat(rc.bf16_values(s).astype(np.float64), 64, 1)
        dw, ds = to_dev(wq, dev), to_dev(s, dev)
    else:
        w = bf16(rng.integers(-127, 128, size=(n, k)) / 64.0)
        deq = rc.bf16_values(w).astype(np.float64)
        dw, ds = to_dev(w, dev), None
    part, span, splits = merge_case(heads, hd, max_seq, rng, exact=True)
    dpart = torch.from_numpy(part.reshape(-1)).to(dev)
    x0 = rc.bf16_normal(rng, (n,))
    for pos in MERGE_POSITIONS[max_seq]:
        attn = merge_expected(part, pos, span, max_seq, hd)
        assert np.all(rc.bf16_values(bf16(attn)) == attn)  # exact in BF16 by design
        terms = deq * attn[None, :]
        assert np.all(np.abs(terms).sum(axis=1) * 2 ** 10 < 2 ** 24), "design not exact"
        ysum = terms.sum(axis=1).astype(np.float32)        # exact
        exp = rc.bf16_words(ysum + rc.bf16_values(x0))     # one FP32 add, then BF16
        x = to_dev(x0, dev)
        dpos = torch.tensor([pos], dtype=torch.int32, device=dev)
        dec.attention_merge_o_proj(dpart, dpos, heads, hd, span, splits, max_seq, dw, ds, x, n)
        got = words(x)
        bad = np.nonzero(got != exp)[0]
        assert bad.size == 0, (f"pos {pos} ({min(pos, max_seq - 1) // span + 1} splits): "
                               f"{bad.size}/{n} rows differ, first {bad[0]}")


@pytest.mark.parametrize("w8", [True, False])
def test_attention_merge_o_proj_softmax_weights(dec, dev, w8):
    # Real merge weights e^(m_i - M) / sum l_i e^(m_i - M) at every split
    # count, against float64 (the BF16 rounding of the merged attention is
    # the only coarse step: bound 2^-8 |a| per element through the GEMV).
    import torch
    rng = rc.philox(500 + w8)
    heads, hd, n, max_seq = 14, 64, 896, 2048
    k = heads * hd
    if w8:
        q, s = rc.w8a16_synthetic(rng, n, k)
        deq = q.astype(np.float64) * np.repeat(rc.bf16_values(s).astype(np.float64), 64, 1)
        dw, ds = to_dev(q, dev), to_dev(s, dev)
    else:
        w = rc.bf16_normal(rng, (n, k), 0.02)
        deq = rc.bf16_values(w).astype(np.float64)
        dw, ds = to_dev(w, dev), None
    part, span, splits = merge_case(heads, hd, max_seq, rng, exact=False)
    dpart = torch.from_numpy(part.reshape(-1)).to(dev)
    x0 = rc.bf16_normal(rng, (n,))
    for pos in MERGE_POSITIONS[max_seq]:
        attn = merge_expected(part, pos, span, max_seq, hd)
        y = deq @ attn + rc.bf16_values(x0)
        bound = np.abs(deq) @ (np.abs(attn) * 2.0 ** -8) + 2.0 ** -8 * np.abs(y) + 1e-6
        x = to_dev(x0, dev)
        dpos = torch.tensor([pos], dtype=torch.int32, device=dev)
        dec.attention_merge_o_proj(dpart, dpos, heads, hd, span, splits, max_seq, dw, ds, x, n)
        got = rc.bf16_values(words(x)).astype(np.float64)
        err = np.abs(got - y)
        assert np.all(err <= bound), (pos, float(np.max(err / bound)))


# ------------------------------------------- RMSNorm + LM head + argmax --

def lm_workspace(dec, dev, vocab):
    import torch
    return torch.zeros(dec.lm_head_decode_workspace_bytes(vocab), dtype=torch.uint8, device=dev)


def rms_preserving_input(rng, k):
    """BF16 x whose RMSNorm with weight 1 rounds back to x itself (its
    mean square is within 1e-3 of 1), so xn is known exactly."""
    for _ in range(100):
        v = rng.normal(0, 1, k)
        v = v / np.sqrt(np.mean(v * v))
        x = rc.bf16_words(v.astype(np.float32))
        xf = rc.bf16_values(x)
        ms = np.float32(np.sum(xf.astype(np.float64) ** 2)) / np.float32(k)
        scale = np.float32(1) / np.sqrt(ms + np.float32(EPS))
        if abs(float(scale) - 1.0) < 1e-3 and np.all(rc.bf16_words(xf * scale) == x):
            return x
    raise AssertionError("no RMS-preserving input found")


def test_lm_head_decode_full_vocab_exact_argmax(dec, dev):
    # Config 2's shape and distribution, through the decode step's fused
    # kernel: the argmax must be the float64 argmax wherever the top-two
    # margin exceeds the FP32 accumulation bound, with a planted tie.
    import torch
    vocab, k = rc.VOCAB, rc.HIDDEN
    rng = rc.philox(2)
    e = rc.bf16_normal(rng, (vocab, k), 0.02)
    x = rms_preserving_input(rng, k)
    ones = rc.bf16_words(np.ones(k, np.float32))
    ev = rc.bf16_values(e).astype(np.float64)
    xv = rc.bf16_values(x).astype(np.float64)
    ws = lm_workspace(dec, dev, vocab)
    de, dx, dn = to_dev(e, dev), to_dev(x, dev), to_dev(ones, dev)
    for trial in range(3):
        l64 = ev @ xv
        order = np.argsort(-l64, kind="stable")
        bound = k * 2.0 ** -23 * (np.abs(ev) @ np.abs(xv))
        logits = bf16_out((vocab,), dev)
        am = torch.full((1,), -7, dtype=torch.int32, device=dev)
        dec.rms_norm_lm_head_argmax(dx, dn, EPS, de, vocab, k, logits, ws, am)
        got = int(am.cpu().item())
        top, second = order[0], order[1]
        if l64[top] - l64[second] > bound[top] + bound[second]:
            assert got == top, (trial, got, top)
        else:
            assert got in (top, second)
        lw = words(logits)
        err = np.abs(rc.bf16_values(lw).astype(np.float64) - l64)
        assert np.all(err <= 2.0 ** -8 * np.abs(l64) + bound + 1e-30)
        if trial == 0:
            # plant the maximum twice: rows 1000 and 150000 become copies of
            # the current winner scaled up; ties go to the lower index
            e[1000] = rc.bf16_words(rc.bf16_values(e[top]) * 1.5)
            e[150000] = e[1000]
            ev[1000] = ev[150000] = rc.bf16_values(e[1000])
            de = to_dev(e, dev)
        elif trial == 1:
            assert got == 1000, got
            # the workspace counter is left at zero: a third call works too


@pytest.mark.parametrize("case", [c for c in rc.LM_HEAD_TIE_CASES if c[1] % 8 == 0],
                         ids=lambda c: "x".join(map(str, c)))
def test_lm_head_decode_tie_cases(dec, dev, case):
    # The reference's planted ties (tests/test_cuda.cpp:790-880: rows tie_a
    # and tie_b all 2.0) with a normalised input of exact +-1 / 2 values, so
    # both tied rows have the same FP32 sum in any order; the lower index
    # wins.  (K = 10 and 4 are below the fused kernel's 8-value chunks; the
    # runtime takes the two-kernel LM head there.)
    import torch
    vocab, k, ta, tb = case
    rng = rc.philox(600 + vocab)
    e = bf16(rng.integers(-64, 64, size=(vocab, k)) / 64.0)
    e[ta] = e[tb] = rc.bf16_words(np.float32(2.0))
    pos = sparse_positions(k, 3)
    x = np.zeros(k, np.float32)
    x[pos] = 1.0
    nw = np.ones(k, np.float32)
    nw[pos] = rng.choice([0.25, 0.5], size=pos.size)
    xw, nww = rc.bf16_words(x), rc.bf16_words(nw)
    xn = np.zeros(k)
    xn[pos] = nw[pos] * 4.0
    l64 = rc.bf16_values(e).astype(np.float64) @ xn
    assert l64.argmax() == ta and l64[ta] == l64[tb]
    ws = lm_workspace(dec, dev, vocab)
    for _ in range(2):
        logits = bf16_out((vocab,), dev)
        am = torch.full((1,), -7, dtype=torch.int32, device=dev)
        dec.rms_norm_lm_head_argmax(to_dev(xw, dev), to_dev(nww, dev), EPS, to_dev(e, dev), vocab,
                                    k, logits, ws, am)
        assert int(am.cpu().item()) == ta
        np.testing.assert_array_equal(words(logits), bf16(l64))


# ------------------------------------- RMSNorm + q|k|v + RoPE + KV store --

def rope_candidates(a_words, b_words, cs):
    """BF16 words the rotated pair may round to: (a c - b s, b c + a s) with
    FP32 products rounded separately, or with either product fused into
    the add (FMA contraction), or exactly."""
    a = rc.bf16_values(a_words).astype(np.float64)
    b = rc.bf16_values(b_words).astype(np.float64)
    c, s = cs[:, 0].astype(np.float64), cs[:, 1].astype(np.float64)
    f32 = lambda v: np.asarray(v, np.float64).astype(np.float32)  # noqa: E731
    r32 = lambda v: f32(v).astype(np.float64)  # one FP32 rounding  # noqa: E731

    def forms(x, y, sign):  # x c + sign * y s
        return [rc.bf16_words(f32(r32(x * c) + sign * r32(y * s))),
                rc.bf16_words(f32(x * c + sign * r32(y * s))),
                rc.bf16_words(f32(r32(x * c) + sign * y * s)),
                rc.bf16_words(f32(x * c + sign * y * s))]
    return forms(a, b, -1.0), forms(b, a, 1.0)


QKV_ROPE_SHAPES = [  # (in_features, heads, kv_heads, head_dim, max_seq)
    (896, 14, 2, 64, 1024),     # Qwen2.5-0.5B
    (1024, 4, 1, 128, 64),      # head_dim 128, GQA 4
    (512, 8, 8, 64, 16),        # no grouping
]


@pytest.mark.parametrize("shape", QKV_ROPE_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_rms_norm_qkv_rope(dec, dev, shape):
    import torch
    k, heads, kvh, hd, max_seq = shape
    half = hd // 2
    rng = rc.philox(700 + k + heads)
    nq, nkv = heads * hd, kvh * hd
    w = {n: w8_rows(rng, m, k) for n, m in (("q", nq), ("k", nkv), ("v", nkv))}
    s = {n: pow2_scales(w[n].shape[0], k, salt=i) for i, n in enumerate("qkv")}
    b = {n: dyadic_bias(rng, w[n].shape[0]) for n in "qkv"}
    b["v"] = None  # a null bias too
    dw = {n: (to_dev(w[n], dev), to_dev(s[n], dev), to_dev(b[n], dev) if b[n] is not None
              else None) for n in "qkv"}
    sentinel = np.uint16(0x7FC0)  # NaN: every row but the token's must keep it
    for position in (0, 5, max_seq - 1, max_seq + 100):
        p = min(position, max_seq - 1)
        xw, nw, xn = norm_input(k, position % 16, rng)
        y = {n: bf16(exact_gemv(w[n], s[n], xn, b[n])) for n in "qkv"}  # before the rotation
        cs = dec.rope_row(1e6, hd, p)
        kc = torch.full((kvh * max_seq * hd,), -1, dtype=torch.int16, device=dev)
        kc.fill_(int(sentinel.view(np.int16)))
        vc = kc.clone()
        q_out = bf16_out((nq,), dev)
        dpos = torch.tensor([position], dtype=torch.int32, device=dev)
        dec.rms_norm_qkv_rope_w8a16(to_dev(xw, dev), to_dev(nw, dev), EPS, k, dw["q"], dw["k"],
                                    dw["v"], q_out, kc, vc, torch.from_numpy(cs.copy()).to(dev),
                                    dpos, heads, kvh, hd, max_seq)
        kcache = kc.cpu().numpy().view(np.uint16).reshape(kvh, max_seq, hd)
        vcache = vc.cpu().numpy().view(np.uint16).reshape(kvh, max_seq, hd)
        other = np.ones(max_seq, bool)
        other[p] = False
        assert np.all(kcache[:, other] == sentinel) and np.all(vcache[:, other] == sentinel)
        np.testing.assert_array_equal(vcache[:, p].reshape(-1), y["v"])  # v: not rotated
        for name, got in (("q", words(q_out).reshape(-1, hd)), ("k", kcache[:, p])):
            yy = y[name].reshape(-1, hd)
            if p == 0:  # cos 1, sin 0: the rotation is exact
                np.testing.assert_array_equal(got, yy)
                continue
            first, second = rope_candidates(yy[:, :half], yy[:, half:], cs)
            ok1 = np.any([got[:, :half] == c for c in first], axis=0)
            ok2 = np.any([got[:, half:] == c for c in second], axis=0)
            assert ok1.all() and ok2.all(), (name, position, np.argwhere(~ok1)[:3],
                                             np.argwhere(~ok2)[:3])


@pytest.mark.parametrize("weights", ["w8a16", "bf16"])
def test_rms_norm_qkv_rope_negative_position_stores_nothing(dec, dev, weights):
    """A negative position is an empty context: the launch writes q_out and
    nothing in the caches.  The caches are carved out of one tensor with
    guard rows in front of and behind them, which must stay untouched."""
    import torch
    k, heads, kvh, hd, max_seq = 896, 14, 2, 64, 32
    rng = rc.philox(4242)
    nq, nkv = heads * hd, kvh * hd
    xw, nw, xn = norm_input(k, 3, rng)
    cs = dec.rope_row(1e6, hd, 0)  # cos 1, sin 0: q_out is the GEMV itself
    if weights == "w8a16":
        w = {n: w8_rows(rng, m, k) for n, m in (("q", nq), ("k", nkv), ("v", nkv))}
        sc = {n: pow2_scales(w[n].shape[0], k, salt=i) for i, n in enumerate("qkv")}
        dw = {n: (to_dev(w[n], dev), to_dev(sc[n], dev), None) for n in "qkv"}
        exp_q = bf16(exact_gemv(w["q"], sc["q"], xn, None))
    else:
        w = {n: bf16_rows(rng, m, k) for n, m in (("q", nq), ("k", nkv), ("v", nkv))}
        dw = {n: (to_dev(w[n][0], dev), None) for n in "qkv"}
        exp_q = bf16(exact_dot(w["q"][1], xn))
    sentinel = np.uint16(0x7FC0)
    cache_words = kvh * max_seq * hd
    guard = 2 * hd  # guard words on either side of each cache
    buf = torch.full((2 * (cache_words + 2 * guard),), int(sentinel.view(np.int16)),
                     dtype=torch.int16, device=dev)
    kc = buf[guard:guard + cache_words]
    vc = buf[3 * guard + cache_words:3 * guard + 2 * cache_words]
    q_out = bf16_out((nq,), dev)
    dpos = torch.tensor([-1], dtype=torch.int32, device=dev)
    print(f"qkv_rope negative position weights={weights}", flush=True)
    fn = dec.rms_norm_qkv_rope_w8a16 if weights == "w8a16" else dec.rms_norm_qkv_rope_bf16
    fn(to_dev(xw, dev), to_dev(nw, dev), EPS, k, dw["q"], dw["k"], dw["v"], q_out, kc, vc,
       torch.from_numpy(cs.copy()).to(dev), dpos, heads, kvh, hd, max_seq)
    torch.cuda.synchronize()
    assert np.all(buf.cpu().numpy().view(np.uint16) == sentinel), "a cache or guard row changed"
    np.testing.assert_array_equal(words(q_out), exp_q)


# ------------------------------------------- whole-context decode attention --

@pytest.mark.parametrize("heads,kvh", [(14, 2), (4, 4), (8, 1)])
def test_attention_decode_bf16_matches_oracle(dec, orc, dev, heads, kvh):
    """Against the oracle's attention (cpu_ops.cpp:58-91 restated) on the
    same BF16 values: q rotated already, the caches holding rows [0, p];
    rows past p hold NaN and must not matter."""
    import torch
    hd, max_seq = 64, 1024
    rng = rc.philox(800 + heads)
    q = rc.bf16_normal(rng, (heads * hd,), 0.5)
    kcache = rc.bf16_normal(rng, (kvh, max_seq, hd))
    vcache = rc.bf16_normal(rng, (kvh, max_seq, hd))
    for position in (0, 1, 63, 64, 127, 511, 512, 767, 1022, 1023, 2000):
        p = min(position, max_seq - 1)
        kc, vc = kcache.copy(), vcache.copy()
        kc[:, p + 1:] = 0x7FC0
        vc[:, p + 1:] = 0x7FC0
        exp = orc.attention_decode(rc.bf16_values(q), rc.bf16_values(kcache),
                                   rc.bf16_values(vcache), heads, kvh, hd, p + 1, max_seq)
        out = bf16_out((heads * hd,), dev)
        dpos = torch.tensor([position], dtype=torch.int32, device=dev)
        dec.attention_decode_bf16(to_dev(q, dev), to_dev(kc, dev), to_dev(vc, dev), dpos, out,
                                  heads, kvh, hd, max_seq)
        got = rc.bf16_values(words(out)).astype(np.float64)
        e = np.asarray(exp, dtype=np.float64)
        # BF16 output rounding plus FP32 softmax / accumulation error
        tol = 2.0 ** -8 * np.abs(e) + 1e-4 * np.max(np.abs(e))
        assert np.all(np.isfinite(got)), position
        assert np.all(np.abs(got - e) <= tol), (position, float(np.max(np.abs(got - e) / tol)))


# ------------------------ two-halves attention + merge in the o GEMV --

HALF_POSITIONS = (0, 1, 63, 64, 255, 256, 257, 511, 512, 513, 767, 768, 769, 1022, 1023, 2000)


def run_attention_parts(dec, parts, q, kc, vc, dpos, rec, heads, kvh, hd, max_seq):
    """The halves operator for 2 parts, the parts operator otherwise."""
    if parts == 2:
        dec.attention_decode_halves_bf16(q, kc, vc, dpos, rec, heads, kvh, hd, max_seq)
    else:
        dec.attention_decode_parts_bf16(q, kc, vc, dpos, rec, heads, kvh, hd, max_seq, parts)


@pytest.mark.parametrize("parts", [2, 4])
@pytest.mark.parametrize("heads,kvh,max_seq", [(14, 2, 1024), (8, 1, 1024), (4, 4, 1024),
                                               (14, 2, 700), (8, 1, 300)])
def test_attention_decode_halves_matches_oracle(dec, orc, dev, heads, kvh, max_seq, parts):
    """Each part's record against the oracle's attention (cpu_ops.cpp:58-91
    restated): merged on the host in float64 they give the whole context's
    output; rows past p hold NaN and must not matter, and a part past the
    context leaves its record untouched (halves: 512 positions each,
    quarters: 256, whatever the KV capacity; at 700 or 300 positions the
    last live part ends inside the cache's end and the later parts start
    past it)."""
    import torch
    hd, R = 64, dec.PART_RECORD
    span = 1024 // parts
    rng = rc.philox(900 + heads + max_seq)
    q = rc.bf16_normal(rng, (heads * hd,), 0.5)
    kcache = rc.bf16_normal(rng, (kvh, max_seq, hd))
    vcache = rc.bf16_normal(rng, (kvh, max_seq, hd))
    for position in HALF_POSITIONS:
        p = min(position, max_seq - 1)
        kc, vc = kcache.copy(), vcache.copy()
        kc[:, p + 1:] = 0x7FC0
        vc[:, p + 1:] = 0x7FC0
        exp = np.asarray(orc.attention_decode(rc.bf16_values(q), rc.bf16_values(kcache),
                                              rc.bf16_values(vcache), heads, kvh, hd, p + 1,
                                              max_seq), dtype=np.float64)
        rec = torch.full((heads, parts, R), float("nan"), dtype=torch.float32, device=dev)
        dpos = torch.tensor([position], dtype=torch.int32, device=dev)
        run_attention_parts(dec, parts, to_dev(q, dev), to_dev(kc, dev), to_dev(vc, dev), dpos,
                            rec, heads, kvh, hd, max_seq)
        r = rec.cpu().numpy().astype(np.float64)
        used = p // span + 1
        assert np.all(np.isfinite(r[:, :used, :hd + 2])), position
        assert np.all(np.isnan(r[:, used:])), f"position {position}: a part past p written"
        m = r[:, :used, hd]
        big = m.max(axis=1, keepdims=True)
        e = np.exp(m - big)
        got = ((r[:, :used, :hd] * e[:, :, None]).sum(axis=1) /
               (r[:, :used, hd + 1] * e).sum(axis=1)[:, None]).reshape(-1)
        tol = 2.0 ** -12 * np.abs(exp) + 1e-5 * np.max(np.abs(exp))  # FP32 softmax / sums
        assert np.all(np.abs(got - exp) <= tol), (position, float(np.max(np.abs(got - exp) / tol)))


@pytest.mark.parametrize("heads,kvh,hd,max_seq", [(14, 2, 64, 2048), (4, 1, 128, 1024),
                                                (8, 8, 64, 512), (16, 2, 128, 2048)])
def test_attention_decode_spans_matches_oracle(dec, orc, dev, heads, kvh, hd, max_seq):
    """infer_hip_attention_decode_spans_bf16 (the split form on a rotated q and
    a cache holding the token): each span's record against the oracle's
    attention (cpu_ops.cpp:58-91 restated), merged on the host in float64;
    rows past p hold NaN and must not matter, spans past the context leave
    their records untouched.  Then the records through
    infer_hip_attention_merge_o_proj against the oracle's output through
    the o-projection (BF16 attention, FP32 GEMV, one rounding with the
    residual), within the GEMV's bar."""
    import torch
    span = dec.attention_decode_span(max_seq, hd)
    splits = dec.attention_decode_splits(max_seq, hd)
    rng = rc.philox(1600 + heads + hd + max_seq)
    q = rc.bf16_normal(rng, (heads * hd,), 0.5)
    kcache = rc.bf16_normal(rng, (kvh, max_seq, hd))
    vcache = rc.bf16_normal(rng, (kvh, max_seq, hd))
    n = 96
    w = rc.bf16_normal(rng, (n, heads * hd), 0.05)
    x0 = rc.bf16_normal(rng, (n,))
    for position in (0, 1, span - 1, span, 2 * span + 5, max_seq - 1, max_seq + 100):
        p = min(position, max_seq - 1)
        kc, vc = kcache.copy(), vcache.copy()
        kc[:, p + 1:] = 0x7FC0
        vc[:, p + 1:] = 0x7FC0
        exp = np.asarray(orc.attention_decode(rc.bf16_values(q), rc.bf16_values(kcache),
                                              rc.bf16_values(vcache), heads, kvh, hd, p + 1,
                                              max_seq), dtype=np.float64)
        rec = torch.full((heads, splits, hd + 2), float("nan"), dtype=torch.float32, device=dev)
        dpos = torch.tensor([position], dtype=torch.int32, device=dev)
        dec.attention_decode_spans_bf16(to_dev(q, dev), to_dev(kc, dev), to_dev(vc, dev), dpos,
                                        rec, heads, kvh, hd, max_seq)
        r = rec.cpu().numpy().astype(np.float64)
        used = p // span + 1
        assert np.all(np.isfinite(r[:, :used])), position
        assert np.all(np.isnan(r[:, used:])), f"position {position}: a span past p written"
        m = r[:, :used, hd]
        big = m.max(axis=1, keepdims=True)
        e = np.exp(m - big)
        got = ((r[:, :used, :hd] * e[:, :, None]).sum(axis=1) /
               (r[:, :used, hd + 1] * e).sum(axis=1)[:, None]).reshape(-1)
        tol = 2.0 ** -12 * np.abs(exp) + 1e-5 * np.max(np.abs(exp))  # FP32 softmax / sums
        assert np.all(np.abs(got - exp) <= tol), (position, float(np.max(np.abs(got - exp) / tol)))
        # the records through the exported merge + o-projection + residual
        if heads * hd <= 4096 and heads <= 32:
            x = to_dev(x0, dev)
            dec.attention_merge_o_proj(rec, dpos, heads, hd, span, splits, max_seq, to_dev(w, dev),
                                       None, x, n)
            a = rc.bf16_values(rc.bf16_words(exp.astype(np.float32))).astype(np.float64)
            ref = rc.bf16_values(w).astype(np.float64) @ a + rc.bf16_values(x0)
            got_x = rc.bf16_values(words(x)).astype(np.float64)
            bound = np.maximum(1e-2 * np.abs(ref), 2e-2 * np.sqrt(np.mean(ref ** 2)))
            assert np.all(np.abs(got_x - ref) <= bound), (position, float(np.max(np.abs(got_x - ref))))


def exact_part_records(rng, heads, parts, pos, max_seq, hd, R):
    """Records whose merge is exact: every live part has m = 0, the first
    l = 1 and the others l = 0 (merge weights exactly 1), accumulators in
    multiples of 1/8; parts past the context hold NaN.  Returns the records
    and the merged attention."""
    acc = rng.integers(-1, 2, size=(heads, parts, hd)) / 8.0
    live = min(pos, max_seq - 1) // (max_seq // parts) + 1
    part = np.full((heads, parts, R), np.nan, np.float32)
    part[:, :live, :hd] = acc[:, :live]
    part[:, :live, hd] = 0.0
    part[:, :live, hd + 1] = 0.0
    part[:, 0, hd + 1] = 1.0
    attn = acc[:, :live].sum(axis=1).reshape(-1)
    assert np.all(rc.bf16_values(bf16(attn)) == attn)  # exact in BF16 by design
    return part, attn


PART_O_POSITIONS = (0, 1, 255, 256, 511, 512, 513, 767, 768, 1023, 2000)


@pytest.mark.parametrize("parts", [2, 4])
@pytest.mark.parametrize("heads,n", [(14, 896), (2, 130), (64, 65)])
def test_attention_halves_o_proj_bit_exact(dec, dev, heads, n, parts):
    """Merge weights exactly 1 and accumulators in multiples of 1/8
    (exact_part_records): the merged attention and the o GEMV with
    power-of-two scales are exact, so the result is compared bit for bit.
    Parts past the context hold NaN and must not reach the output.  Two
    parts through the halves operator, four through the parts operator."""
    import torch
    hd, max_seq, R = 64, 1024, dec.PART_RECORD
    rng = rc.philox(950 + heads + n + parts)
    k = heads * hd
    wq = w8_rows(rng, n, k)
    s = pow2_scales(n, k, 5)
    deq = wq.astype(np.float64) * np.repeat(rc.bf16_values(s).astype(np.float64), 64, 1)
    dw, ds = to_dev(wq, dev), to_dev(s, dev)
    x0 = rc.bf16_normal(rng, (n,))
    for pos in PART_O_POSITIONS:
        part, attn = exact_part_records(rng, heads, parts, pos, max_seq, hd, R)
        terms = deq * attn[None, :]
        assert np.all(np.abs(terms).sum(axis=1) * 2 ** 10 < 2 ** 24), "design not exact"
        exp = rc.bf16_words(terms.sum(axis=1).astype(np.float32) + rc.bf16_values(x0))
        x = to_dev(x0, dev)
        dpos = torch.tensor([pos], dtype=torch.int32, device=dev)
        rec = torch.from_numpy(part.reshape(-1)).to(dev)
        if parts == 2:
            dec.attention_halves_o_proj_w8a16(rec, dpos, heads, max_seq, dw, ds, x, n)
        else:
            dec.attention_parts_o_proj_w8a16(rec, dpos, heads, max_seq, parts, dw, ds, x, n)
        got = words(x)
        bad = np.nonzero(got != exp)[0]
        assert bad.size == 0, f"pos {pos}: {bad.size}/{n} rows differ, first {bad[0]}"


# ------------------------------------ the same launches on BF16 weights --
#
# The W16A16 decode step runs the kernels above instantiated for 8 BF16
# weights per 16-byte chunk (include/infer_decode.h's _bf16 siblings).  The
# bit-exact design carries over: weights are integers / 64 (at most 7
# significant bits, exact in BF16), so with the sparse +-1 / +-2 inputs
# every FP32 partial sum is exact and the BF16 output must equal
# bf16(exact).  Rotating the nonzero slot over 16 positions puts every
# weight of a row into some output (a BF16 chunk holds 8 of them, so each
# chunk is hit by two of the 16 slots), checking the BF16 unpacking and the
# chunk -> input mapping at the K limits of this format (512 weights per
# slab: 1, 2 and 4 slabs for the norm launches, 10 for the rows launch).

def bf16_rows(rng, n, k, div=64.0):
    """BF16 words of integers in [-127, 127] / div, and their values."""
    w = bf16(rng.integers(-127, 128, size=(n, k)) / div)
    return w, rc.bf16_values(w).astype(np.float64)


def exact_dot(deq, xv, bias_words=None, grid_bits=6):
    terms = deq * xv.astype(np.float64)[None, :]
    assert np.all(np.abs(terms).sum(axis=1) * 2 ** grid_bits < 2 ** 24), "design not exact"
    y = terms.sum(axis=1)
    if bias_words is not None:
        y = y + rc.bf16_values(bias_words).astype(np.float64)
    return y


NORM_GEMV_BF16_SHAPES = [
    (896, (896, 128, 128)),    # the decode step's q|k|v (2 slabs)
    (64, (3, 5, 130)),
    (512, (1, 897)),           # one slab
    (576, (257,)),             # two slabs, the second mostly past K
    (2048, (64, 2, 33)),       # four slabs, the limit
]


@pytest.mark.parametrize("shape", NORM_GEMV_BF16_SHAPES,
                         ids=lambda s: f"k{s[0]}_n{'-'.join(map(str, s[1]))}")
def test_rms_norm_gemv_bf16_bit_exact(dec, dev, shape):
    k, ns = shape
    rng = rc.philox(1100 + k)
    ws = [bf16_rows(rng, n, k) for n in ns]
    bs = [dyadic_bias(rng, n) if i != 1 else None for i, n in enumerate(ns)]
    dws = [to_dev(w, dev) for w, _ in ws]
    dbs = [to_dev(b, dev) if b is not None else None for b in bs]
    for t in (range(16) if k in (896, 64) else (0, 7, 8, 15)):
        xw, nw, xn = norm_input(k, t, rng)
        outs = [bf16_out((n,), dev) for n in ns]
        dec.rms_norm_gemv_bf16(to_dev(xw, dev), to_dev(nw, dev), EPS, k,
                               [(dws[i], dbs[i], outs[i], n) for i, n in enumerate(ns)])
        for i, n in enumerate(ns):
            exp = bf16(exact_dot(ws[i][1], xn, bs[i]))
            got = words(outs[i])
            bad = np.nonzero(got != exp)[0]
            assert bad.size == 0, (f"K={k} gemv {i} slot {t}: {bad.size}/{n} rows differ, "
                                   f"first row {bad[0]}: {got[bad[0]]:#06x} vs {exp[bad[0]]:#06x}")


@pytest.mark.parametrize("k,n", [(896, 4864), (64, 5), (1024, 33), (2048, 130)])
def test_rms_norm_gate_up_silu_bf16(dec, dev, k, n):
    rng = rc.philox(1200 + k)
    # integers / 1024 keep |gate| well inside expf's range
    (wg, dg), (wu, du) = bf16_rows(rng, n, k, 1024.0), bf16_rows(rng, n, k, 1024.0)
    dwg, dwu = to_dev(wg, dev), to_dev(wu, dev)
    ambiguous = 0
    for t in (range(16) if n == 4864 else (0, 9)):
        xw, nw, xn = norm_input(k, t, rng)
        g = bf16(exact_dot(dg, xn, grid_bits=10))
        u = bf16(exact_dot(du, xn, grid_bits=10))
        a, b = silu_mul_expected(g, u)
        out = bf16_out((n,), dev)
        dec.rms_norm_gate_up_silu_bf16(to_dev(xw, dev), to_dev(nw, dev), EPS, k, dwg, dwu, out, n)
        got = words(out)
        ok = (got == a) | (got == b)
        assert ok.all(), (f"K={k} slot {t}: {np.sum(~ok)} rows differ, first "
                          f"{np.nonzero(~ok)[0][0]}")
        ambiguous += int(np.sum(a != b))
    assert ambiguous <= max(2, n // 100), ambiguous


@pytest.mark.parametrize("k,n", [(4864, 896), (64, 3), (896, 897), (512, 4), (576, 65),
                                 (4096, 33), (5120, 7)])
@pytest.mark.parametrize("bias", ["none", "separate", "residual"])
def test_gemv_bf16_rows_bit_exact(dec, dev, k, n, bias):
    rng = rc.philox(1300 + k + n)
    w, deq = bf16_rows(rng, n, k)
    dw = to_dev(w, dev)
    b = dyadic_bias(rng, n) if bias != "none" else None
    for t in ((0, 3, 8, 15) if k == 4864 else (0, 11)):
        pos = sparse_positions(k, t)
        xv = np.zeros(k, np.float64)
        xv[pos] = rng.choice([-2.0, -1.0, 1.0, 2.0], size=pos.size)
        y = bf16_out((n,), dev)
        if bias == "residual":
            y.copy_(to_dev(b, dev))   # the output holds the residual and is updated in place
            dec.gemv_bf16_rows(dw, y, to_dev(bf16(xv), dev), y, n, k)
        else:
            dec.gemv_bf16_rows(dw, to_dev(b, dev) if b is not None else None,
                               to_dev(bf16(xv), dev), y, n, k)
        exp = bf16(exact_dot(deq, xv, b))
        got = words(y)
        bad = np.nonzero(got != exp)[0]
        assert bad.size == 0, (f"K={k} n={n} slot {t}: {bad.size} rows differ, first {bad[0]}: "
                               f"{got[bad[0]]:#06x} vs {exp[bad[0]]:#06x}")


@pytest.mark.parametrize("shape", QKV_ROPE_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_rms_norm_qkv_rope_bf16(dec, dev, shape):
    import torch
    k, heads, kvh, hd, max_seq = shape
    half = hd // 2
    rng = rc.philox(1400 + k + heads)
    nq, nkv = heads * hd, kvh * hd
    w = {n: bf16_rows(rng, m, k) for n, m in (("q", nq), ("k", nkv), ("v", nkv))}
    b = {n: dyadic_bias(rng, w[n][0].shape[0]) for n in "qkv"}
    b["k"] = None  # a null bias too
    dw = {n: (to_dev(w[n][0], dev), to_dev(b[n], dev) if b[n] is not None else None)
          for n in "qkv"}
    sentinel = np.uint16(0x7FC0)
    for position in (0, 5, max_seq - 1, max_seq + 100):
        p = min(position, max_seq - 1)
        xw, nw, xn = norm_input(k, (3 * position) % 16, rng)
        y = {n: bf16(exact_dot(w[n][1], xn, b[n])) for n in "qkv"}
        cs = dec.rope_row(1e6, hd, p)
        kc = torch.full((kvh * max_seq * hd,), int(sentinel.view(np.int16)), dtype=torch.int16,
                        device=dev)
        vc = kc.clone()
        q_out = bf16_out((nq,), dev)
        dpos = torch.tensor([position], dtype=torch.int32, device=dev)
        dec.rms_norm_qkv_rope_bf16(to_dev(xw, dev), to_dev(nw, dev), EPS, k, dw["q"], dw["k"],
                                   dw["v"], q_out, kc, vc, torch.from_numpy(cs.copy()).to(dev),
                                   dpos, heads, kvh, hd, max_seq)
        kcache = kc.cpu().numpy().view(np.uint16).reshape(kvh, max_seq, hd)
        vcache = vc.cpu().numpy().view(np.uint16).reshape(kvh, max_seq, hd)
        other = np.ones(max_seq, bool)
        other[p] = False
        assert np.all(kcache[:, other] == sentinel) and np.all(vcache[:, other] == sentinel)
        np.testing.assert_array_equal(vcache[:, p].reshape(-1), y["v"])
        for name, got in (("q", words(q_out).reshape(-1, hd)), ("k", kcache[:, p])):
            yy = y[name].reshape(-1, hd)
            if p == 0:
                np.testing.assert_array_equal(got, yy)
                continue
            first, second = rope_candidates(yy[:, :half], yy[:, half:], cs)
            ok1 = np.any([got[:, :half] == c for c in first], axis=0)
            ok2 = np.any([got[:, half:] == c for c in second], axis=0)
            assert ok1.all() and ok2.all(), (name, position, np.argwhere(~ok1)[:3],
                                             np.argwhere(~ok2)[:3])


@pytest.mark.parametrize("parts", [2, 4])
@pytest.mark.parametrize("heads,n", [(14, 896), (2, 130), (32, 65)])
def test_attention_halves_o_proj_bf16_bit_exact(dec, dev, heads, n, parts):
    """As test_attention_halves_o_proj_bit_exact on a BF16 weight: lane
    chunks of 8 inputs, eight per head, each reading two 16-byte pieces of
    every part's record.  32 heads is the format's K limit (2048)."""
    import torch
    hd, max_seq, R = 64, 1024, dec.PART_RECORD
    rng = rc.philox(1500 + heads + n + parts)
    k = heads * hd
    w, deq = bf16_rows(rng, n, k)
    dw = to_dev(w, dev)
    x0 = rc.bf16_normal(rng, (n,))
    for pos in PART_O_POSITIONS:
        part, attn = exact_part_records(rng, heads, parts, pos, max_seq, hd, R)
        terms = deq * attn[None, :]
        assert np.all(np.abs(terms).sum(axis=1) * 2 ** 10 < 2 ** 24), "design not exact"
        exp = rc.bf16_words(terms.sum(axis=1).astype(np.float32) + rc.bf16_values(x0))
        x = to_dev(x0, dev)
        dpos = torch.tensor([pos], dtype=torch.int32, device=dev)
        rec = torch.from_numpy(part.reshape(-1)).to(dev)
        if parts == 2:
            dec.attention_halves_o_proj_bf16(rec, dpos, heads, max_seq, dw, x, n)
        else:
            dec.attention_parts_o_proj_bf16(rec, dpos, heads, max_seq, parts, dw, x, n)
        got = words(x)
        bad = np.nonzero(got != exp)[0]
        assert bad.size == 0, f"pos {pos}: {bad.size}/{n} rows differ, first {bad[0]}"
