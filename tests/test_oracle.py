"""Pins the CPU oracle (oracle/vai_oracle.c) before anything is compared to it.

Every check is independent of the oracle's own formulas: numpy's IEEE
float16, float64 closed forms written differently (einsum, explicit padding,
np.triu masks), brute-force bounds on fp32 accumulation error, and shapes
chosen so a transposed operand, a wrong bias/residual index, a swapped
residual order or a dropped scale fails.
"""
import math

import numpy as np
import pytest

from oracle import oracle

EPS32 = np.finfo(np.float32).eps


# ---- fp16 conversion: /root/reference/vai/engine/tensor.cpp:42-90 ----------

def test_half_to_float_all_codes():
    codes = np.arange(65536, dtype=np.uint16)
    got = oracle.from_f16(codes.view(np.float16))
    want = codes.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_float_to_half_normal_range_is_ieee_rne():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(1 << 18) * np.exp(rng.uniform(-9, 10, 1 << 18))).astype(np.float32)
    x = x[(np.abs(x) >= 6.104e-5) & (np.abs(x) < 65504)]
    # ties: exact midpoints between neighbouring halves round to even
    h = np.arange(0x0400, 0x7BFF, 7, dtype=np.uint16).view(np.float16).astype(np.float32)
    mid = (h + np.nextafter(h.astype(np.float16), np.float16(np.inf)).astype(np.float32)) / 2
    for v in (x, mid, -mid):
        assert np.array_equal(oracle.to_f16(v).view(np.uint16), v.astype(np.float16).view(np.uint16))


def test_float_to_half_flushes_subnormals_and_saturates():
    tiny = np.array([6.0e-5, 1e-7, -3e-6, 5.96e-8], np.float32)
    assert np.array_equal(oracle.to_f16(tiny).view(np.uint16), np.array([0, 0, 0x8000, 0], np.uint16))
    big = np.array([65520.0, 1e6, -1e9, np.inf], np.float32)
    assert np.array_equal(oracle.to_f16(big).view(np.uint16), np.array([0x7C00, 0x7C00, 0xFC00, 0x7C00], np.uint16))
    assert np.isnan(oracle.to_f16(np.array([np.nan], np.float32))).all()
    assert oracle.to_f16(np.array([65504.0], np.float32)).view(np.uint16)[0] == 0x7BFF


# ---- epilogues: /root/reference/vai/shaders/common/activation.h:19-58 -------

X = np.concatenate([np.linspace(-12, 12, 2001), [0.0, 1e-3, -1e-3, 3.0, -3.0]]).astype(np.float32)


def _closed(epi, x):
    x = x.astype(np.float64)
    erf = np.vectorize(math.erf)
    return {
        "NONE": x,
        "RELU": np.maximum(x, 0),
        "GELU": 0.5 * x * (1 + erf(x / math.sqrt(2))),
        "GELU_TANH": 0.5 * x * (1 + np.tanh(math.sqrt(2 / math.pi) * (x + 0.044715 * x ** 3))),
        "SILU": x / (1 + np.exp(-x)),
        "SIGMOID": 1 / (1 + np.exp(-x)),
    }[epi]


@pytest.mark.parametrize("epi", list(oracle.EPILOGUES))
def test_epilogue_closed_forms(epi):
    got = oracle.epilogue(X, epi).astype(np.float64)
    want = _closed(epi, X)
    # A&S 7.1.26 is within 1.5e-7 of erf; the rest is fp32 rounding.
    err = np.abs(got - want)
    assert (err <= 2e-6 * np.abs(want) + 2e-7 * (1 + np.abs(X))).all(), float(err.max())


def test_epilogue_special_points():
    z = np.zeros(1, np.float32)
    for epi in ("RELU", "GELU", "GELU_TANH", "SILU"):
        assert oracle.epilogue(z, epi)[0] == 0.0
    assert oracle.epilogue(z, "SIGMOID")[0] == 0.5
    assert oracle.epilogue(np.array([-5.0], np.float32), "RELU")[0] == 0.0
    # GELU(x) -> x for large x, -> 0 for very negative x
    assert abs(oracle.epilogue(np.array([8.0], np.float32), "GELU")[0] - 8.0) < 1e-6
    assert abs(oracle.epilogue(np.array([-8.0], np.float32), "GELU_TANH")[0]) < 1e-6


# ---- Linear -----------------------------------------------------------------

def _bound(x, w):
    """|fp32 dot - exact| <= gamma_K * sum |x w| (Higham), plus operand rounding."""
    k = x.shape[-1]
    return 1.01 * k * EPS32 * (np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T) + 1e-30


@pytest.mark.parametrize("m, k, n", [(1, 7, 5), (3, 64, 9), (12, 33, 17), (40, 130, 3)])
@pytest.mark.parametrize("idt, wdt", [(np.float32, np.float32), (np.float16, np.float16),
                                      (np.float32, np.float16)])
def test_linear_plain_vs_float64(m, k, n, idt, wdt):
    rng = np.random.default_rng(m * 1000 + k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = rng.standard_normal((n, k)).astype(np.float32)
    x16, w16 = x.astype(idt), w.astype(wdt)
    for stage in ("slab", "tile"):
        got = oracle.linear(x16, w16, stage=stage).astype(np.float64)
        xs, ws = x16.astype(np.float32), w16.astype(np.float32)
        if stage == "tile" and not (idt == np.float32 and wdt == np.float32):
            xs, ws = xs.astype(np.float16).astype(np.float32), ws.astype(np.float16).astype(np.float32)
        exact = xs.astype(np.float64) @ ws.astype(np.float64).T
        assert (np.abs(got - exact) <= _bound(xs, ws)).all(), stage
    if idt != wdt:   # the tile contract really rounds the fp32 side: the results differ
        assert not np.array_equal(oracle.linear(x16, w16, stage="slab"), oracle.linear(x16, w16, stage="tile"))


def test_linear_bias_residual_scale_orders():
    rng = np.random.default_rng(3)
    m, k, n = 6, 20, 10
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = rng.standard_normal((n, k)).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    r = rng.standard_normal((m, n)).astype(np.float32)
    y = x.astype(np.float64) @ w.astype(np.float64).T + b
    tol = dict(rtol=1e-5, atol=1e-5)
    after = oracle.linear(x, w, b, r, epi="RELU", order=0, scale=0.5)
    before = oracle.linear(x, w, b, r, epi="RELU", order=1, scale=0.5)
    np.testing.assert_allclose(after, 0.5 * np.maximum(y, 0) + r, **tol)
    np.testing.assert_allclose(before, 0.5 * np.maximum(y + r, 0), **tol)
    assert not np.allclose(after, before)
    # bias [M,N] vs [N] repeating; residual repeating rows
    bfull = np.tile(b, (m, 1))
    np.testing.assert_array_equal(oracle.linear(x, w, bfull), oracle.linear(x, w, b))
    rrow = r[0].copy()
    np.testing.assert_allclose(oracle.linear(x, w, None, rrow), y - b + rrow, **tol)


def test_linear_split_matches_reduce():
    rng = np.random.default_rng(4)
    m, k, n, span = 9, 100, 7, 32
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = rng.standard_normal((n, k)).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    parts = np.stack([oracle.linear(x[:, s:s + span], w[:, s:s + span], stage="tile")
                      for s in range(0, k, span)])
    red = oracle.linear_reduce(parts, b, epi="GELU")
    direct = oracle.linear(x, w, b, epi="GELU", stage="tile", split_size=span)
    np.testing.assert_array_equal(red, direct)
    exact = oracle.epilogue((x.astype(np.float64) @ w.astype(np.float64).T + b).astype(np.float32), "GELU")
    np.testing.assert_allclose(direct, exact, rtol=1e-5, atol=1e-5)


def test_gated_mul_closed_form():
    rng = np.random.default_rng(5)
    y = rng.standard_normal((4, 2 * 11)).astype(np.float32)
    g, u = y[:, :11].astype(np.float64), y[:, 11:].astype(np.float64)
    np.testing.assert_allclose(oracle.gated_mul(y, epi="SILU"), g / (1 + np.exp(-g)) * u, rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(oracle.gated_mul(y, epi="NONE"), g * u, rtol=1e-6, atol=1e-7)


# ---- Convolution ------------------------------------------------------------

def _conv_ref(x, w, stride):
    """float64 cross-correlation through explicit zero padding and einsum."""
    x = x.astype(np.float64)
    w = w.astype(np.float64)
    co, ci, k, _ = w.shape
    p = k // 2
    xp = np.pad(x, [(0, 0)] * (x.ndim - 2) + [(p, p), (p, p)])
    hi, wi = x.shape[-2:]
    ho, wo = (hi - 1) // stride + 1, (wi - 1) // stride + 1
    out = np.zeros(x.shape[:-3] + (co, ho, wo))
    for kh in range(k):
        for kw in range(k):
            patch = xp[..., kh:kh + stride * (ho - 1) + 1:stride, kw:kw + stride * (wo - 1) + 1:stride]
            out += np.einsum("oc,...chw->...ohw", w[:, :, kh, kw], patch)
    return out


@pytest.mark.parametrize("ci, co, k, s, h, w_, batch", [
    (3, 4, 3, 1, 7, 9, 1), (5, 2, 1, 1, 4, 4, 2), (2, 3, 5, 2, 9, 6, 1), (4, 4, 3, 2, 8, 8, 3), (1, 1, 3, 1, 1, 1, 1)])
def test_conv_vs_float64(ci, co, k, s, h, w_, batch):
    rng = np.random.default_rng(ci * 7 + k)
    x = rng.standard_normal((batch, ci, h, w_)).astype(np.float32)
    w = rng.standard_normal((co, ci, k, k)).astype(np.float32)
    b = rng.standard_normal(co).astype(np.float32)
    got = oracle.conv2d(x, w, b, stride=s).astype(np.float64)
    want = _conv_ref(x, w, s) + b[:, None, None]
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)


def test_conv_scale_residual_and_fp16_staging():
    rng = np.random.default_rng(9)
    x = rng.standard_normal((1, 3, 6, 6)).astype(np.float32)
    w = rng.standard_normal((4, 3, 3, 3)).astype(np.float32)
    b = rng.standard_normal(4).astype(np.float32)
    sc = rng.uniform(0.5, 2, 4).astype(np.float32)
    r = rng.standard_normal((1, 4, 6, 6)).astype(np.float32)
    base = _conv_ref(x, w, 1) * sc[:, None, None] + b[:, None, None]
    np.testing.assert_allclose(oracle.conv2d(x, w, b, sc, r, epi="RELU", order=0), np.maximum(base, 0) + r,
                               rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(oracle.conv2d(x, w, b, sc, r, epi="RELU", order=1), np.maximum(base + r, 0),
                               rtol=1e-5, atol=1e-5)
    # fp16 weights stage the fp32 input as fp16 (conv-k3s1-implicit-gemm.comp writeB)
    w16 = w.astype(np.float16)
    got = oracle.conv2d(x, w16).astype(np.float64)
    want = _conv_ref(x.astype(np.float16), w16, 1)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)


# ---- Attention scores -------------------------------------------------------

@pytest.mark.parametrize("hq, hkv, tq, tkv, d, causal, span", [
    (2, 2, 9, 9, 8, True, 0), (4, 2, 5, 12, 16, True, 0), (2, 1, 10, 10, 4, True, 3), (1, 1, 6, 4, 8, False, 0)])
def test_scores_vs_float64(hq, hkv, tq, tkv, d, causal, span):
    rng = np.random.default_rng(hq + tq)
    q = rng.standard_normal((hq, tq, d)).astype(np.float32)
    k = rng.standard_normal((hkv, tkv, d)).astype(np.float32)
    got = oracle.attn_scores(q, k, scale=0.25, causal=causal, span=span)
    kk = np.repeat(k.astype(np.float64), hq // hkv, axis=0)
    s = np.einsum("hid,hjd->hij", q.astype(np.float64), kk) * 0.25
    off = tkv - tq
    hide = np.zeros((tq, tkv), bool)
    if causal:
        hide |= np.triu(np.ones((tq, tkv), bool), k=off + 1)
    if span:
        pos = np.arange(tq)[:, None] + off
        j = np.arange(tkv)[None, :]
        hide |= (pos >= span) & (j < pos + 1 - span)
    s[:, hide] = -np.inf
    assert np.array_equal(np.isneginf(got), np.isneginf(s))
    fin = ~np.isneginf(s)
    np.testing.assert_allclose(got[fin], s[fin], rtol=1e-5, atol=1e-5)


def _attn_inputs(rng, hq, hkv, tq, tkv, d):
    q = rng.standard_normal((1, hq, tq, d)).astype(np.float16)
    k = rng.standard_normal((1, hkv, tkv, d)).astype(np.float16)
    v = rng.standard_normal((1, hkv, tkv, d)).astype(np.float16)
    return q, k, v


def _np_attention_head_major(q, k, v, scale):
    """float64 softmax(q k^T scale) v per head with no mask, head-major
    [B, Hq, Tq, D], written with numpy alone (no oracle code)."""
    q, k, v = (np.asarray(t, np.float64) for t in (q, k, v))
    g = q.shape[1] // k.shape[1]
    k, v = np.repeat(k, g, axis=1), np.repeat(v, g, axis=1)
    s = np.einsum("bhid,bhjd->bhij", q, k) * scale
    p = np.exp(s - s.max(-1, keepdims=True))
    return np.einsum("bhij,bhjd->bhid", p / p.sum(-1, keepdims=True), v)


def test_attention_oracle_pins():
    """oracle.attention composes the pinned scores with softmax and P.V;
    these properties fail for a dropped normalisation, a reversed mask or a
    transposed V. O is token-major: o[b, i, h] is query i of head h."""
    rng = np.random.default_rng(0)
    q, k, v = _attn_inputs(rng, 2, 1, 5, 7, 8)
    # V of ones: every row with a visible key returns exactly 1
    o = oracle.attention(q, k, np.ones_like(v), causal=True, out_dtype=np.float64)
    np.testing.assert_allclose(o, 1.0, rtol=1e-12)
    # V = identity rows (Tkv = D): O is the softmax matrix itself
    q2, k2, _ = _attn_inputs(rng, 1, 1, 6, 8, 8)
    eye = np.eye(8, dtype=np.float16)[None, None]
    o = oracle.attention(q2, k2, eye, causal=False, out_dtype=np.float64)[0, :, 0]
    s = q2[0, 0].astype(np.float64) @ k2[0, 0].astype(np.float64).T / np.sqrt(8)
    p = np.exp(s - s.max(1, keepdims=True))
    np.testing.assert_allclose(o, p / p.sum(1, keepdims=True), rtol=1e-6)
    # causal with Tq = Tkv: query 0 sees key 0 alone, so O[0] = V[0]; the
    # last query sees every key
    q3, k3, v3 = _attn_inputs(rng, 1, 1, 6, 6, 8)
    o = oracle.attention(q3, k3, v3, causal=True, out_dtype=np.float64)[0, :, 0]
    np.testing.assert_array_equal(o[0], v3[0, 0, 0].astype(np.float64))
    full = oracle.attention(q3, k3, v3, causal=False, out_dtype=np.float64)[0, :, 0]
    np.testing.assert_allclose(o[-1], full[-1], rtol=1e-12)
    # GQA: two query heads over one K/V head equal two single-head calls
    qa, kb, vb = _attn_inputs(rng, 2, 1, 4, 4, 8)
    both = oracle.attention(qa, kb, vb, causal=True, out_dtype=np.float64)
    for h in range(2):
        one = oracle.attention(qa[:, h:h + 1], kb, vb, causal=True, out_dtype=np.float64)
        np.testing.assert_allclose(both[:, :, h:h + 1], one, rtol=1e-12)
    # Tq > Tkv under the causal rule: the first queries see no key and give 0
    q4, k4, v4 = _attn_inputs(rng, 1, 1, 5, 3, 8)
    o = oracle.attention(q4, k4, v4, causal=True, out_dtype=np.float64)[0, :, 0]
    np.testing.assert_array_equal(o[:2], 0.0)


def test_attention_oracle_layout_and_defaults():
    """The reference's contract (attention.h:77-79,129; attention-fa.comp:96):
    out0 is [B, Tq, Hq, D] -- the independent head-major float64 result
    transposed by numpy -- and no mask applies unless one is asked for.
    Distinct Tq, Hq and D (and Hq != Hkv) make a wrong axis order fail."""
    rng = np.random.default_rng(11)
    q, k, v = _attn_inputs(rng, 4, 2, 5, 9, 24)
    want = np.transpose(_np_attention_head_major(q, k, v, 1 / np.sqrt(24)), (0, 2, 1, 3))
    got = oracle.attention(q, k, v, out_dtype=np.float64)
    assert got.shape == (1, 5, 4, 24)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)
    causal = oracle.attention(q, k, v, causal=True, out_dtype=np.float64)
    assert not np.allclose(causal, got)
    # fp32 Q with fp16 K / V (the reference's typeI / typeKV, attention.h:86-88)
    q32 = rng.standard_normal(q.shape).astype(np.float32)
    got = oracle.attention(q32, k, v, out_dtype=np.float64)
    want = np.transpose(_np_attention_head_major(q32, k, v, 1 / np.sqrt(24)), (0, 2, 1, 3))
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)
    # fp32 everything, head dim 72 (SigLIP's, /root/reference/models/common.h:30)
    q, k, v = (rng.standard_normal((2, 3, 7, 72)).astype(np.float32) for _ in range(3))
    got = oracle.attention(q, k, v, out_dtype=np.float64)
    want = np.transpose(_np_attention_head_major(q, k, v, 1 / np.sqrt(72)), (0, 2, 1, 3))
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)


# ---- fp16 accumulation (Linear::setAccDtype(Fp16), linear-tile.comp:292-320) --

def _round_half_exact(fr):
    """An exact rational rounded to fp16 (IEEE RNE, subnormals, overflow -> inf),
    written independently of the oracle's double-based rounding."""
    from fractions import Fraction
    if fr == 0:
        return np.float16(0.0)
    sign = -1 if fr < 0 else 1
    a = abs(fr)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    quantum = Fraction(2) ** (max(e, -14) - 10)
    n = round(a / quantum)            # Fraction rounding: ties to even
    v = n * quantum
    if v >= 65536:
        return np.float16(sign * np.inf)
    return np.float16(sign * float(v))


def _fma16_exact(a, b, c):
    from fractions import Fraction
    return _round_half_exact(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def test_fma16_against_exact_rationals():
    rng = np.random.default_rng(11)
    a = rng.standard_normal(3000).astype(np.float16)
    b = (rng.standard_normal(3000) * np.exp2(rng.integers(-12, 8, 3000))).astype(np.float16)
    c = (rng.standard_normal(3000) * np.exp2(rng.integers(-20, 12, 3000))).astype(np.float16)
    got = oracle.fma16(a, b, c)
    want = np.array([_fma16_exact(x, y, z) for x, y, z in zip(a, b, c)], np.float16)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
    h = np.float16
    # one rounding, not two: (1 + 2^-10)(1 - 2^-10) - 1 = -2^-20 (a subnormal half)
    assert oracle.fma16([h(1 + 2 ** -10)], [h(1 - 2 ** -10)], [h(-1)])[0] == h(-(2.0 ** -20))
    # ties to even: 1 + 2^-11 -> 1, (1 + 2^-10) + 2^-11 -> 1 + 2^-9
    assert oracle.fma16([h(2 ** -6)], [h(2 ** -5)], [h(1)])[0] == h(1)
    assert oracle.fma16([h(2 ** -6)], [h(2 ** -5)], [h(1 + 2 ** -10)])[0] == h(1 + 2 ** -9)
    # overflow: 65504 + 16 is a tie that rounds to inf; 65504 + 15 stays
    assert np.isposinf(oracle.fma16([h(16)], [h(1)], [h(65504)])[0])
    assert oracle.fma16([h(15)], [h(1)], [h(65504)])[0] == h(65504)


def _acc16_brute(x, w, split):
    """The fma chain of linear-tile.comp, by exact rationals, tiny shapes only."""
    M, K = x.shape
    N = w.shape[0]
    x16, w16 = x.astype(np.float16), w.astype(np.float16)
    out = np.zeros((M, N), np.float32)
    for m in range(M):
        for n in range(N):
            tot = np.float32(0)
            for k0 in range(0, K, split):
                k1 = min(K, k0 + split)
                s = np.float16(0)
                for k in range(k0, k1, 4):
                    for q in (3, 2, 1, 0):
                        kk = k + q
                        s = _fma16_exact(x16[m, kk] if kk < k1 else 0, w16[n, kk] if kk < k1 else 0, s)
                s = np.float32(min(max(float(s), -65504.0), 65504.0))
                tot = np.float32(tot + s)
            out[m, n] = tot
    return out


@pytest.mark.parametrize("k, split", [(9, 9), (13, 8), (32, 32), (40, 12)])
def test_linear_acc16_brute_force(k, split):
    rng = np.random.default_rng(k)
    x = rng.standard_normal((3, k)).astype(np.float16)
    w = (rng.standard_normal((4, k)) * 3).astype(np.float16)
    got = oracle.linear_acc16(x, w, split_size=split)
    assert np.array_equal(got, _acc16_brute(x, w, split))


def test_linear_acc16_order_clamp_and_error_bound():
    h = np.float16
    # within a 4-step k+3 comes first: -2048 + 1 + 1 + 2048 = 2 (ascending order would give 0)
    x = np.ones((1, 4), h)
    assert oracle.linear_acc16(x, np.array([[2048, 1, 1, -2048]], h))[0, 0] == 2.0
    # the 4-steps go up in k: 2048 first, then +1 +1 at 2048's spacing of 2 stay 2048
    x = np.ones((1, 8), h)
    w = np.array([[0, 0, 0, 2048, 1, 1, 0, 0]], h)
    assert oracle.linear_acc16(x, w)[0, 0] == 2048.0
    # overflowing sums clamp to +-65504, then the fp32 bias is added
    x = np.full((2, 8), 100, h)
    w = np.array([np.full(8, 100), np.full(8, -100)], h)
    got = oracle.linear_acc16(x, w, np.array([0.5, -0.5], np.float32))
    assert (got == np.array([65504.5, -65504.5], np.float32)).all()
    # random data: within the fp16 accumulation bound of the float64 result
    rng = np.random.default_rng(5)
    x = rng.standard_normal((20, 300)).astype(h)
    w = (rng.standard_normal((30, 300)) * 0.1).astype(h)
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    mag = np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    err = np.abs(oracle.linear_acc16(x, w) - exact)
    assert (err <= 300 * 2.0 ** -11 * mag).all()
    assert err.max() > 10 * np.abs(oracle.linear(x, w, stage="tile") - exact).max()   # really fp16 sums


# ---- block masks (writeCausalMask, attention.h:40-55; causal_mask.h:25-38) ----

def _visible_literal(rows):
    """Rows of the visibility matrix written out by hand: a list of key ends
    (exclusive) per query, from key 0 (no span)."""
    tkv = max(rows)
    return np.array([[j < e for j in range(tkv)] for e in rows])


@pytest.mark.parametrize("tq, tkv, blocks, ends_per_row", [
    # prefix-LM: rows 0-3 read the whole 4-token prefix, then causal
    (10, 10, (0b01, [4]), [4, 4, 4, 4, 5, 6, 7, 8, 9, 10]),
    # causal / full / causal with ends 3 and 7
    (10, 10, (0b101, [3, 7]), [1, 2, 3, 7, 7, 7, 7, 8, 9, 10]),
    # full / causal / full
    (9, 9, (0b010, [2, 5]), [2, 2, 3, 4, 5, 9, 9, 9, 9]),
    # fewer queries than keys: queries sit at the keys' end (offset 6)
    (4, 10, (0b01, [2]), [8, 8, 9, 10]),
    # one causal block is the plain causal mask; ends past Tq are clipped
    (6, 6, (0b1, []), [1, 2, 3, 4, 5, 6]),
    (6, 6, (0b01, [20]), [6, 6, 6, 6, 6, 6]),
    (6, 6, (0b10, [20]), [1, 2, 3, 4, 5, 6]),
])
def test_scores_block_masks(tq, tkv, blocks, ends_per_row):
    rng = np.random.default_rng(tq + tkv)
    q = rng.standard_normal((2, tq, 8)).astype(np.float16)
    k = rng.standard_normal((2, tkv, 8)).astype(np.float16)
    got = oracle.attn_scores(q, k, scale=0.5, blocks=blocks)
    vis = _visible_literal(ends_per_row)
    assert vis.shape == (tq, tkv)
    assert np.array_equal(np.isfinite(got), np.broadcast_to(vis, got.shape))
    want = np.einsum("hid,hjd->hij", q.astype(np.float64), k.astype(np.float64)) * 0.5
    np.testing.assert_allclose(got[:, vis], want[:, vis], rtol=1e-5, atol=1e-5)
    if blocks == (0b1, []):
        assert np.array_equal(got, oracle.attn_scores(q, k, scale=0.5, causal=True))
    # a span still cuts from below
    got = oracle.attn_scores(q, k, scale=0.5, blocks=blocks, span=2)
    pos = np.arange(tq) + tkv - tq
    lo = np.where(pos >= 2, pos - 1, 0)
    vis2 = vis & (np.arange(tkv)[None, :] >= lo[:, None])
    assert np.array_equal(np.isfinite(got[0]), vis2)


def test_acc16_nan_chain_stays_nan():
    """The fp16 accumulator's clamp to +-65504 keeps a NaN sum NaN (GLSL
    leaves clamp of a NaN undefined; a finite clamp would hide the fault), and
    still clamps an overflowed chain: a row that overflows to +inf and then
    meets -inf gives NaN, a row that only overflows gives 65504."""
    x = np.zeros((2, 8), np.float16)
    w = np.zeros((1, 8), np.float16)
    w[0, :] = 1
    x[0, 0], x[0, 4] = 60000, np.float16(np.inf)     # an overflowing chain ...
    x[0, 1] = -np.float16(np.inf)                     # ... meets -inf: NaN
    x[1, :2] = 60000                                  # 120000 overflows to +inf: clamped
    out = oracle.linear_acc16(x, w)
    assert np.isnan(out[0, 0])
    assert out[1, 0] == 65504.0


# ---- the KV-cache restatement (oracle.attention_cached) against the plain
# attention oracle where the reference's formulas reduce to it ----

def _cache_case(rng, hkv, size, d, positions, dtype=np.float32):
    """A cache plane pair holding the given positions' rows of a key history."""
    kc = np.full((hkv, size, d), np.nan, dtype)
    return kc, kc.copy()


def test_attention_cached_empty_cache_is_plain_attention():
    """count = 0: keyEnd and keyPos are the plain end-aligned rule, whatever
    Tq and Tkv are (attention-fa.comp:137-146)."""
    rng = np.random.default_rng(11)
    for tq, tkv, causal, span in [(5, 5, True, 0), (3, 7, True, 0), (7, 3, True, 0), (4, 4, False, 0), (6, 6, True, 3)]:
        q = rng.standard_normal((4, tq, 16)).astype(np.float32)
        k = rng.standard_normal((2, tkv, 16)).astype(np.float32)
        v = rng.standard_normal((2, tkv, 16)).astype(np.float32)
        kc, vc = _cache_case(rng, 2, 32, 16, [])
        got, kc2, vc2 = oracle.attention_cached(q, k, v, kc, vc, 0, causal=causal, span=span)
        np.testing.assert_allclose(got, oracle.attention(q, k, v, causal=causal, span=span), rtol=1e-6, atol=1e-6)
        assert np.array_equal(kc2[:, :tkv], k) and np.array_equal(vc2[:, :tkv], v)
        assert np.isnan(kc2[:, tkv:]).all()   # rows past the append untouched


def test_attention_cached_is_attention_over_the_key_history():
    """Tq <= Tkv: query t sits at count + t + Tkv - Tq, the end alignment of
    plain attention over the count + Tkv keys of the whole history."""
    rng = np.random.default_rng(12)
    for tq, tkv, count, causal, span in [(2, 3, 10, True, 0), (1, 1, 20, True, 0), (4, 4, 7, False, 0),
                                         (3, 3, 9, True, 5)]:
        hk = rng.standard_normal((2, count + tkv, 16)).astype(np.float32)
        hv = rng.standard_normal((2, count + tkv, 16)).astype(np.float32)
        kc, vc = _cache_case(rng, 2, 32, 16, [])
        kc[:, :count], vc[:, :count] = hk[:, :count], hv[:, :count]
        q = rng.standard_normal((4, tq, 16)).astype(np.float32)
        got, kc2, _ = oracle.attention_cached(q, hk[:, count:], hv[:, count:], kc, vc, count, causal=causal, span=span)
        np.testing.assert_allclose(got, oracle.attention(q, hk, hv, causal=causal, span=span), rtol=1e-6, atol=1e-6)
        assert np.array_equal(kc2[:, :count + tkv], hk)


def test_attention_cached_ring_is_the_windowed_history():
    """A ring of 16 rows holding the last 16 positions (row p % 16) under an
    8-key window gives what plain windowed attention over the whole history
    gives."""
    rng = np.random.default_rng(13)
    size, count, tkv, tq, span = 16, 37, 2, 2, 8
    hk = rng.standard_normal((2, count + tkv, 16)).astype(np.float32)
    hv = rng.standard_normal((2, count + tkv, 16)).astype(np.float32)
    kc, vc = _cache_case(rng, 2, size, 16, [])
    for p in range(count - size, count):
        kc[:, p % size], vc[:, p % size] = hk[:, p], hv[:, p]
    q = rng.standard_normal((4, tq, 16)).astype(np.float32)
    got, kc2, _ = oracle.attention_cached(q, hk[:, count:], hv[:, count:], kc, vc, count, ring=True, causal=True,
                                          span=span)
    np.testing.assert_allclose(got, oracle.attention(q, hk, hv, causal=True, span=span), rtol=1e-6, atol=1e-6)
    assert np.array_equal(kc2[:, count % size], hk[:, count])


def test_attention_cached_without_new_keys_reads_the_cache():
    """Tkv = 0: every query sits past the last cached key and reads them all."""
    rng = np.random.default_rng(14)
    kc = rng.standard_normal((2, 16, 16)).astype(np.float32)
    vc = rng.standard_normal((2, 16, 16)).astype(np.float32)
    q = rng.standard_normal((4, 3, 16)).astype(np.float32)
    got, _, _ = oracle.attention_cached(q, None, None, kc, vc, 9, causal=True)
    np.testing.assert_allclose(got, oracle.attention(q, kc[:, :9], vc[:, :9]), rtol=1e-6, atol=1e-6)
