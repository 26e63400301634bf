"""Pins of the CPU baseline (oracle/cpu_baseline.c) and of orc_gemm_f32, the
CPU code bench.py times beside the GPU kernels: float64 closed forms with the
fp32 accumulation bound |fp32 sum - exact| <= 1.01 K eps sum|a b| (Higham),
at shapes with row, column and K tails so that a dropped tail, a transposed
operand or a wrong gate/up pairing fails."""
import numpy as np
import pytest

from helpers import np_epilogue
from oracle import oracle

EPS32 = np.finfo(np.float32).eps


def _exact_and_bound(x, w, b=None):
    xf, wf = np.asarray(x, np.float64), np.asarray(w, np.float64)
    y = xf @ wf.T + (0 if b is None else np.asarray(b, np.float64))
    bound = 1.01 * (x.shape[-1] + 1) * EPS32 * (np.abs(xf) @ np.abs(wf).T + (0 if b is None else np.abs(b)))
    return y, bound


@pytest.mark.parametrize("m, k, n", [(1, 40, 7), (3, 2048, 50), (8, 77, 33), (7, 2049, 5)])
def test_orc_gemm_f32_vs_float64(m, k, n):
    rng = np.random.default_rng(m + k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = rng.standard_normal((n, k)).astype(np.float32)
    got = oracle.gemm_f32(x, w).astype(np.float64)
    y, bound = _exact_and_bound(x, w)
    assert (np.abs(got - y) <= bound + 1e-30).all()
    # a transposed use of w would not even have this shape; a dropped k fails
    assert not (np.abs(oracle.gemm_f32(x[:, :-1], w[:, :-1]) - y) <= bound).all()


@pytest.mark.parametrize("m, k, n", [(1, 2048, 100), (4, 2048, 64), (8, 1000, 37), (2, 13, 9),
                                     (130, 768, 101), (65, 1030, 50), (9, 5, 3)])
@pytest.mark.parametrize("dt", [np.float32, np.float16])
def test_cpu_linear_vs_float64(m, k, n, dt):
    rng = np.random.default_rng(m * 7 + k)
    w = (rng.standard_normal((n, k)) * 0.05).astype(dt)
    b = (rng.standard_normal(n) * 0.05).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(dt)
    y, bound = _exact_and_bound(x, w, b)
    got = oracle.cpu_linear(x, w, b).astype(np.float64)
    assert (np.abs(got - y) <= bound).all()
    got = oracle.cpu_linear(x, w, b, epi="GELU_TANH").astype(np.float64)
    np.testing.assert_allclose(got, np_epilogue("GELU_TANH", y), rtol=1e-5, atol=1e-5 + float(bound.max()))


@pytest.mark.parametrize("m, k, h", [(2, 256, 40), (70, 384, 30), (64, 512, 24)])
def test_cpu_linear_gated(m, k, h):
    rng = np.random.default_rng(h)
    w = (rng.standard_normal((2 * h, k)) * 0.05).astype(np.float16)
    x = rng.standard_normal((m, k)).astype(np.float16)
    y, bound = _exact_and_bound(x, w)
    want = np_epilogue("SILU", y[:, :h]) * y[:, h:]
    got = oracle.cpu_linear(x, w, gated=True, gate_epi="SILU").astype(np.float64)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)
    # gate and up swapped gives something else
    assert not np.allclose(got, np_epilogue("SILU", y[:, h:]) * y[:, :h], rtol=1e-3, atol=1e-3)


@pytest.mark.parametrize("ci, co, hw, ks, s", [(16, 24, 11, 3, 1), (8, 5, 9, 3, 2), (32, 16, 6, 1, 1)])
def test_cpu_conv2d_vs_float64(ci, co, hw, ks, s):
    rng = np.random.default_rng(ci + co)
    w = (rng.standard_normal((co, ci, ks, ks)) * 0.1).astype(np.float16)
    b = (rng.standard_normal(co) * 0.1).astype(np.float32)
    x = rng.uniform(-1, 1, (ci, hw, hw + 2)).astype(np.float16)
    p = ks // 2
    xp = np.pad(x.astype(np.float64), ((0, 0), (p, p), (p, p)))
    Ho, Wo = (hw - 1) // s + 1, (hw + 2 - 1) // s + 1
    want = np.zeros((co, Ho, Wo))
    mag = np.zeros((co, Ho, Wo))
    for kh in range(ks):
        for kw in range(ks):
            patch = xp[:, kh:kh + s * (Ho - 1) + 1:s, kw:kw + s * (Wo - 1) + 1:s]
            want += np.einsum("oc,chw->ohw", w[:, :, kh, kw].astype(np.float64), patch)
            mag += np.einsum("oc,chw->ohw", np.abs(w[:, :, kh, kw].astype(np.float64)), np.abs(patch))
    want += b[:, None, None]
    got = oracle.cpu_conv2d(x, w, b, stride=s).astype(np.float64)
    assert got.shape == want.shape
    assert (np.abs(got - want) <= 1.01 * (ci * ks * ks + 1) * EPS32 * (mag + np.abs(b)[:, None, None])).all()
    got = oracle.cpu_conv2d(x, w, b, stride=s, epi="SILU").astype(np.float64)
    np.testing.assert_allclose(got, np_epilogue("SILU", want), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("h, tq, tkv, d, causal", [(2, 100, 100, 64, True), (1, 70, 130, 32, True),
                                                    (3, 65, 33, 48, False)])
def test_cpu_attn_scores_vs_float64(h, tq, tkv, d, causal):
    rng = np.random.default_rng(tq)
    q = rng.standard_normal((h, tq, d)).astype(np.float16)
    k = rng.standard_normal((h, tkv, d)).astype(np.float16)
    got = oracle.cpu_attn_scores(q, k, scale=0.125, causal=causal)
    want = np.einsum("hid,hjd->hij", q.astype(np.float64), k.astype(np.float64)) * 0.125
    i, j = np.indices((tq, tkv))
    hidden = (j > i + (tkv - tq)) if causal else np.zeros((tq, tkv), bool)
    assert np.isneginf(got[:, hidden]).all() and np.isfinite(got[:, ~hidden]).all()
    mag = np.einsum("hid,hjd->hij", np.abs(q.astype(np.float64)), np.abs(k.astype(np.float64))) * 0.125
    assert (np.abs(got[:, ~hidden] - want[:, ~hidden]) <= 1.01 * d * EPS32 * mag[:, ~hidden] + 1e-30).all()


@pytest.mark.parametrize("h, tq, tkv, d, causal", [(2, 100, 100, 64, True), (1, 70, 130, 32, True),
                                                    (2, 130, 60, 16, True), (3, 65, 33, 48, False)])
def test_cpu_attention_vs_float64(h, tq, tkv, d, causal):
    rng = np.random.default_rng(tq + d)
    q = rng.standard_normal((h, tq, d)).astype(np.float16)
    k = rng.standard_normal((h, tkv, d)).astype(np.float16)
    v = rng.standard_normal((h, tkv, d)).astype(np.float16)
    got = oracle.cpu_attention(q, k, v, scale=0.2, causal=causal)
    S = np.einsum("hid,hjd->hij", q.astype(np.float64), k.astype(np.float64)) * 0.2
    i, j = np.indices((tq, tkv))
    if causal:
        S = np.where(j > i + (tkv - tq), -np.inf, S)
    m = S.max(-1, keepdims=True)
    P = np.where(np.isfinite(S), np.exp(S - np.where(np.isfinite(m), m, 0)), 0.0)
    l = P.sum(-1, keepdims=True)
    want = np.where(l > 0, (P @ v.astype(np.float64)) / np.where(l > 0, l, 1), 0.0)
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=2e-5)
    # rows with no visible key (Tq > Tkv) are exactly zero
    if causal and tq > tkv:
        assert (got[:, : tq - tkv] == 0).all()
