"""BASELINE configs against committed golden vectors (tests/golden/).

The golden file holds float64 closed-form outputs on sampled rows plus
checksums over every row (gen_golden.py, numpy only). CPU tests pin the oracle
to them; GPU tests hold the HIP kernels to them at the full config sizes.
"""
import os
import sys

import numpy as np
import pytest

from helpers import FP32, TRANS, assert_close
from oracle import oracle

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
import configs as C  # noqa: E402

G = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "baseline_configs.npz"))


def test_numpy_f16_matches_reference_rounding():
    x = np.random.default_rng(3).standard_normal(1 << 16).astype(np.float32) * np.float32(1e-3)
    assert np.array_equal(C.f16(x).view(np.uint16), oracle.to_f16(x).view(np.uint16))


# ---- the oracle at the config shapes (sampled rows) ----

def test_oracle_cfg1():
    x, w, b = C.cfg1()
    got = oracle.linear(x[C.CFG1_ROWS], w, b, epi="GELU_TANH", stage="tile")
    assert_close(got, G["cfg1_rows"], FP32)


def test_oracle_cfg2():
    x, w = C.cfg2()
    assert_close(oracle.linear(x, w, stage="slab"), G["cfg2_out"], FP32)


def test_oracle_cfg3():
    x, w = C.cfg3()
    got = oracle.gated_mul(oracle.linear(x[C.CFG3_ROWS], w, stage="tile"), epi="SILU")
    assert_close(got, G["cfg3_rows"], TRANS)


def test_oracle_cfg4():
    q, k = C.cfg4()
    for n, h in enumerate(C.CFG4_HEADS):
        got = oracle.attn_scores(q[h:h + 1], k[h:h + 1], scale=1.0 / 16, causal=True)[0]
        assert_close(got[C.CFG4_QROWS], G["cfg4_rows"][n], FP32)


def test_oracle_cfg5():
    x, w, b = C.cfg5()
    got = oracle.conv2d(x, w[C.CFG5_CHANNELS], b[C.CFG5_CHANNELS], epi="SILU")[0]
    assert_close(got, G["cfg5_channels"], TRANS)


# ---- the HIP kernels at full size ----

def _sums_close(got, want, scale, rtol=2e-5):
    err = np.abs(np.asarray(got, np.float64) - want)
    assert (err <= rtol * scale).all(), float((err / scale).max())


@pytest.mark.gpu
def test_gpu_cfg1(gpu):
    x, w, b = C.cfg1()
    D = gpu.DeviceArray.from_numpy
    out = gpu.DeviceArray((128, 3072), np.float32)
    gpu.linear(out, D(x), D(w), D(b), epi="GELU_TANH")
    got = out.numpy()
    assert_close(got[C.CFG1_ROWS], G["cfg1_rows"], FP32)
    _sums_close(got.astype(np.float64).sum(1), G["cfg1_rowsum"], np.abs(got).sum(1))


@pytest.mark.gpu
@pytest.mark.parametrize("m", [1, 4, 8])
def test_gpu_cfg2(gpu, m):
    x, w = C.cfg2()
    D = gpu.DeviceArray.from_numpy
    out = gpu.DeviceArray((m, 8192), np.float32)
    gpu.linear(out, D(x[:m]), D(w))
    assert_close(out.numpy(), G["cfg2_out"][:m], FP32)


@pytest.mark.gpu
def test_gpu_cfg3(gpu):
    x, w = C.cfg3()
    D = gpu.DeviceArray.from_numpy
    out = gpu.DeviceArray((2048, 8192), np.float32)
    gpu.linear(out, D(x), D(w), gated=True, gate_epi="SILU")
    got = out.numpy()
    assert_close(got[C.CFG3_ROWS], G["cfg3_rows"], TRANS)
    _sums_close(got.astype(np.float64).sum(1), G["cfg3_rowsum"], np.abs(got).sum(1), rtol=1e-4)


@pytest.mark.gpu
def test_gpu_cfg4(gpu):
    q, k = C.cfg4()
    D = gpu.DeviceArray.from_numpy
    s = gpu.DeviceArray((8, 1024, 1024), np.float32)
    gpu.attn_scores(s, D(q), D(k), scale=1.0 / 16, causal=True)
    got = s.numpy()
    for n, h in enumerate(C.CFG4_HEADS):
        assert_close(got[h][C.CFG4_QROWS], G["cfg4_rows"][n], FP32)
    i, j = np.indices((1024, 1024))
    assert np.isneginf(got[:, j > i]).all() and np.isfinite(got[:, j <= i]).all()
    vis = np.where(j <= i, got.astype(np.float64), 0.0).sum(2)
    _sums_close(vis, G["cfg4_visible_rowsum"], np.abs(np.where(j <= i, got, 0)).sum(2))


@pytest.mark.gpu
def test_gpu_cfg5(gpu):
    x, w, b = C.cfg5()
    D = gpu.DeviceArray.from_numpy
    out = gpu.DeviceArray((1, 128, 80, 80), np.float32)
    gpu.conv2d(out, D(x), D(w), D(b), epi="SILU")
    got = out.numpy()[0]
    assert_close(got[C.CFG5_CHANNELS], G["cfg5_channels"], TRANS)
    _sums_close(got.astype(np.float64).sum((1, 2)), G["cfg5_chansum"], np.abs(got).sum((1, 2)), rtol=1e-4)
