"""Shared test helpers: the reference's draw convention and tolerance tiers.

Tolerance tiers are the reference's (/root/reference/python/tests/
node_check.py:20-28): (rtol, atol) for numpy.testing.assert_allclose.
"""
import numpy as np

from oracle import oracle

EXACT = (0.0, 0.0)
FP32 = (1e-5, 1e-5)
TRANS = (1e-4, 1e-5)
FP16 = (1e-3, 5e-3)
# BASELINE's fp16-with-fp32-accumulation bound, as an allclose tier.
FP16_BASELINE = (1e-2, 1e-2)


def normal(shape, scale=1.0):
    return lambda rng: scale * rng.standard_normal(shape)


def uniform(shape, low, high):
    return lambda rng: rng.uniform(low, high, shape)


def draw(gen, rng, dtype=np.float32):
    """Draw as float32 (node_check._draw), then round to fp16 the way the
    reference host does (tensor.cpp floatToHalf) when dtype is fp16."""
    a = gen(rng) if callable(gen) else rng.standard_normal(gen)
    a = np.ascontiguousarray(a, dtype=np.float32)
    if np.dtype(dtype) == np.float16:
        return oracle.to_f16(a)
    return a


def max_rel_err(got, want):
    """BASELINE's metric: max |got-ref| / max(|ref|, 1e-6 * max|ref|) over finite refs."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    fin = np.isfinite(want)
    if not fin.any():
        return 0.0
    floor = 1e-6 * np.abs(want[fin]).max()
    return float((np.abs(got[fin] - want[fin]) / np.maximum(np.abs(want[fin]), floor)).max())


def cond_rel_err(got, want, mag):
    """BASELINE's relative error with each element's floor raised to the
    magnitude its fp32 accumulation works at: max |got-ref| / max(|ref|, mag),
    mag = sum_k |a_k b_k| (carried through the epilogue). Any fp32-accumulating
    kernel, the reference's included, differs from the float64 truth by up to
    about sqrt(K) * 2^-24 * mag, so where a dot product cancels to near zero the
    literal metric (floor 1e-6 max|ref|) measures the cancellation, not the
    kernel."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    mag = np.broadcast_to(np.asarray(mag, np.float64), want.shape)
    fin = np.isfinite(want)
    if not fin.any():
        return 0.0
    return float((np.abs(got[fin] - want[fin]) / np.maximum(np.abs(want[fin]), mag[fin])).max())


def assert_close(got, want, tol, what=""):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    same_inf = np.isinf(want)
    assert np.array_equal(np.isinf(got), same_inf), f"{what}: -inf pattern differs"
    assert (got[same_inf] == want[same_inf]).all(), f"{what}: inf sign differs"
    np.testing.assert_allclose(got[~same_inf], want[~same_inf], rtol=tol[0], atol=tol[1], err_msg=what)


def np_epilogue(name, y):
    """float64 closed forms of the reference's epilogues (activation.h:19-58)."""
    import math
    y = np.asarray(y, np.float64)
    if name == "NONE":
        return y
    if name == "RELU":
        return np.maximum(y, 0)
    if name == "GELU":
        erf = np.vectorize(math.erf)
        return 0.5 * y * (1 + erf(y / math.sqrt(2)))
    if name == "GELU_TANH":
        return 0.5 * y * (1 + np.tanh(math.sqrt(2 / math.pi) * (y + 0.044715 * y ** 3)))
    if name == "SILU":
        return y / (1 + np.exp(-y))
    if name == "SIGMOID":
        return 1 / (1 + np.exp(-y))
    raise ValueError(name)
