"""The five BASELINE.json configurations as seeded inputs (test infrastructure).

Draw convention of /root/reference/python/tests/node_check.py:51-78:
default_rng(0), parameters (weight, then bias) before inputs, drawn as
float32, then rounded to fp16 where the config says fp16 -- here with the
reference host's rounding (tensor.cpp:61-90: round-to-nearest-even, results
below the smallest normal half flushed to zero), restated in numpy so the
golden vectors do not depend on the oracle under test. Weights are drawn in
BASELINE's [K, N] layout and transposed to Linear's [N, K].
"""
import numpy as np

SMALLEST_NORMAL_F16 = 2.0 ** -14


def f16(x):
    x = np.asarray(x, np.float32)
    h = x.astype(np.float16)
    return np.where(np.abs(x) < SMALLEST_NORMAL_F16, np.copysign(np.float16(0), x).astype(np.float16), h)


def cfg1():
    rng = np.random.default_rng(0)
    w = (rng.standard_normal((768, 3072)) * 0.02).astype(np.float32).T.copy()
    b = (rng.standard_normal(3072) * 0.02).astype(np.float32)
    x = rng.standard_normal((128, 768)).astype(np.float32)
    return x, w, b


def cfg2():
    """X [8, 2048] (M = 1 and 4 use its leading rows), W [8192, 2048]."""
    rng = np.random.default_rng(0)
    w = f16((rng.standard_normal((2048, 8192)) * 0.02).astype(np.float32)).T.copy()
    x = f16(rng.standard_normal((8, 2048)).astype(np.float32))
    return x, w


def cfg3():
    rng = np.random.default_rng(0)
    wg = f16((rng.standard_normal((3072, 8192)) * 0.02).astype(np.float32)).T
    wu = f16((rng.standard_normal((3072, 8192)) * 0.02).astype(np.float32)).T
    w = np.ascontiguousarray(np.concatenate([wg, wu], axis=0))
    x = f16(rng.standard_normal((2048, 3072)).astype(np.float32))
    return x, w


def cfg4():
    rng = np.random.default_rng(0)
    q = f16(rng.standard_normal((8, 1024, 256)).astype(np.float32))
    k = f16(rng.standard_normal((8, 1024, 256)).astype(np.float32))
    return q, k


def cfg5():
    """Bias ~N(0, 0.02): BASELINE gives none, so this is chosen and recorded."""
    rng = np.random.default_rng(0)
    w = f16((rng.standard_normal((128, 128, 3, 3)) * 0.03).astype(np.float32))
    b = f16((rng.standard_normal(128) * 0.02).astype(np.float32))
    x = f16(rng.uniform(-1.0, 1.0, (1, 128, 80, 80)).astype(np.float32))
    return x, w, b


# Rows / heads / channels whose full outputs the fixtures hold.
CFG1_ROWS = np.array([0, 1, 31, 64, 100, 127])
CFG3_ROWS = np.array([0, 1, 511, 1024, 1500, 2047])
CFG4_HEADS = np.array([0, 7])
CFG4_QROWS = np.array([0, 1, 2, 255, 511, 1000, 1023])
CFG5_CHANNELS = np.array([0, 1, 64, 127])
