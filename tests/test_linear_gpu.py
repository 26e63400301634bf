"""Linear through the C ABI on the MI355X vs the oracle (and float64).

Cases follow the reference's own Linear tests (/root/reference/python/tests/
nodes/test_linear.py:11-84): slab M <= 8 at the FP32 tier, tile M > 8, odd N,
split-K, K tails, residual before/after; then BASELINE's configs 1-3.
Draws follow node_check: default_rng(0), params (weight, bias) before inputs.
"""
import ctypes

import numpy as np
import pytest

from helpers import FP16, FP32, TRANS, assert_close, draw, max_rel_err, normal
from oracle import oracle

pytestmark = pytest.mark.gpu


def run_linear(capi, x, w, b=None, r=None, out_dtype=np.float32, **kw):
    dx, dw = capi.DeviceArray.from_numpy(x), capi.DeviceArray.from_numpy(w)
    db = capi.DeviceArray.from_numpy(b) if b is not None else None
    dr = capi.DeviceArray.from_numpy(r) if r is not None else None
    N = w.shape[0] // 2 if kw.get("gated") else w.shape[0]
    out = capi.DeviceArray(x.shape[:-1] + (N,), out_dtype)
    capi.linear(out, dx, dw, db, dr, **kw)
    return out.numpy()


@pytest.mark.parametrize(
    "m, k, n, has_bias, epi, split, tol",
    [
        (1, 64, 32, True, "NONE", 0, FP32),
        (33, 64, 32, True, "NONE", 0, FP32),   # the reference reruns slab_m1 at M=33
        (8, 96, 40, False, "NONE", 0, FP32),
        (33, 96, 48, True, "RELU", 0, FP32),
        (64, 128, 100, False, "GELU_TANH", 0, TRANS),
        (16, 256, 64, True, "NONE", 64, FP32),
        (33, 1000, 100, True, "NONE", 0, FP32),
        (33, 100, 48, False, "NONE", 0, FP32),
        (33, 102, 48, False, "NONE", 0, FP32),
        (33, 101, 48, False, "NONE", 0, FP32),
        (16, 2050, 64, True, "NONE", 0, FP32),
        (33, 1000, 48, False, "NONE", 100, FP32),
        (3, 101, 77, True, "SILU", 0, TRANS),
        (200, 300, 260, True, "GELU", 0, TRANS),
        (130, 64, 70, True, "SIGMOID", 0, TRANS),
    ],
)
def test_linear_f32(gpu, m, k, n, has_bias, epi, split, tol):
    rng = np.random.default_rng(0)
    w = draw(normal((n, k), 1.0 / np.sqrt(k)), rng)
    b = draw((n,), rng) if has_bias else None
    x = draw((m, k), rng)
    got = run_linear(gpu, x, w, b, epi=epi, split_size=split)
    want = oracle.linear(x, w, b, epi=epi, split_size=split)
    assert_close(got, want, tol, "vs oracle")
    # and the float64 closed form at the reference's own tier for this path
    ref = x.astype(np.float64) @ w.astype(np.float64).T + (0 if b is None else b.astype(np.float64))
    ref = oracle.epilogue(ref.astype(np.float32), epi) if epi != "NONE" else ref
    assert_close(got, ref, FP16 if m > 8 else TRANS, "vs float64")
    # replay is bit-identical (node_check's second forward)
    again = run_linear(gpu, x, w, b, epi=epi, split_size=split)
    np.testing.assert_array_equal(again, got)


@pytest.mark.parametrize("m, order", [(4, 0), (4, 1), (33, 0), (33, 1), (64, 1)])
def test_linear_residual(gpu, m, order):
    k, n = 64, 48
    rng = np.random.default_rng(0)
    w = draw(normal((n, k), 1.0 / np.sqrt(k)), rng)
    b = draw((n,), rng)
    x = draw((m, k), rng)
    r = draw((m, n), rng)
    got = run_linear(gpu, x, w, b, r, epi="RELU", order=order)
    want = oracle.linear(x, w, b, r, epi="RELU", order=order)
    assert_close(got, want, FP32)


@pytest.mark.parametrize("m, scale, rep", [(5, 0.5, True), (40, -2.0, True), (40, 0.25, False)])
def test_linear_scale_repeat(gpu, m, scale, rep):
    """scalarScale and [N]-repeating vs full [M,N] residual (linear.h:49-50,2333-2338)."""
    k, n = 96, 64
    rng = np.random.default_rng(1)
    w = draw(normal((n, k), 0.1), rng)
    b = draw((n,), rng)
    x = draw((m, k), rng)
    r = draw((n,) if rep else (m, n), rng)
    got = run_linear(gpu, x, w, b, r, epi="SILU", scale=scale)
    want = oracle.linear(x, w, b, r, epi="SILU", scale=scale)
    assert_close(got, want, TRANS)


@pytest.mark.parametrize("m, k, n, idt, wdt, odt", [
    (1, 2048, 512, np.float16, np.float16, np.float32),
    (8, 2048, 256, np.float16, np.float16, np.float16),
    (5, 512, 96, np.float32, np.float16, np.float32),
    (64, 512, 256, np.float16, np.float16, np.float32),
    (100, 300, 130, np.float32, np.float16, np.float32),   # tile stages I as fp16
    (70, 256, 64, np.float16, np.float32, np.float32),     # tile stages W as fp16
    (128, 1024, 512, np.float16, np.float16, np.float16),
])
def test_linear_mixed_dtypes(gpu, m, k, n, idt, wdt, odt):
    rng = np.random.default_rng(0)
    w = draw(normal((n, k), 0.02), rng, wdt)
    b = draw(normal((n,), 0.02), rng, wdt)
    x = draw((m, k), rng, idt)
    got = run_linear(gpu, x, w, b, out_dtype=odt, epi="GELU_TANH")
    want = oracle.linear(x, w, b, epi="GELU_TANH", out_dtype=odt)
    tol = FP16 if odt == np.float16 else TRANS
    assert_close(got.astype(np.float32), want.astype(np.float32), tol)


@pytest.mark.parametrize("m, k, h, split", [(8, 256, 96, 0), (64, 256, 64, 0), (300, 512, 200, 0),
                                           (40, 4096, 64, 0), (33, 1000, 48, 100)])
def test_linear_gated(gpu, m, k, h, split):
    """Linear over concat(gate, up) + GatedMul(SiLU), fused (gated-feed-forward.h:37-46)."""
    rng = np.random.default_rng(0)
    w = draw(normal((2 * h, k), 0.05), rng, np.float16)
    b = draw(normal((2 * h,), 0.02), rng, np.float16)
    x = draw((m, k), rng, np.float16)
    got = run_linear(gpu, x, w, b, gated=True, gate_epi="SILU", split_size=split)
    y = oracle.linear(x, w, b)
    want = oracle.gated_mul(y, epi="SILU")
    assert_close(got, want, TRANS)


def test_gated_mul_alone(gpu):
    rng = np.random.default_rng(0)
    x = draw((37, 2 * 50), rng)
    d = gpu.DeviceArray.from_numpy(x)
    out = gpu.DeviceArray((37, 50), np.float32)
    gpu.gated_mul(out, d, "GELU")
    assert_close(out.numpy(), oracle.gated_mul(x, epi="GELU"), TRANS)


# ---- BASELINE configs ----

def test_config1_gpt2_cfc(gpu):
    """X[128,768] f32, W[768,3072]^T, bias, GELU-tanh; fp32 tier 1e-5."""
    rng = np.random.default_rng(0)
    w = draw(normal((768, 3072), 0.02), rng).T.copy()
    b = draw(normal((3072,), 0.02), rng)
    x = draw((128, 768), rng)
    got = run_linear(gpu, x, w, b, epi="GELU_TANH")
    want = oracle.linear(x, w, b, epi="GELU_TANH")
    assert_close(got, want, FP32)


@pytest.mark.parametrize("m", [1, 4, 8])
def test_config2_decode_gemv(gpu, m):
    rng = np.random.default_rng(0)
    w = draw(normal((2048, 8192), 0.02), rng, np.float16).T.copy()
    x = draw((m, 2048), rng, np.float16)
    got = run_linear(gpu, x, w)
    want = oracle.linear(x, w)
    assert_close(got, want, FP32)


def test_config3_prefill_gate_up(gpu):
    """X[2048,3072], concat(W_gate, W_up) -> [16384, 3072], SiLU(g)*u, fp32 out.
    The oracle checks a sample of 48 rows at full size."""
    rng = np.random.default_rng(0)
    wg = draw(normal((3072, 8192), 0.02), rng, np.float16).T
    wu = draw(normal((3072, 8192), 0.02), rng, np.float16).T
    w = np.ascontiguousarray(np.concatenate([wg, wu], axis=0))
    x = draw((2048, 3072), rng, np.float16)
    got = run_linear(gpu, x, w, gated=True, gate_epi="SILU")
    assert np.isfinite(got).all()
    rows = np.random.default_rng(5).choice(2048, 48, replace=False)
    rows[:2] = [0, 2047]
    want = oracle.gated_mul(oracle.linear(x[rows], w, stage="tile"), epi="SILU")
    assert_close(got[rows], want, TRANS)


@pytest.mark.parametrize("m, k, n, gated, odt, epi, residual", [
    (1024, 512, 8192, False, np.float32, "GELU_TANH", True),     # 256x256 tiles, residual [N]
    (1000, 384, 8200, False, np.float16, "RELU", False),         # M and N tails
    (777, 256, 2 * 4160, True, np.float32, "SILU", False),       # gated, M and H tails
    (2048, 512, 2 * 4096, True, np.float16, "GELU", False),
])
def test_linear_big_tile(gpu, m, k, n, gated, odt, epi, residual):
    """The 256x256 MFMA path (large M, K % 32 == 0) vs the oracle on sampled rows."""
    rng = np.random.default_rng(0)
    w = draw(normal((n, k), 0.05), rng, np.float16)
    b = draw(normal((n,), 0.05), rng, np.float16)
    x = draw((m, k), rng, np.float16)
    r = draw((n,), rng, odt) if residual else None
    kw = dict(gated=True, gate_epi=epi) if gated else dict(epi=epi)
    a = gpu.linear_args(gpu.DeviceArray((m, n // 2 if gated else n), odt), gpu.DeviceArray((m, k), np.float16),
                        gpu.DeviceArray((n, k), np.float16), **kw)
    assert gpu.linear_plan(a)[0].startswith("tile_f16_256x256")
    got = run_linear(gpu, x, w, b, r, out_dtype=odt, **kw)
    rows = np.unique(np.concatenate([np.arange(4), np.arange(m - 4, m),
                                     np.random.default_rng(1).choice(m, 24, replace=False)]))
    if gated:
        want = oracle.gated_mul(oracle.linear(x[rows], w, b, stage="tile"), epi=epi, out_dtype=odt)
    else:
        want = oracle.linear(x[rows], w, b, r, epi=epi, out_dtype=odt, stage="tile")
    tol = FP16 if odt == np.float16 else TRANS
    assert_close(got[rows].astype(np.float32), want.astype(np.float32), tol)


@pytest.mark.parametrize("m, k, n, gated, odt, epi, residual, bias", [
    (1024, 512, 8192, False, np.float32, "GELU_TANH", True, True),    # residual [N]: per-output path
    (1000, 384, 8200, False, np.float16, "RELU", False, True),        # M and N tails, fp16 out
    (777, 256, 2 * 4160, True, np.float32, "SILU", False, True),      # gated, M and H tails
    (2048, 512, 2 * 4096, True, np.float16, "GELU", False, False),
    (2048, 768, 2 * 4096, True, np.float32, "GELU_TANH", False, True),
    (4096, 256, 4096, False, np.float32, "NONE", False, False),       # full tiles, fast stores
    (2304, 1280, 2 * 2048, True, np.float32, "SIGMOID", False, False),  # runtime-activation fast path
])
def test_linear_packed_weight(gpu, m, k, n, gated, odt, epi, residual, bias):
    """The packed-weight prefill path (weight streamed into VGPRs in fragment
    order) vs the oracle on sampled rows, through vai_linear_pack_weight."""
    rng = np.random.default_rng(0)
    w = draw(normal((n, k), 0.05), rng, np.float16)
    b = draw(normal((n,), 0.05), rng, np.float16) if bias else None
    x = draw((m, k), rng, np.float16)
    r = draw((n,), rng, odt) if residual else None
    kw = dict(gated=True, gate_epi=epi) if gated else dict(epi=epi)
    D = gpu.DeviceArray.from_numpy
    dx, dw = D(x), D(w)
    out = gpu.DeviceArray((m, n // 2 if gated else n), odt)
    a = gpu.linear_args(out, dx, dw, D(b) if bias else None, D(r) if residual else None, **kw)
    packed = gpu.linear_pack_weight(a)
    assert packed is not None
    a.packed_weight = packed.ptr
    assert gpu.linear_plan(a)[0].startswith("tile_f16_256x256_packed")
    got = gpu.linear(out, dx, dw, D(b) if bias else None, D(r) if residual else None, packed=packed, **kw).numpy()
    rows = np.unique(np.concatenate([np.arange(4), np.arange(m - 4, m),
                                     np.random.default_rng(1).choice(m, 24, replace=False)]))
    if gated:
        want = oracle.gated_mul(oracle.linear(x[rows], w, b, stage="tile"), epi=epi, out_dtype=odt)
    else:
        want = oracle.linear(x[rows], w, b, r, epi=epi, out_dtype=odt, stage="tile")
    tol = FP16 if odt == np.float16 else TRANS
    assert_close(got[rows].astype(np.float32), want.astype(np.float32), tol)
    # same MFMA order as the LDS-staged kernel: bit-identical fp32 sums. The
    # two epilogues may contract the activation arithmetic differently, so an
    # fp16 output may differ by one fp16 ulp (and no more).
    ref = run_linear(gpu, x, w, b, r, out_dtype=odt, **kw)
    if odt == np.float16:
        mag = np.maximum(np.abs(got), np.abs(ref)).astype(np.float16)
        diff = np.abs(got.astype(np.float32) - ref.astype(np.float32)) > np.spacing(mag).astype(np.float32)
    else:
        diff = got != ref
    if diff.any():
        # say where, and which of the two kernels the oracle sides with
        rr, cc = np.nonzero(diff)
        rows_bad = np.unique(rr)[:8]
        if gated:
            w_rows = oracle.gated_mul(oracle.linear(x[rows_bad], w, b, stage="tile"), epi=epi, out_dtype=odt)
        else:
            w_rows = oracle.linear(x[rows_bad], w, b, r, epi=epi, out_dtype=odt, stage="tile")
        e_packed = np.abs(got[rows_bad].astype(np.float64) - w_rows).max()
        e_lds = np.abs(ref[rows_bad].astype(np.float64) - w_rows).max()
        pytest.fail(f"{diff.sum()} outputs differ; rows {np.unique(rr)[:16]} (of {len(np.unique(rr))}), "
                    f"cols {np.unique(cc)[:16]} (of {len(np.unique(cc))}); rows % 256 {np.unique(rr % 256)[:16]}, "
                    f"cols % 128 {np.unique(cc % 128)[:16]}; max error vs oracle on those rows: packed {e_packed:.3g}, "
                    f"LDS-staged {e_lds:.3g}")


def test_linear_packed_weight_rejects(gpu):
    """No packed path for fp32 weights or K % 128 != 0; a short buffer is refused."""
    D = gpu.DeviceArray
    a = gpu.linear_args(D((512, 512), np.float32), D((512, 384), np.float32), D((512, 384), np.float32))
    assert gpu.lib().vai_linear_packed_weight_size(ctypes.byref(a)) == 0
    a = gpu.linear_args(D((512, 512), np.float32), D((512, 320), np.float16), D((512, 320), np.float16))
    assert gpu.lib().vai_linear_packed_weight_size(ctypes.byref(a)) == 0
    a = gpu.linear_args(D((512, 512), np.float32), D((512, 384), np.float16), D((512, 384), np.float16))
    n = gpu.lib().vai_linear_packed_weight_size(ctypes.byref(a))
    assert n == 2 * 8 * 384 * 64
    small = D((n - 16,), np.uint8)
    assert gpu.lib().vai_linear_pack_weight(ctypes.byref(a), small.ptr, small.nbytes, None) == 1004


@pytest.mark.parametrize("m, k, n, bias, res, order, odt, epi", [
    (128, 768, 3072, "row", None, 0, np.float32, "GELU_TANH"),   # config 1's shape, 32x48 tiles
    (9, 32, 16, "row", None, 0, np.float32, "NONE"),              # one K stage: waves 1-3 idle
    (33, 96, 100, "full", "full", 1, np.float32, "RELU"),         # ragged M and N, 3 stages
    (100, 800, 130, None, "row", 0, np.float16, "SILU"),          # fp16 output, [N] residual
    (64, 1024, 1000, "row", "full", 0, np.float32, "SIGMOID"),
    (200, 288, 60, "row", None, 0, np.float32, "GELU"),           # 9 stages: not a multiple of 4
    (40, 7 * 32 * 4, 50, "row", None, 0, np.float32, "NONE"),     # 7 stages per wave: ring tail of 1
])
def test_linear_f32_small(gpu, m, k, n, bias, res, order, odt, epi):
    """The one-launch fp32 path (32 x 16*nf tiles, K split over the four
    waves and summed in LDS) vs the oracle and the float64 closed form."""
    rng = np.random.default_rng(3)
    w = draw(normal((n, k), 1.0 / np.sqrt(k)), rng)
    b = draw((n,) if bias == "row" else (m, n), rng) if bias else None
    x = draw((m, k), rng)
    r = draw((n,) if res == "row" else (m, n), rng, odt) if res else None
    D = gpu.DeviceArray.from_numpy
    a = gpu.linear_args(gpu.DeviceArray((m, n), odt), D(x), D(w), D(b) if bias else None, D(r) if res else None,
                        epi=epi, order=order)
    name, splits = gpu.linear_plan(a)
    assert name.startswith("tile_f32_32x") and splits == 1, name
    assert gpu.lib().vai_linear_workspace_size(ctypes.byref(a)) == 0
    got = run_linear(gpu, x, w, b, r, out_dtype=odt, epi=epi, order=order)
    want = oracle.linear(x, w, b, r, epi=epi, order=order, out_dtype=odt)
    tol = FP16 if odt == np.float16 else (FP32 if epi in ("NONE", "RELU") else TRANS)
    assert_close(got.astype(np.float32), want.astype(np.float32), tol)
    again = run_linear(gpu, x, w, b, r, out_dtype=odt, epi=epi, order=order)
    np.testing.assert_array_equal(again, got)


@pytest.mark.parametrize("m, k, n, odt, epi, residual, bias, splits", [
    (2048, 8192, 3072, np.float16, "NONE", True, False, 2),    # the FFN down projection: 96 tiles
    (1000, 2048, 1000, np.float32, "GELU_TANH", False, True, 8),   # 16 tiles, M and N tails
    (512, 4096, 2304, np.float32, "SILU", True, True, 8),      # [M,N] residual; 14 splits do not divide K
])
def test_linear_packed_split_k(gpu, m, k, n, odt, epi, residual, bias, splits):
    """Packed-weight GEMMs with too few 256x256 tiles split K into units
    that fill the CUs; the partial planes go through the reduce pass, which
    applies bias, activation and residual. vs the oracle on sampled rows."""
    rng = np.random.default_rng(2)
    w = draw(normal((n, k), 0.02), rng, np.float16)
    b = draw(normal((n,), 0.05), rng, np.float16) if bias else None
    x = draw((m, k), rng, np.float16)
    r = draw((m, n), rng, odt) if residual else None
    D = gpu.DeviceArray.from_numpy
    dx, dw = D(x), D(w)
    out = gpu.DeviceArray((m, n), odt)
    db, dr = (D(b) if bias else None), (D(r) if residual else None)
    a = gpu.linear_args(out, dx, dw, db, dr, epi=epi)
    packed = gpu.linear_pack_weight(a)
    a.packed_weight = packed.ptr
    name, got_splits = gpu.linear_plan(a)
    assert name == "tile_f16_256x256_packed" and got_splits == splits, (name, got_splits)
    got = gpu.linear(out, dx, dw, db, dr, packed=packed, epi=epi).numpy()
    rows = np.unique(np.concatenate([np.arange(4), np.arange(m - 4, m),
                                     np.random.default_rng(1).choice(m, 24, replace=False)]))
    want = oracle.linear(x[rows], w, b, r[rows] if residual else None, epi=epi, out_dtype=odt, stage="tile")
    tol = FP16 if odt == np.float16 else TRANS
    assert_close(got[rows].astype(np.float32), want.astype(np.float32), tol)
    again = gpu.linear(out, dx, dw, db, dr, packed=packed, epi=epi).numpy()
    np.testing.assert_array_equal(again, got)


@pytest.mark.parametrize("m, k, n, gated, odt", [
    (777, 256, 2 * 4160, True, np.float32),    # one tile per workgroup, 4 K stages
    (512, 4096, 2304, False, np.float32),      # split-K units, one per workgroup
    (1000, 384, 8200, False, np.float16),      # 6 K stages, M and N tails
])
def test_linear_packed_repeatable(gpu, m, k, n, gated, odt):
    """Regression test for two causes of intermittent wrong blocks: operand
    registers reused by the loads interleaved with the MFMAs (the last rows of
    one wave's fragment off by a k step), and a stage-end wait count that
    relied on LDS copies completing before younger VGPR loads (the 8 rows one
    LDS copy writes, stale in some waves). Six launches give bit-identical
    outputs that match the oracle on sampled rows."""
    rng = np.random.default_rng(11)
    w = draw(normal((n, k), 0.05), rng, np.float16)
    b = draw(normal((n,), 0.05), rng, np.float16)
    x = draw((m, k), rng, np.float16)
    kw = dict(gated=True, gate_epi="SILU") if gated else dict(epi="SILU")
    D = gpu.DeviceArray.from_numpy
    dx, dw, db = D(x), D(w), D(b)
    out = gpu.DeviceArray((m, n // 2 if gated else n), odt)
    a = gpu.linear_args(out, dx, dw, db, **kw)
    packed = gpu.linear_pack_weight(a)
    first = gpu.linear(out, dx, dw, db, packed=packed, **kw).numpy()
    rows = np.unique(np.concatenate([np.arange(8), np.random.default_rng(3).choice(m, 24, replace=False)]))
    if gated:
        want = oracle.gated_mul(oracle.linear(x[rows], w, b, stage="tile"), epi="SILU", out_dtype=odt)
    else:
        want = oracle.linear(x[rows], w, b, epi="SILU", out_dtype=odt, stage="tile")
    assert_close(first[rows].astype(np.float32), want.astype(np.float32), FP16 if odt == np.float16 else TRANS)
    for _ in range(5):
        out.fill_(0xFF)
        np.testing.assert_array_equal(gpu.linear(out, dx, dw, db, packed=packed, **kw).numpy(), first)


@pytest.mark.parametrize("m, k, n, epi, bias, resid, odt, gated", [
    (3, 256, 1000, "NONE", True, False, np.float32, False),       # N tail inside a 32-row block
    (4, 2048, 8192, "NONE", False, False, np.float32, False),     # config 2's shape
    (8, 2048, 8192, "GELU_TANH", True, True, np.float32, False),
    (5, 4096, 640, "SILU", True, False, np.float16, False),       # two fragment passes per wave
    (8, 384, 96, "NONE", False, False, np.float32, False),        # fewer fragments than waves
    (4, 512, 2 * 520, "SILU", True, False, np.float32, True),     # gated: packed gate/up blocks, H tail
    (7, 1024, 2 * 4096, "GELU", False, False, np.float16, True),
])
def test_gemv_packed(gpu, m, k, n, epi, bias, resid, odt, gated):
    """The decode GEMV over the packed weight (M 3-8) vs the oracle and vs the
    row-streaming kernels on the same inputs."""
    rng = np.random.default_rng(m * 100 + k)
    w = draw(normal((n, k), 0.02), rng, np.float16)
    b = draw(normal((n,), 0.02), rng, np.float16) if bias else None
    x = draw((m, k), rng, np.float16)
    cols = n // 2 if gated else n
    r = draw((m, cols), rng, odt) if resid else None
    kw = dict(gated=True, gate_epi=epi) if gated else dict(epi=epi)
    D = gpu.DeviceArray.from_numpy
    dx, dw = D(x), D(w)
    db, dr = (D(b) if bias else None), (D(r) if resid else None)
    out = gpu.DeviceArray((m, cols), odt)
    a = gpu.linear_args(out, dx, dw, db, dr, **kw)
    packed = gpu.linear_pack_weight(a)
    a.packed_weight = packed.ptr
    assert gpu.linear_plan(a)[0].startswith("slab_packed")
    print(f"gemv packed m={m} k={k} n={n} gated={gated}", flush=True)
    got = gpu.linear(out, dx, dw, db, dr, packed=packed, **kw).numpy()
    if gated:
        want = oracle.gated_mul(oracle.linear(x, w, b, stage="slab"), epi=epi, out_dtype=odt)
    else:
        want = oracle.linear(x, w, b, r, epi=epi, out_dtype=odt, stage="slab")
    tol = FP16 if odt == np.float16 else (TRANS if epi != "NONE" else FP32)
    assert_close(got.astype(np.float32), want.astype(np.float32), tol)
    ref = run_linear(gpu, x, w, b, r, out_dtype=odt, **kw)
    assert_close(got.astype(np.float32), ref.astype(np.float32), tol)


@pytest.mark.parametrize("m", [1, 2, 4, 8])
def test_gemv_fp16_subnormals(gpu, m):
    """fp16 weights and inputs with subnormal values (a device-made fp16
    tensor keeps them): the GEMV's dot products must use them as stored."""
    rng = np.random.default_rng(m)
    k, n = 512, 256
    w = (rng.standard_normal((n, k)) * 2.0 ** -16).astype(np.float16)   # mostly subnormal halves
    x = rng.standard_normal((m, k)).astype(np.float16)
    assert (np.abs(w) < np.float16(2.0 ** -14)).mean() > 0.5
    got = run_linear(gpu, x, w)
    want = x.astype(np.float64) @ w.astype(np.float64).T
    assert_close(got, want, (1e-5, 1e-9))
