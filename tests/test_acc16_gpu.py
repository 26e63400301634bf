"""Linear with an fp16 accumulator (Linear::setAccDtype(Fp16), /root/reference/
vai/nodes/linear.h:289,2320; vai/shaders/linear-tile.comp:55,71,292-320) on the
MI355X against the oracle's restatement of the same fma chain. The sums follow
one fixed order, so raw sums (and bias / residual / scale, fp32 adds) are
bit-identical; transcendental epilogues are held to the TRANS tier."""
import numpy as np
import pytest

from helpers import TRANS, assert_close, draw, normal
from oracle import oracle
from test_linear_gpu import run_linear

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("m, k, n, bias, resid, odt, split", [
    (9, 64, 32, False, False, np.float32, 0),
    (64, 256, 64, True, False, np.float32, 0),
    (100, 1000, 130, True, True, np.float32, 0),      # K tail inside a 4-step, row / column tails
    (130, 517, 70, False, False, np.float16, 0),
    (77, 1024, 96, True, False, np.float32, 256),     # requested split-K: fp16 sums per span, fp32 fold
    (33, 300, 50, True, True, np.float32, 100),
])
def test_acc16_bit_exact(gpu, m, k, n, bias, resid, odt, split):
    rng = np.random.default_rng(m + k)
    w = draw(normal((n, k), 0.05), rng, np.float16)
    b = draw(normal((n,), 0.05), rng) if bias else None
    x = draw((m, k), rng, np.float16)
    r = draw((m, n), rng, odt) if resid else None
    args = gpu.linear_args(gpu.DeviceArray((m, n), odt), gpu.DeviceArray((m, k), np.float16),
                           gpu.DeviceArray((n, k), np.float16), split_size=split, acc=np.float16)
    plan = gpu.linear_plan(args)
    assert plan[0] == "tile_acc16_64x64" and plan[1] == (-(-k // split) if split else 1)
    got = run_linear(gpu, x, w, b, r, out_dtype=odt, split_size=split, acc=np.float16)
    want = oracle.linear_acc16(x, w, b, r, out_dtype=odt, split_size=split)
    assert np.array_equal(got, want), f"{(got != want).sum()} outputs differ, max {np.abs(got - want).max()}"
    # and it is not the fp32-accumulated result
    f32 = oracle.linear(x, w, b, r, out_dtype=odt, stage="tile", split_size=split)
    assert not np.array_equal(got, f32)


def test_acc16_epilogues_gated_and_fp32_input(gpu):
    rng = np.random.default_rng(3)
    w = draw(normal((96, 384), 0.05), rng, np.float16)
    b = draw(normal((96,), 0.05), rng)
    x = draw((70, 384), rng)   # fp32 input: staged to fp16 by the tile contract
    got = run_linear(gpu, x, w, b, epi="GELU_TANH", scale=0.5, acc=np.float16)
    assert_close(got, oracle.linear_acc16(x, w, b, epi="GELU_TANH", scale=0.5), TRANS)
    got = run_linear(gpu, x, w, b, gated=True, gate_epi="SILU", acc=np.float16)
    assert_close(got, oracle.linear_acc16(x, w, b, gated=True, gate_epi="SILU"), TRANS)
    got = run_linear(gpu, x, w, None, gated=True, gate_epi="NONE", acc=np.float16, split_size=128)
    assert np.array_equal(got, oracle.linear_acc16(x, w, gated=True, gate_epi="NONE", split_size=128))


def test_acc16_clamps_overflow(gpu):
    x = np.full((16, 64), 100, np.float16)
    w = np.stack([np.full(64, 100), np.full(64, -100), np.full(64, 0.5)]).astype(np.float16)
    got = run_linear(gpu, x, w, acc=np.float16)
    assert (got == np.array([65504, -65504, 3200], np.float32)).all()


def test_acc16_where_the_reference_keeps_fp32(gpu):
    """The GEMV (M <= 8) and fp32 x fp32 products accumulate in fp32 whatever
    is asked, as the reference's linear-slab and stageF32 tile do."""
    D = gpu.DeviceArray
    a = gpu.linear_args(D((8, 64), np.float32), D((8, 256), np.float16), D((64, 256), np.float16), acc=np.float16)
    assert gpu.linear_plan(a)[0].startswith("slab")
    a = gpu.linear_args(D((64, 64), np.float32), D((64, 256), np.float32), D((64, 256), np.float32), acc=np.float16)
    assert "acc16" not in gpu.linear_plan(a)[0]
    rng = np.random.default_rng(1)
    x = draw((4, 256), rng, np.float16)
    w = draw(normal((64, 256), 0.05), rng, np.float16)
    assert_close(run_linear(gpu, x, w, acc=np.float16), oracle.linear(x, w, stage="slab"), (1e-5, 1e-6))


@pytest.mark.parametrize("m, k, n, want_splits", [
    (64, 4096, 64, 8),     # one 64x64 tile: 8 spans of 512, each its own fp16 chain
    (130, 2304, 260, 5),   # 6 tiles of 128: 8-6 splits leave the last span empty, 5 do not
])
def test_acc16_auto_split_bit_exact(gpu, m, k, n, want_splits):
    """splitSize 0 with K >= 2048 on an underfilled grid: the reference splits
    K by ggmlGuessSplitCount (linear.h:600-632) and so does the plan; the sums
    match the oracle's chains over the same 256-rounded spans bit for bit."""
    rng = np.random.default_rng(k)
    w = draw(normal((n, k), 0.02), rng, np.float16)
    x = draw((m, k), rng, np.float16)
    args = gpu.linear_args(gpu.DeviceArray((m, n), np.float32), gpu.DeviceArray((m, k), np.float16),
                           gpu.DeviceArray((n, k), np.float16), acc=np.float16)
    assert gpu.linear_plan(args)[1] == want_splits
    span = -(-(-(-k // want_splits)) // 256) * 256
    got = run_linear(gpu, x, w, acc=np.float16)
    want = oracle.linear_acc16(x, w, split_size=span)
    assert np.array_equal(got, want), f"{(got != want).sum()} outputs differ"
    assert not np.array_equal(got, oracle.linear_acc16(x, w))   # one chain over all of K differs
