"""Fused attention forward (scores, online softmax, P.V in one kernel)
through the C ABI vs the oracle's float64 softmax(S) V. The reference's
Attention node (/root/reference/vai/nodes/attention.h:979-1304, shaders/
attention-fa.comp) with its causal / sliding-window rule (common/
causal_mask.h:25-42), GQA, Tq != Tkv, head dims 64/128/256, tails.
P enters the P.V product as fp16 (as the reference's fp16 P.V operand), so
the comparison uses the fp16 tier.
"""
import numpy as np
import pytest

from helpers import FP16, assert_close, draw
from oracle import oracle

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("b, hq, hkv, tq, tkv, d, causal, span, odt", [
    (1, 8, 8, 1024, 1024, 256, True, 0, np.float32),     # config 4's shape, full attention output
    (1, 8, 8, 1024, 1024, 256, True, 0, np.float16),     # the bench's attn line: split, fp16 partials
    (1, 8, 2, 200, 200, 128, True, 0, np.float16),       # GQA, row and key tails
    (1, 4, 4, 3, 300, 64, True, 0, np.float32),          # decode-like: 3 new queries over 300 keys
    (1, 2, 1, 257, 257, 64, True, 50, np.float32),       # sliding window
    (2, 2, 2, 100, 130, 128, False, 0, np.float32),      # no mask, batch 2
    (1, 1, 1, 70, 40, 64, True, 0, np.float32),          # Tq > Tkv: the first 30 queries see no key
    (1, 2, 2, 64, 1000, 128, False, 0, np.float32),      # one query tile, 16 key tiles: split in 4 and merged
    (1, 2, 2, 600, 520, 64, True, 0, np.float16),        # split, and a query tile that sees no key
    (1, 2, 2, 64, 4096, 64, False, 0, np.float16),       # 32 chunks per query tile: the merge's general path
    (1, 1, 1, 2176, 2176, 64, True, 0, np.float16),      # 17 query tiles: the merge reads the unit table
])
def test_attention(gpu, b, hq, hkv, tq, tkv, d, causal, span, odt):
    rng = np.random.default_rng(7)
    q = draw((b, hq, tq, d), rng, np.float16)
    k = draw((b, hkv, tkv, d), rng, np.float16)
    v = draw((b, hkv, tkv, d), rng, np.float16)
    D = gpu.DeviceArray.from_numpy
    out = gpu.DeviceArray((b, hq, tq, d), odt)
    print(f"attention b={b} hq={hq} hkv={hkv} tq={tq} tkv={tkv} d={d} causal={causal} span={span}", flush=True)
    got = gpu.attention(out, D(q), D(k), D(v), causal=causal, span=span).numpy().astype(np.float32)
    want = oracle.attention(q, k, v, causal=causal, span=span, out_dtype=np.float32)
    assert_close(got, want, FP16)
    if causal and tq > tkv:
        np.testing.assert_array_equal(got[..., : tq - tkv, :], 0.0)


@pytest.mark.parametrize("hq, hkv, tq, tkv, d, blocks, span", [
    (4, 2, 300, 300, 128, (0b01, [120]), 0),          # prefix-LM over a causal tail
    (2, 2, 257, 257, 64, (0b101, [70, 190]), 0),      # causal / full / causal
    (2, 1, 200, 260, 256, (0b010, [50, 130]), 60),    # full / causal / full, Tq < Tkv, window
    (2, 2, 64, 1000, 64, (0b10, [20]), 0),            # one query tile, key split and merge
])
def test_attention_block_mask(gpu, hq, hkv, tq, tkv, d, blocks, span):
    rng = np.random.default_rng(tq + d)
    q = draw((1, hq, tq, d), rng, np.float16)
    k = draw((1, hkv, tkv, d), rng, np.float16)
    v = draw((1, hkv, tkv, d), rng, np.float16)
    D = gpu.DeviceArray.from_numpy
    out = gpu.DeviceArray((1, hq, tq, d), np.float32)
    print(f"attention blocks={blocks} hq={hq} hkv={hkv} tq={tq} tkv={tkv} d={d} span={span}", flush=True)
    got = gpu.attention(out, D(q), D(k), D(v), blocks=blocks, span=span).numpy()
    want = oracle.attention(q, k, v, blocks=blocks, span=span, out_dtype=np.float32)
    assert_close(got, want, FP16)


def test_attention_rejects(gpu):
    """fp32 inputs and head dims other than 64/128/256 are refused."""
    import ctypes
    D = gpu.DeviceArray
    a = gpu.attention_args(D((1, 1, 8, 64), np.float32), D((1, 1, 8, 64), np.float32), D((1, 1, 8, 64), np.float32),
                           D((1, 1, 8, 64), np.float32))
    assert gpu.lib().vai_attention_launch(ctypes.byref(a), None) == 1003
    a = gpu.attention_args(D((1, 1, 8, 96), np.float32), D((1, 1, 8, 96), np.float16), D((1, 1, 8, 96), np.float16),
                           D((1, 1, 8, 96), np.float16))
    assert gpu.lib().vai_attention_launch(ctypes.byref(a), None) == 1005


def test_attention_workspace(gpu):
    """The key-range split asks for a workspace (config 4's shape: its 64
    query tiles of 128 rows leave CUs idle) and refuses to run without one;
    a shape whose query tiles fill the GPU (32 heads x 8 tiles) needs none."""
    import ctypes
    D = gpu.DeviceArray
    q = D((8, 1024, 256), np.float16)
    a = gpu.attention_args(D((8, 1024, 256), np.float32), q, q, q, causal=True)
    need = gpu.lib().vai_attention_workspace_size(ctypes.byref(a))
    assert need > 0
    assert gpu.lib().vai_attention_launch(ctypes.byref(a), None) == 1004
    q2 = D((32, 1024, 64), np.float16)
    a2 = gpu.attention_args(D((32, 1024, 64), np.float32), q2, q2, q2, causal=True)
    assert gpu.lib().vai_attention_workspace_size(ctypes.byref(a2)) == 0
