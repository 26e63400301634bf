"""Attention forward through the C ABI vs the oracle's float64 softmax(S) V.
The reference's Attention node (/root/reference/vai/nodes/attention.h:77-129,
979-1304, shaders/attention-fa.comp, attention.comp): O token-major
[B, Tq, Hq, D], no mask unless one is set, Q and K / V each fp32 or fp16, any
head dim; the causal / sliding-window / block rule of common/causal_mask.h:
25-42, GQA, Tq != Tkv, tails. The flash kernel computes Q.K^T and P.V on
fp16 operands (fp32 Q / K / V rounded to fp16, P rounded to fp16, as the
reference's f16-staged tiles and fp16 P.V operand), so it is held to the
fp16 tier; the plain fp32 kernel (head dims the flash kernel does not take)
to a tighter one.
"""
import ctypes

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
    out = gpu.DeviceArray((b, tq, hq, d), odt)
    print(f"attention b={b} hq={hq} hkv={hkv} tq={tq} tkv={tkv} d={d} causal={causal} span={span}", flush=True)
    got = gpu.attention(out, D(q), D(k), D(v), causal=causal, span=span).numpy().astype(np.float32)
    want = oracle.attention(q, k, v, causal=causal, span=span, out_dtype=np.float32)
    assert_close(got, want, FP16)
    if causal and tq > tkv:
        np.testing.assert_array_equal(got[:, : tq - tkv], 0.0)


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
    out = gpu.DeviceArray((1, tq, hq, d), np.float32)
    print(f"attention blocks={blocks} hq={hq} hkv={hkv} tq={tq} tkv={tkv} d={d} span={span}", flush=True)
    got = gpu.attention(out, D(q), D(k), D(v), blocks=blocks, span=span).numpy()
    want = oracle.attention(q, k, v, blocks=blocks, span=span, out_dtype=np.float32)
    assert_close(got, want, FP16)


NAIVE = (1e-4, 1e-5)


@pytest.mark.parametrize("b, hq, hkv, tq, tkv, d, qdt, kvdt, odt, causal", [
    (1, 16, 16, 729, 729, 72, np.float32, np.float32, np.float32, False),   # SigLIP's encoder attention (Dh 72)
    (2, 4, 2, 100, 100, 72, np.float16, np.float16, np.float16, True),      # Dh 72 in fp16, GQA, causal
    (1, 8, 2, 130, 300, 128, np.float32, np.float16, np.float32, True),     # fp32 Q over fp16 K / V (Linear -> cache dtype)
    (1, 4, 4, 64, 1000, 64, np.float16, np.float32, np.float16, False),     # fp32 K / V: fp16 copies, key split
    (1, 2, 1, 50, 50, 16, np.float32, np.float32, np.float32, True),        # smallest flash head dim
    (1, 2, 2, 70, 90, 200, np.float32, np.float16, np.float32, False),      # Dh 200: padded to 256
    (1, 3, 3, 40, 40, 40, np.float16, np.float16, np.float32, True),        # Dh 40: padded to 64
])
def test_attention_dtypes_and_head_dims(gpu, b, hq, hkv, tq, tkv, d, qdt, kvdt, odt, causal):
    rng = np.random.default_rng(d + tq)
    q = draw((b, hq, tq, d), rng, qdt)
    k = draw((b, hkv, tkv, d), rng, kvdt)
    v = draw((b, hkv, tkv, d), rng, kvdt)
    D = gpu.DeviceArray.from_numpy
    out = gpu.DeviceArray((b, tq, hq, d), odt)
    print(f"attention b={b} hq={hq} hkv={hkv} tq={tq} tkv={tkv} d={d} q={qdt.__name__} kv={kvdt.__name__}",
          flush=True)
    got = gpu.attention(out, D(q), D(k), D(v), causal=causal).numpy().astype(np.float32)
    assert_close(got, oracle.attention(q, k, v, causal=causal, out_dtype=np.float32), FP16)


@pytest.mark.parametrize("b, hq, hkv, tq, tkv, d, qdt, kvdt, causal, span", [
    (1, 2, 1, 33, 47, 20, np.float32, np.float32, True, 0),     # Dh % 8 != 0: the plain kernel
    (2, 2, 2, 17, 17, 8, np.float16, np.float16, False, 0),     # Dh < 16
    (1, 2, 2, 40, 300, 300, np.float32, np.float16, True, 100),  # Dh > 256, window, more keys than a tile
    (1, 1, 1, 9, 3, 12, np.float16, np.float32, True, 0),       # queries with no visible key give 0
])
def test_attention_plain_kernel(gpu, b, hq, hkv, tq, tkv, d, qdt, kvdt, causal, span):
    rng = np.random.default_rng(d)
    q = draw((b, hq, tq, d), rng, qdt)
    k = draw((b, hkv, tkv, d), rng, kvdt)
    v = draw((b, hkv, tkv, d), rng, kvdt)
    D = gpu.DeviceArray.from_numpy
    out = gpu.DeviceArray((b, tq, hq, d), np.float32)
    a = gpu.attention_args(out, D(q), D(k), D(v), causal=causal, span=span)
    assert gpu.lib().vai_attention_workspace_size(ctypes.byref(a)) == 0
    print(f"attention plain b={b} hq={hq} tq={tq} tkv={tkv} d={d} span={span}", flush=True)
    got = gpu.attention(out, D(q), D(k), D(v), causal=causal, span=span).numpy()
    assert_close(got, oracle.attention(q, k, v, causal=causal, span=span, out_dtype=np.float32), NAIVE)


def test_attention_layout_and_no_mask_default(gpu):
    """The output is token-major: the independent head-major float64 result
    transposed by numpy (Tq, Hq and D all distinct). Without a mask argument
    every query attends every key (attention.h:129), on both kernels."""
    rng = np.random.default_rng(21)
    for d in (72, 36):
        q = draw((2, 3, 40, d), rng, np.float32)
        k = draw((2, 3, 56, d), rng, np.float32)
        v = draw((2, 3, 56, d), rng, np.float32)
        s = np.einsum("bhid,bhjd->bhij", q.astype(np.float64), k.astype(np.float64)) / np.sqrt(d)
        p = np.exp(s - s.max(-1, keepdims=True))
        head_major = np.einsum("bhij,bhjd->bhid", p / p.sum(-1, keepdims=True), v.astype(np.float64))
        D = gpu.DeviceArray.from_numpy
        print(f"attention layout d={d}", flush=True)
        got = gpu.attention(gpu.DeviceArray((2, 40, 3, d), np.float32), D(q), D(k), D(v)).numpy()
        assert_close(got, np.transpose(head_major, (0, 2, 1, 3)), FP16)


def test_attention_rejects(gpu):
    """A dtype other than fp32 / fp16 and a zero head dim are refused."""
    D = gpu.DeviceArray
    a = gpu.attention_args(D((1, 1, 8, 64), np.float32), D((1, 1, 8, 64), np.float32), D((1, 1, 8, 64), np.float32),
                           D((1, 1, 8, 64), np.float32))
    a.kv_dtype = 5
    assert gpu.lib().vai_attention_launch(ctypes.byref(a), None) == 1003
    a.kv_dtype, a.head_dim = 0, 0
    assert gpu.lib().vai_attention_launch(ctypes.byref(a), None) == 1002


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


# ---- the KV cache (attention.h:108-140, 1003-1023; attention-fa.comp:
# 137-146, 344-478): append, then attend positions [0, count + Tkv) ----

def _cache_planes(rng, hkv, size, d, count, ring, dtype):
    """Cache planes whose rows for positions < count hold data; every other
    row holds NaN bytes, so that a read past the live keys would show."""
    kc = np.full((hkv, size, d), np.nan, dtype)
    vc = kc.copy()
    for p in range(max(0, count - size) if ring else 0, count):
        r = p % size if ring else p
        kc[:, r] = draw((hkv, d), rng, dtype)
        vc[:, r] = draw((hkv, d), rng, dtype)
    return kc, vc


@pytest.mark.parametrize("d, hq, hkv, tq, tkv, count, size, ring, causal, span, cdt, kdt, qdt", [
    (128, 4, 2, 200, 200, 0, 512, False, True, 0, np.float16, np.float16, np.float16),    # prefill, empty cache
    (128, 4, 2, 1, 1, 300, 512, False, True, 0, np.float16, np.float16, np.float16),      # decode
    (256, 8, 8, 1, 1, 1000, 1024, False, True, 0, np.float16, np.float16, np.float16),    # decode, long cache
    (128, 4, 4, 48, 48, 100, 256, False, True, 0, np.float16, np.float16, np.float16),    # a prompt chunk
    (64, 4, 2, 1, 1, 700, 256, True, True, 200, np.float16, np.float16, np.float16),      # ring, sliding window
    (64, 4, 2, 16, 16, 600, 256, True, True, 128, np.float16, np.float16, np.float16),    # ring, chunk
    (128, 4, 2, 3, 0, 50, 128, False, False, 0, np.float16, np.float16, np.float16),      # cache alone
    (64, 2, 1, 5, 5, 77, 128, False, True, 0, np.float32, np.float32, np.float32),        # fp32 cache and inputs
    (64, 8, 2, 1, 1, 513, 1024, False, True, 0, np.float16, np.float32, np.float32),      # fp32 K / V into fp16
    (20, 2, 2, 2, 2, 30, 64, False, True, 0, np.float16, np.float16, np.float16),         # plain kernel
])
def test_attention_kv_cache(gpu, d, hq, hkv, tq, tkv, count, size, ring, causal, span, cdt, kdt, qdt):
    rng = np.random.default_rng(count + tq)
    kc, vc = _cache_planes(rng, hkv, size, d, count, ring, cdt)
    q = draw((1, hq, tq, d), rng, qdt)
    k = draw((1, hkv, tkv, d), rng, kdt) if tkv else None
    v = draw((1, hkv, tkv, d), rng, kdt) if tkv else None
    D = gpu.DeviceArray.from_numpy
    dkc, dvc = D(kc), D(vc)
    cnt = D(np.array([count], np.uint32))
    out = gpu.DeviceArray((1, tq, hq, d), np.float32)
    print(f"kv cache d={d} hq={hq} hkv={hkv} tq={tq} tkv={tkv} count={count} size={size} ring={ring}", flush=True)
    got = gpu.attention(out, D(q), None if k is None else D(k), None if v is None else D(v), causal=causal, span=span,
                        cache=(dkc, dvc, cnt, ring)).numpy()
    want, wkc, wvc = oracle.attention_cached(q[0], k, v, kc, vc, count, ring=ring, causal=causal, span=span)
    assert_close(got[0], want, NAIVE if d % 8 else FP16)
    # the appended rows hold the new K / V in the cache dtype, every other row is as it was
    gkc, gvc = dkc.numpy(), dvc.numpy()
    np.testing.assert_array_equal(gkc, wkc)
    np.testing.assert_array_equal(gvc, wvc)
    assert int(cnt.numpy()[0]) == count   # the caller advances the count


@pytest.mark.parametrize("d, tq, count, size, ring, blocks, span", [
    (128, 96, 200, 512, False, (0b101, [24, 72]), 0),    # causal / full (an image) / causal chunk after cached text
    (64, 40, 300, 256, True, (0b01, [16]), 128),         # a full prefix block in a ring, sliding window
    (256, 1, 500, 512, False, (0b10, [1]), 0),           # decode step whose block list has one entry
])
def test_attention_kv_cache_block_mask(gpu, d, tq, count, size, ring, blocks, span):
    """The block masks of common/causal_mask.h over a cached chunk: blocks
    index the call's new tokens (keyEnd = count + newTokenEnd(t) + Tkv -
    Tq), the cached positions stay visible to every query, and the window
    counts global positions."""
    rng = np.random.default_rng(count + tq + d)
    hq, hkv = 4, 2
    kc, vc = _cache_planes(rng, hkv, size, d, count, ring, np.float16)
    q = draw((1, hq, tq, d), rng, np.float16)
    k = draw((1, hkv, tq, d), rng, np.float16)
    v = draw((1, hkv, tq, d), rng, np.float16)
    D = gpu.DeviceArray.from_numpy
    dkc, dvc = D(kc), D(vc)
    out = gpu.DeviceArray((1, tq, hq, d), np.float32)
    print(f"kv cache blocks={blocks} d={d} tq={tq} count={count} size={size} ring={ring} span={span}", flush=True)
    got = gpu.attention(out, D(q), D(k), D(v), blocks=blocks, span=span,
                        cache=(dkc, dvc, D(np.array([count], np.uint32)), ring)).numpy()
    want, wkc, _ = oracle.attention_cached(q[0], k, v, kc, vc, count, ring=ring, span=span, blocks=blocks)
    assert_close(got[0], want, FP16)
    np.testing.assert_array_equal(dkc.numpy(), wkc)


def test_attention_kv_cache_ring_longer_call(gpu):
    """A ring call with more new tokens than rows: each row ends up holding the
    newest position that maps to it (the call's last `size` tokens; no race
    between the tokens that share a row), and a query whose window lies in
    the live ring reads them."""
    rng = np.random.default_rng(41)
    d, hq, hkv, tq, count, size, span = 64, 2, 1, 100, 10, 64, 32
    kc, vc = _cache_planes(rng, hkv, size, d, count, True, np.float16)
    q = draw((1, hq, tq, d), rng, np.float16)
    k = draw((1, hkv, tq, d), rng, np.float16)
    v = draw((1, hkv, tq, d), rng, np.float16)
    D = gpu.DeviceArray.from_numpy
    dkc, dvc = D(kc), D(vc)
    out = gpu.DeviceArray((1, tq, hq, d), np.float32)
    got = gpu.attention(out, D(q), D(k), D(v), causal=True, span=span,
                        cache=(dkc, dvc, D(np.array([count], np.uint32)), True)).numpy()
    want, wkc, wvc = oracle.attention_cached(q[0], k, v, kc, vc, count, ring=True, causal=True, span=span)
    np.testing.assert_array_equal(dkc.numpy(), wkc)
    np.testing.assert_array_equal(dvc.numpy(), wvc)
    # queries from position count + tq - size + span - 1 on see only live rows
    t0 = tq - size + span - 1
    assert_close(got[0, t0:], want[t0:], FP16)


def test_attention_kv_cache_decode_steps(gpu):
    """Decode as a model runs it: one token per call, the count advanced on
    the device between calls; each step matches the reference's formulas over
    the cache the earlier steps left."""
    rng = np.random.default_rng(5)
    hq, hkv, d, size, count = 8, 4, 128, 256, 40
    kc, vc = _cache_planes(rng, hkv, size, d, count, False, np.float16)
    D = gpu.DeviceArray.from_numpy
    dkc, dvc = D(kc), D(vc)
    cnt = gpu.DeviceArray((1,), np.uint32)
    for step in range(3):
        gpu.lib().vai_memcpy_h2d(cnt.ptr, np.array([count], np.uint32).ctypes.data, 4, None)
        q = draw((1, hq, 1, d), rng, np.float16)
        k = draw((1, hkv, 1, d), rng, np.float16)
        v = draw((1, hkv, 1, d), rng, np.float16)
        out = gpu.DeviceArray((1, 1, hq, d), np.float32)
        got = gpu.attention(out, D(q), D(k), D(v), causal=True, cache=(dkc, dvc, cnt, False)).numpy()
        want, kc, vc = oracle.attention_cached(q[0], k, v, kc, vc, count, causal=True)
        assert_close(got[0], want, FP16)
        count += 1
    np.testing.assert_array_equal(dkc.numpy(), kc)


def test_attention_kv_cache_rejects(gpu):
    D = gpu.DeviceArray
    q, k = D((1, 4, 2, 64), np.float16), D((1, 2, 2, 64), np.float16)
    kc, cnt = D((2, 100, 64), np.float16), D((1,), np.uint32)
    out = D((1, 2, 4, 64), np.float32)
    a = gpu.attention_args(out, q, k, k, cache=(kc, kc, cnt, True))      # ring of 100 rows: not a multiple of 64
    assert gpu.lib().vai_attention_launch(ctypes.byref(a), None) == 1002
    q2 = D((2, 4, 2, 64), np.float16)
    k2 = D((2, 2, 2, 64), np.float16)
    out2 = D((2, 2, 4, 64), np.float32)
    a = gpu.attention_args(out2, q2, k2, k2, cache=(kc, kc, cnt, False))  # one counter: batch 1 only
    assert gpu.lib().vai_attention_launch(ctypes.byref(a), None) == 1002
