"""CPU-side checks of the C ABI: the library loads and exports every symbol
include/vai_amd.h declares; argument checks reject bad input without a GPU."""
import ctypes
import os
import re

import numpy as np

from vai_amd import _capi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "vai_amd.h")).read()
    return sorted(set(re.findall(r"^[a-z_ ]+\**\s*\b(vai_[a-z0-9_]+)\(", text, re.M)))


def test_header_and_binding_agree():
    assert sorted(_capi.EXPORTS) == declared_symbols()


def test_library_exports_every_declared_symbol():
    lib = _capi.lib()
    for name in declared_symbols():
        assert hasattr(lib, name), name


def test_argument_checks_need_no_gpu():
    lib = _capi.lib()
    a = _capi.LinearArgs()
    assert lib.vai_linear_launch(ctypes.byref(a), None) == 1001   # null pointers
    a.out = a.inp = a.weight = 16
    assert lib.vai_linear_launch(ctypes.byref(a), None) == 1002   # zero sizes
    a.M, a.N, a.K = 4, 8, 8
    a.o_dtype = 7
    assert lib.vai_linear_launch(ctypes.byref(a), None) == 1003
    a.o_dtype = 0
    a.epilogue = 9
    assert lib.vai_linear_launch(ctypes.byref(a), None) == 1001
    a.epilogue = 0
    a.gated, a.N = 1, 7
    assert lib.vai_linear_launch(ctypes.byref(a), None) == 1002   # odd 2H
    assert lib.vai_linear_launch_noalloc(ctypes.byref(a), None) == 1002
    # a split-K launch whose partials (4 x 4096 x 8192 fp32) exceed the
    # no-allocation scratch is refused before anything reaches a GPU
    a.gated, a.M, a.N, a.K, a.split_size = 0, 4096, 8192, 1024, 256
    assert _capi.linear_workspace_size(a) == 4 * 4096 * 8192 * 4
    assert lib.vai_linear_launch_noalloc(ctypes.byref(a), None) == 1004
    c = _capi.Conv2dArgs()
    c.out = c.inp = c.weight = 16
    c.batch = c.ci = c.co = c.hi = c.wi = c.stride = 1
    c.kernel = 2
    assert lib.vai_conv2d_launch(ctypes.byref(c), None) == 1002   # even kernel
    c.kernel, c.w_dtype, c.i_dtype = 3, 0, 1
    assert lib.vai_conv2d_launch(ctypes.byref(c), None) == 1003   # fp16 input needs fp16 weights
    s = _capi.AttnScoresArgs()
    s.scores = s.q = s.k = 16
    s.batch, s.hq, s.hkv, s.tq, s.tkv, s.head_dim = 1, 3, 2, 4, 4, 8
    assert lib.vai_attn_scores_launch(ctypes.byref(s), None) == 1002   # Hq % Hkv


def test_plans():
    """Kernel selection (the selectLinearTile replacement) by shape and dtype."""
    def plan(m, n, k, idt=np.float16, wdt=np.float16, **kw):
        a = _capi.LinearArgs()
        a.out = a.inp = a.weight = 256
        a.M, a.N, a.K = m, n, k
        a.o_dtype, a.i_dtype, a.w_dtype = 0, _capi.dtype_code(idt), _capi.dtype_code(wdt)
        a.scalar_scale = 1.0
        for key, v in kw.items():
            setattr(a, key, v)
        return _capi.linear_plan(a)
    assert plan(1, 8192, 2048) == ("slab", 1)
    assert plan(8, 8192, 2048)[0] == "slab_mfma"
    assert plan(8, 8192, 2048, np.float32, np.float16)[0] == "slab"
    assert plan(8, 8192, 2047)[0] == "slab_scalar"
    assert plan(9, 8192, 2048)[0].startswith("tile_f16")
    assert plan(128, 3072, 768, np.float32, np.float32)[0].startswith("tile_f32")
    name, splits = plan(16, 64, 256, np.float32, np.float32, split_size=64)
    assert splits == 4
    name, splits = plan(2048, 16384, 3072, gated=1, gate_epilogue=4)
    assert name.endswith("_gated") and splits == 1


def test_acc16_auto_split_follows_the_reference():
    """An fp16-accumulating Linear with splitSize 0 splits K as the reference's
    ggmlGuessSplitCount does for its scalar tile (linear.h:600-632): each
    split starts its own fp16 chain, so the count changes the sums. Counts
    below are worked by hand from that rule for 256 compute units."""
    def plan(m, n, k, split_size=0):
        a = _capi.LinearArgs()
        a.out = a.inp = a.weight = 256
        a.M, a.N, a.K = m, n, k
        a.o_dtype, a.i_dtype, a.w_dtype = 0, 1, 1
        a.acc_dtype = 1
        a.scalar_scale = 1.0
        a.split_size = split_size
        return _capi.linear_plan(a)
    # 64x64: the M tier (64x64 tiles), 1 tile <= 128 -> min(256, 8) = 8 spans of 512
    assert plan(64, 64, 4096)[1] == 8
    # K < 2048: never split
    assert plan(64, 64, 2047)[1] == 1
    # 256x256 (L tier, 128x128): 4 tiles -> 8 splits; K = 2048: spans of 256, 8 * 256 - 256 < 2048
    assert plan(256, 256, 2048)[1] == 8
    # K = 2304: 8, 7 and 6 splits all round to spans of 512 that leave the last split empty
    # (7, 6, 5 x 512 >= 2304); 5 splits: span 512, 4 x 512 = 2048 < 2304
    assert plan(256, 256, 2304)[1] == 5
    # 2048 x 2048: 256 tiles of 128 > 256 * 2 / 3: no split
    assert plan(2048, 2048, 4096)[1] == 1
    # 1536 x 1536: 144 tiles, > 128 but <= 170: 3 splits
    assert plan(1536, 1536, 4096)[1] == 3
    # N below the tile: no split (ggml's N < wgN gate); M, N <= 32: S tier 32x32
    assert plan(64, 16, 4096)[1] == 1
    # an explicit span wins
    assert plan(64, 64, 4096, split_size=1024)[1] == 4


def test_attention_argument_checks_need_no_gpu():
    """bf16-like dtype codes and zero sizes are refused; any head dim passes
    the checks (the plain kernel takes what the flash kernel cannot)."""
    lib = _capi.lib()
    a = _capi.AttentionArgs()
    a.out = a.q = a.k = a.v = 256
    a.batch, a.hq, a.hkv, a.tq, a.tkv, a.head_dim = 1, 2, 1, 4, 4, 72
    a.q_dtype, a.kv_dtype, a.o_dtype = 0, 7, 0
    assert lib.vai_attention_launch(ctypes.byref(a), None) == 1003
    a.kv_dtype = 0
    a.head_dim = 0
    assert lib.vai_attention_launch(ctypes.byref(a), None) == 1002
    # fp32 K / V at a flash head dim need fp16 copies: 2 x (4 x 72) x 2 = 1152 bytes, rounded to 1280
    a.head_dim = 72
    assert lib.vai_attention_workspace_size(ctypes.byref(a)) == 1280
    # fp16 K / V at head dim 20 (not a multiple of 8): the plain kernel, no workspace
    a.head_dim, a.kv_dtype = 20, 1
    assert lib.vai_attention_workspace_size(ctypes.byref(a)) == 0


def test_attention_kv_cache_argument_checks_need_no_gpu():
    """The KV cache fields (attention.h:216-245, 959-1023): a cache needs its
    planes and counter, fp32 / fp16, one sequence, a ring of whole 64-row
    tiles, and room for the new rows; K / V may be absent (Tkv = 0) only with
    a cache. The workspace of an fp32 cache at a flash head dim covers fp16
    copies of the whole planes (the count is only known when the kernels run)."""
    lib = _capi.lib()
    a = _capi.AttentionArgs()
    a.out = a.q = a.k = a.v = 256
    a.batch, a.hq, a.hkv, a.tq, a.tkv, a.head_dim = 1, 4, 2, 1, 1, 64
    a.q_dtype, a.kv_dtype, a.o_dtype = 1, 1, 0
    a.cache_size, a.cache_dtype = 128, 1
    assert lib.vai_attention_launch(ctypes.byref(a), None) == 1001   # no planes, no counter
    a.k_cache = a.v_cache = a.cache_count = 512
    a.cache_dtype = 5
    assert lib.vai_attention_launch(ctypes.byref(a), None) == 1003
    a.cache_dtype = 0
    a.batch = 2
    assert lib.vai_attention_launch(ctypes.byref(a), None) == 1002   # one counter, one sequence
    a.batch, a.cache_ring = 1, 1
    assert lib.vai_attention_workspace_size(ctypes.byref(a)) > 0       # a ring of 128 rows is two tiles: fine ...
    a.cache_size = 100
    assert lib.vai_attention_launch(ctypes.byref(a), None) == 1002   # ... 100 is not a whole number of tiles
    a.cache_size, a.cache_ring, a.tkv = 128, 0, 200
    assert lib.vai_attention_launch(ctypes.byref(a), None) == 1002   # 200 new rows do not fit 128
    # fp32 planes [2, 128, 64] at a flash head dim: fp16 copies, 2 x 2 x 128 x 64 x 2 bytes
    a.tkv = 1
    assert lib.vai_attention_workspace_size(ctypes.byref(a)) % 256 == 0
    assert lib.vai_attention_workspace_size(ctypes.byref(a)) >= 2 * 2 * 128 * 64 * 2
    # K / V absent: fine with a cache (Tkv = 0), refused without one
    a.k = a.v = None
    a.tkv = 0
    assert lib.vai_attention_workspace_size(ctypes.byref(a)) > 0
    a.cache_size = 0
    assert lib.vai_attention_launch(ctypes.byref(a), None) == 1001
