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
