"""vai_linear_launch_noalloc against vai_linear_launch through the C ABI: the
same kernels on the same inputs, so outputs must be bit-identical; two calls in
a row (the second smaller) share the library's scratch array."""
import ctypes

import numpy as np
import pytest

from helpers import draw, normal


def _launch(gpu, fn, out, x, w, packed=None, workspace=None, **kw):
    a = gpu.linear_args(out, x, w, workspace=workspace, **kw)
    if packed is not None:
        a.packed_weight = packed.ptr
    gpu.check(fn(ctypes.byref(a), None), fn.__name__)
    gpu.check(gpu.lib().vai_stream_sync(None), "sync")
    return out.numpy()


def _case(gpu, m, k, n, packed, **kw):
    rng = np.random.default_rng(m + n)
    D = gpu.DeviceArray.from_numpy
    w = D(draw(normal((n, k), 0.02), rng, np.float16))
    x = D(draw((m, k), rng, np.float16))
    cols = n // 2 if kw.get("gated") else n
    a = gpu.linear_args(gpu.DeviceArray((m, cols), np.float32), x, w, **kw)
    pk = None
    if packed:
        pk = gpu.linear_pack_weight(a)
        a.packed_weight = pk.ptr
    need = gpu.linear_workspace_size(a)
    assert need > 0, "each case must use the workspace"
    ws = gpu.DeviceArray((need,), np.uint8)
    want = _launch(gpu, gpu.lib().vai_linear_launch, gpu.DeviceArray((m, cols), np.float32), x, w, pk, ws, **kw)
    out = gpu.DeviceArray((m, cols), np.float32)
    out.fill_(0xFF)   # NaNs: every output must be written
    got = _launch(gpu, gpu.lib().vai_linear_launch_noalloc, out, x, w, pk, **kw)
    return got, want, gpu.linear_plan(a)


@pytest.mark.gpu
def test_noalloc_matches_linear_launch(gpu):
    # 1) the FFN down projection: packed weight, 2 K splits, 48 MiB of partials
    got, want, plan = _case(gpu, 2048, 8192, 3072, True)
    print("case 1", plan, flush=True)
    assert plan == ("tile_f16_256x256_packed", 2)
    np.testing.assert_array_equal(got, want)
    # 2) smaller, forced split-K on the generic tile (fewer, shorter planes)
    got, want, plan = _case(gpu, 300, 1024, 1000, False, split_size=256, epi="GELU")
    print("case 2", plan, flush=True)
    assert plan[1] == 4
    np.testing.assert_array_equal(got, want)
    # 3) smaller still: the M <= 8 gated GEMV, whose intermediate uses the scratch
    got, want, plan = _case(gpu, 4, 512, 2 * 640, False, gated=True, gate_epi="SILU")
    print("case 3", plan, flush=True)
    assert plan[0].endswith("+gate")
    np.testing.assert_array_equal(got, want)


@pytest.mark.gpu
def test_noalloc_refuses_oversize(gpu):
    D = gpu.DeviceArray
    a = gpu.linear_args(D((4096, 8192), np.float32), D((4096, 1024), np.float16), D((8192, 1024), np.float16),
                        split_size=256)
    assert gpu.lib().vai_linear_launch_noalloc(ctypes.byref(a), None) == 1004
