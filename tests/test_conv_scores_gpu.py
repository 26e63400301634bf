"""Convolution (implicit GEMM) and attention scores through the C ABI on the
MI355X vs the oracle.

Conv cases follow /root/reference/python/tests/nodes/test_convolution.py:
12-87 (k1s1, k3s1 at 12^2 and 28^2, k3s2, k5s1, scale, residual), plus
BASELINE config 5. Scores: BASELINE config 4 plus GQA, Tq != Tkv and the
sliding-window span of common/causal_mask.h.
"""
import numpy as np
import pytest

from helpers import FP16, FP32, TRANS, assert_close, draw, normal, uniform
from oracle import oracle

pytestmark = pytest.mark.gpu


def run_conv(capi, x, w, b=None, s=None, r=None, out_dtype=np.float32, **kw):
    d = capi.DeviceArray.from_numpy
    dx, dw = d(x), d(w)
    db = d(b) if b is not None else None
    ds = d(s) if s is not None else None
    dr = d(r) if r is not None else None
    Co, _, ks, _ = w.shape
    stride = kw.get("stride", 1)
    Hi, Wi = x.shape[-2:]
    out = capi.DeviceArray(x.shape[:-3] + (Co, (Hi - 1) // stride + 1, (Wi - 1) // stride + 1), out_dtype)
    capi.conv2d(out, dx, dw, db, ds, dr, **kw)
    return out.numpy()


@pytest.mark.parametrize("ci, co, ks, stride, hw, batch, epi, dt", [
    (16, 32, 1, 1, 12, 1, "NONE", np.float32),
    (8, 16, 3, 1, 12, 1, "RELU", np.float32),
    (8, 16, 3, 1, 28, 2, "SILU", np.float32),
    (8, 16, 3, 2, 13, 1, "NONE", np.float32),
    (4, 8, 5, 1, 11, 1, "GELU", np.float32),
    (32, 64, 3, 1, 20, 1, "SILU", np.float16),
    (24, 40, 3, 2, 17, 3, "SIGMOID", np.float16),
    (3, 16, 7, 2, 23, 1, "RELU", np.float16),
    # 64-channel workgroups (more 32-channel ones than CUs) with output-channel tails:
    (32, 96, 3, 2, 192, 1, "SILU", np.float16),    # 3x3 stride 2, vector epilogue
    (64, 80, 1, 1, 100, 1, "RELU", np.float16),    # pointwise
    (16, 48, 3, 2, 197, 2, "NONE", np.float16),    # odd output row: scalar epilogue, batch 2
])
def test_conv(gpu, ci, co, ks, stride, hw, batch, epi, dt):
    rng = np.random.default_rng(0)
    w = draw(normal((co, ci, ks, ks), 1.0 / np.sqrt(ci * ks * ks)), rng, dt)
    b = draw(normal((co,), 0.1), rng, dt)
    x = draw((batch, ci, hw, hw), rng, dt)
    got = run_conv(gpu, x, w, b, stride=stride, epi=epi)
    want = oracle.conv2d(x, w, b, stride=stride, epi=epi)
    assert_close(got, want, TRANS if dt == np.float32 else FP16)


@pytest.mark.parametrize("ci, co, ks, stride, hw", [(256, 128, 1, 1, 40), (128, 256, 3, 2, 80)])
def test_conv_yolox_plans(gpu, ci, co, ks, stride, hw):
    """The other YOLOX-s conv plans at their real shapes: a CSP pointwise
    conv (conv-k1s1-gemm.comp) and the 3x3 stride-2 downsample
    (conv-k3s2-gemm.comp), fp16, bias + SiLU, packed weight."""
    rng = np.random.default_rng(5)
    w = draw(normal((co, ci, ks, ks), 0.03), rng, np.float16)
    b = draw(normal((co,), 0.02), rng, np.float16)
    x = draw(uniform((1, ci, hw, hw), -1, 1), rng, np.float16)
    D = gpu.DeviceArray.from_numpy
    ho = (hw - 1) // stride + 1
    out = gpu.DeviceArray((1, co, ho, ho), np.float32)
    a = gpu.conv2d_args(out, D(x), D(w), D(b), stride=stride, epi="SILU")
    packed = gpu.conv2d_pack_weight(a)
    got = gpu.conv2d(out, D(x), D(w), D(b), stride=stride, epi="SILU", packed=packed).numpy()
    assert_close(got, oracle.conv2d(x, w, b, stride=stride, epi="SILU"), FP16)


@pytest.mark.parametrize("order", [0, 1])
def test_conv_scale_residual(gpu, order):
    rng = np.random.default_rng(0)
    ci, co, hw = 8, 16, 14
    w = draw(normal((co, ci, 3, 3), 0.2), rng)
    b = draw((co,), rng)
    s = draw(uniform((co,), 0.5, 1.5), rng)
    x = draw((1, ci, hw, hw), rng)
    r = draw((1, co, hw, hw), rng)
    got = run_conv(gpu, x, w, b, s, r, epi="RELU", order=order)
    want = oracle.conv2d(x, w, b, s, r, epi="RELU", order=order)
    assert_close(got, want, TRANS)


def test_conv_mixed_f32_input_f16_weight(gpu):
    rng = np.random.default_rng(0)
    w = draw(normal((16, 8, 3, 3), 0.1), rng, np.float16)
    x = draw((1, 8, 10, 10), rng)
    got = run_conv(gpu, x, w)
    assert_close(got, oracle.conv2d(x, w), FP16)


def test_config5_yolox_conv(gpu):
    rng = np.random.default_rng(0)
    w = draw(normal((128, 128, 3, 3), 0.03), rng, np.float16)
    b = draw(normal((128,), 0.02), rng, np.float16)
    x = draw(uniform((1, 128, 80, 80), -1.0, 1.0), rng, np.float16)
    got = run_conv(gpu, x, w, b, epi="SILU")
    want = oracle.conv2d(x, w, b, epi="SILU")
    assert_close(got, want, TRANS)


@pytest.mark.parametrize("ci, co, hi, wi, batch, epi", [
    (40, 48, 16, 16, 2, "SILU"),      # channels and output channels past a block, batch 2
    (64, 32, 20, 32, 1, "RELU"),      # two column fragments, H != W
    (160, 32, 9, 48, 1, "SIGMOID"),   # five channel blocks: a wave takes two
    (128, 64, 6, 128, 1, "NONE"),     # eight column fragments (the widest row)
    (3, 16, 5, 16, 1, "GELU"),        # three input channels
    (48, 80, 96, 96, 1, "SILU"),      # 64-channel workgroups (288 32-channel ones > 256 CUs), output-channel tail
    (128, 128, 40, 80, 2, "NONE"),    # 64-channel workgroups over a batch of 2
])
def test_conv3_lds_transpose(gpu, ci, co, hi, wi, batch, epi):
    """The 3x3 stride-1 plan for fp16 rows of 16 NF columns (input copied to
    LDS as NCHW, transposed by the LDS read, kw taps combined by a column
    shift): borders, channel and output-channel tails, several channel
    blocks per wave, one to eight column fragments."""
    rng = np.random.default_rng(ci + wi)
    w = draw(normal((co, ci, 3, 3), 1.0 / np.sqrt(ci * 9)), rng, np.float16)
    b = draw(normal((co,), 0.1), rng, np.float16)
    x = draw((batch, ci, hi, wi), rng, np.float16)
    print(f"conv3 ci={ci} co={co} hi={hi} wi={wi} batch={batch}", flush=True)
    got = run_conv(gpu, x, w, b, epi=epi)
    assert_close(got, oracle.conv2d(x, w, b, epi=epi), FP16)


@pytest.mark.parametrize("order", [0, 1])
def test_conv3_wide_scale_residual(gpu, order):
    """Scale, fp16 residual and fp16 output with 64-channel workgroups (2 x 96
    rows x 2 channel blocks of 32 would be 384 workgroups on 256 CUs)."""
    rng = np.random.default_rng(10 + order)
    ci, co, hw = 32, 64, 96
    w = draw(normal((co, ci, 3, 3), 0.1), rng, np.float16)
    b = draw((co,), rng, np.float16)
    s = draw(uniform((co,), 0.5, 1.5), rng, np.float16)
    x = draw((2, ci, hw, hw), rng, np.float16)
    r = draw((2, co, hw, hw), rng, np.float16)
    got = run_conv(gpu, x, w, b, s, r, out_dtype=np.float16, epi="SILU", order=order).astype(np.float32)
    want = oracle.conv2d(x, w, b, s, r, epi="SILU", order=order)
    assert_close(got, want, FP16)


@pytest.mark.parametrize("order", [0, 1])
def test_conv3_lds_transpose_scale_residual(gpu, order):
    """Scale, fp16 residual (both orders) and fp16 output on the same plan."""
    rng = np.random.default_rng(order)
    ci, co, hw = 32, 32, 32
    w = draw(normal((co, ci, 3, 3), 0.1), rng, np.float16)
    b = draw((co,), rng, np.float16)
    s = draw(uniform((co,), 0.5, 1.5), rng, np.float16)
    x = draw((1, ci, hw, hw), rng, np.float16)
    r = draw((1, co, hw, hw), rng, np.float16)
    got = run_conv(gpu, x, w, b, s, r, out_dtype=np.float16, epi="RELU", order=order).astype(np.float32)
    want = oracle.conv2d(x, w, b, s, r, epi="RELU", order=order)
    assert_close(got, want, FP16)


@pytest.mark.parametrize("ci, co, h, w, batch, order, odt, rdt", [
    (40, 48, 6, 4, 2, 0, np.float16, np.float16),      # channel and output-channel tails, 24 positions (half a fragment)
    (256, 128, 8, 10, 1, 1, np.float32, np.float32),   # eight channel blocks, residual before the activation
    (32, 200, 4, 2, 3, 0, np.float32, np.float16),     # a single partial fragment per image, batch 3
])
def test_conv1_pointwise(gpu, ci, co, h, w, batch, order, odt, rdt):
    """The pointwise kernel (1x1, stride 1, fp16 input: positions taken as one
    flat row of 16-wide fragments) with scale, residual and output dtypes."""
    rng = np.random.default_rng(ci + co)
    wt = draw(normal((co, ci, 1, 1), 1.0 / np.sqrt(ci)), rng, np.float16)
    b = draw((co,), rng, np.float16)
    s = draw(uniform((co,), 0.5, 1.5), rng, np.float16)
    x = draw((batch, ci, h, w), rng, np.float16)
    r = draw((batch, co, h, w), rng, rdt)
    print(f"conv1 ci={ci} co={co} h={h} w={w} batch={batch}", flush=True)
    got = run_conv(gpu, x, wt, b, s, r, out_dtype=odt, epi="SILU", order=order).astype(np.float32)
    want = oracle.conv2d(x, wt, b, s, r, epi="SILU", order=order)
    assert_close(got, want, FP16)


class _Offset:
    """A buffer `off` bytes into a larger DeviceArray (to miss an alignment on purpose)."""

    def __init__(self, gpu, shape, dtype, off, data=None):
        self.dtype = np.dtype(dtype)
        self.shape = tuple(shape)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        self._base = gpu.DeviceArray((self.nbytes + off,), np.uint8)
        self.ptr = self._base.ptr + off
        self.code = gpu.dtype_code(self.dtype)
        self._lib = gpu.lib()
        if data is not None:
            a = np.ascontiguousarray(data, self.dtype)
            gpu.check(self._lib.vai_memcpy_h2d(self.ptr, a.ctypes.data, a.nbytes, None), "h2d")

    def numpy(self):
        import ctypes
        out = np.empty(self.shape, self.dtype)
        self._lib.vai_memcpy_d2h(ctypes.c_void_p(out.ctypes.data), ctypes.c_void_p(self.ptr),
                                 ctypes.c_size_t(self.nbytes), None)
        return out


@pytest.mark.parametrize("off", [0, 16])
def test_conv3_output_alignment(gpu, off):
    """An output and residual 16 bytes past a 32-byte boundary leave the
    LDS-transpose plan (its 8-wide stores need 32-byte alignment) for the
    general kernel; both placements give the oracle's result."""
    rng = np.random.default_rng(11)
    ci, co, hw = 32, 32, 32
    w = draw(normal((co, ci, 3, 3), 0.1), rng, np.float16)
    b = draw((co,), rng, np.float16)
    x = draw((1, ci, hw, hw), rng, np.float16)
    r = draw((1, co, hw, hw), rng, np.float16)
    D = gpu.DeviceArray.from_numpy
    out = _Offset(gpu, (1, co, hw, hw), np.float32, off)
    res = _Offset(gpu, (1, co, hw, hw), np.float16, off, r)
    print(f"conv3 output offset {off}", flush=True)
    gpu.conv2d(out, D(x), D(w), D(b), None, res, epi="SILU", order=0)
    assert_close(out.numpy(), oracle.conv2d(x, w, b, None, r, epi="SILU", order=0), FP16)


@pytest.mark.parametrize("epi, odt, scaled", [
    ("NONE", np.float16, False), ("RELU", np.float16, True), ("SILU", np.float16, False),
    ("SIGMOID", np.float32, True), ("SILU", np.float32, True), ("NONE", np.float32, False),
])
def test_conv3_cheap_epilogue(gpu, epi, odt, scaled):
    """The 3x3 plan's branch-free epilogue (none / SiLU, no residual), whose
    fragments are stored during the last channel block, beside the general
    one (ReLU, sigmoid): both output dtypes, a scale, an output-channel tail
    (80 = 64 + 16: the second workgroup's waves past Co store nothing), and
    nothing written past the output (a guard band after it keeps its fill)."""
    rng = np.random.default_rng(17)
    ci, co, hi, wi, batch = 64, 80, 12, 48, 2
    w = draw(normal((co, ci, 3, 3), 1.0 / np.sqrt(ci * 9)), rng, np.float16)
    b = draw(normal((co,), 0.1), rng, np.float16)
    s = draw(uniform((co,), 0.5, 1.5), rng, np.float16) if scaled else None
    x = draw((batch, ci, hi, wi), rng, np.float16)
    D = gpu.DeviceArray.from_numpy
    shape = (batch, co, hi, wi)
    nbytes = int(np.prod(shape)) * np.dtype(odt).itemsize
    fill = np.full(nbytes + 4096, 0xAB, np.uint8)
    out = _Offset(gpu, shape, odt, 0, None)
    out._base = D(fill)
    out.ptr = out._base.ptr
    print(f"conv3 cheap epilogue {epi} {np.dtype(odt).name} scaled={scaled}", flush=True)
    gpu.conv2d(out, D(x), D(w), D(b), D(s) if scaled else None, None, epi=epi)
    got = out.numpy().astype(np.float32)
    assert_close(got, oracle.conv2d(x, w, b, s, epi=epi), FP16)
    assert (out._base.numpy()[nbytes:] == 0xAB).all()


@pytest.mark.parametrize("epi, odt, scaled", [("NONE", np.float16, True), ("SILU", np.float32, False),
                                             ("SILU", np.float16, True), ("RELU", np.float32, False)])
def test_conv1_cheap_epilogue(gpu, epi, odt, scaled):
    """The pointwise plan's branch-free epilogue (none / SiLU, no residual;
    ReLU takes the general one): four consecutive positions per store, an
    output-channel tail (80), 120 positions (the last workgroup's second half
    lies past H W), batch 2, and a guard band after the output that keeps
    its fill."""
    rng = np.random.default_rng(23)
    ci, co, h, w_, batch = 48, 80, 10, 12, 2
    w = draw(normal((co, ci, 1, 1), 1.0 / np.sqrt(ci)), rng, np.float16)
    b = draw(normal((co,), 0.1), rng, np.float16)
    s = draw(uniform((co,), 0.5, 1.5), rng, np.float16) if scaled else None
    x = draw((batch, ci, h, w_), rng, np.float16)
    D = gpu.DeviceArray.from_numpy
    shape = (batch, co, h, w_)
    nbytes = int(np.prod(shape)) * np.dtype(odt).itemsize
    out = _Offset(gpu, shape, odt, 0, None)
    out._base = D(np.full(nbytes + 4096, 0xAB, np.uint8))
    out.ptr = out._base.ptr
    print(f"conv1 cheap epilogue {epi} {np.dtype(odt).name} scaled={scaled}", flush=True)
    gpu.conv2d(out, D(x), D(w), D(b), D(s) if scaled else None, None, epi=epi)
    assert_close(out.numpy().astype(np.float32), oracle.conv2d(x, w, b, s, epi=epi), FP16)
    assert (out._base.numpy()[nbytes:] == 0xAB).all()


@pytest.mark.parametrize("ks, odt", [(1, np.float32), (1, np.float16), (3, np.float16)])
def test_conv_cheap_epilogue_unaligned_output(gpu, ks, odt):
    """An output 4 bytes off a 16-byte boundary leaves the cheap epilogue
    (16- and 8-byte stores) for the general one; the result is the oracle's."""
    rng = np.random.default_rng(29 + ks)
    ci, co, hw = 32, 48, 16
    w = draw(normal((co, ci, ks, ks), 0.1), rng, np.float16)
    b = draw((co,), rng, np.float16)
    x = draw((1, ci, hw, hw), rng, np.float16)
    D = gpu.DeviceArray.from_numpy
    out = _Offset(gpu, (1, co, hw, hw), odt, 4)
    print(f"conv k{ks} cheap epilogue, output 4 bytes off, {np.dtype(odt).name}", flush=True)
    gpu.conv2d(out, D(x), D(w), D(b), None, None, epi="SILU")
    assert_close(out.numpy().astype(np.float32), oracle.conv2d(x, w, b, epi="SILU"), FP16)


@pytest.mark.parametrize("ci, co, hi, wi, epi, odt", [
    (16, 32, 6, 16, "SILU", np.float16),     # one column fragment, one channel block
    (48, 64, 5, 32, "NONE", np.float32),     # two fragments, two blocks (the second partial)
    (96, 16, 4, 64, "SILU", np.float32),     # four fragments, three blocks, 16 output channels
    (128, 80, 3, 80, "NONE", np.float16),    # config 5's row width, four blocks, a channel tail
    (72, 48, 4, 96, "SILU", np.float16),     # six fragments
    (40, 64, 3, 112, "SILU", np.float32),    # seven fragments
    (128, 128, 2, 128, "NONE", np.float32),  # eight fragments (the widest row)
])
def test_conv3_cheap_epilogue_widths(gpu, ci, co, hi, wi, epi, odt):
    """The 3x3 kernel's cheap epilogue at every row width it is compiled for
    (one to eight 16-column fragments) and one to four channel blocks, both
    output dtypes: the fragments are stored during the last block, the last
    after it."""
    rng = np.random.default_rng(ci * 7 + wi)
    w = draw(normal((co, ci, 3, 3), 1.0 / np.sqrt(ci * 9)), rng, np.float16)
    b = draw(normal((co,), 0.1), rng, np.float16)
    x = draw((1, ci, hi, wi), rng, np.float16)
    print(f"conv3 cheap widths ci={ci} co={co} hi={hi} wi={wi} {epi} {np.dtype(odt).name}", flush=True)
    got = run_conv(gpu, x, w, b, out_dtype=odt, epi=epi).astype(np.float32)
    assert_close(got, oracle.conv2d(x, w, b, epi=epi), FP16)


def run_scores(capi, q, k, **kw):
    dq, dk = capi.DeviceArray.from_numpy(q), capi.DeviceArray.from_numpy(k)
    out = capi.DeviceArray(q.shape[:-1] + (k.shape[-2],), np.float32)
    capi.attn_scores(out, dq, dk, **kw)
    return out.numpy()


@pytest.mark.parametrize("hq, hkv, tq, tkv, d, causal, span, dt", [
    (2, 2, 64, 64, 64, True, 0, np.float16),
    (4, 2, 100, 100, 32, True, 0, np.float16),       # GQA, ragged
    (2, 1, 5, 37, 64, True, 0, np.float16),          # Tq < Tkv: queries align at the end
    (2, 2, 130, 130, 16, True, 24, np.float32),      # sliding window
    (1, 1, 70, 90, 48, False, 0, np.float32),        # no mask
    (3, 3, 257, 257, 128, True, 0, np.float16),
    (12, 4, 130, 130, 64, True, 0, np.float16),      # 12 heads: a partial second round over the 8 XCDs
    (17, 17, 64, 96, 64, False, 0, np.float16),
    # square causal, Tq a multiple of 64, head dim 64/128/256: the strip form
    # (64-row strips, four column classes, Q held in registers)
    (8, 2, 512, 512, 128, True, 0, np.float16),      # 8 heads (one per XCD), GQA
    (3, 3, 320, 320, 64, True, 0, np.float16),       # heads not a multiple of 8, 5 strips
    (8, 8, 1024, 1024, 256, True, 0, np.float16),    # config 4's shape
    (2, 1, 128, 128, 256, True, 0, np.float16),      # 2 strips: classes with no computed tile
    # other head dims: only the tiles on and below the diagonal are launched,
    # each writing its mirror tile's -inf
    (2, 2, 192, 192, 192, True, 0, np.float16),
])
def test_scores(gpu, hq, hkv, tq, tkv, d, causal, span, dt):
    rng = np.random.default_rng(0)
    q = draw((hq, tq, d), rng, dt)
    k = draw((hkv, tkv, d), rng, dt)
    got = run_scores(gpu, q, k, causal=causal, span=span)
    want = oracle.attn_scores(q, k, causal=causal, span=span)
    assert_close(got, want, FP32 if dt == np.float16 else TRANS)


@pytest.mark.parametrize("tq, tkv, d, blocks, span, dt", [
    (300, 300, 64, (0b01, [100]), 0, np.float16),            # prefix-LM, fast kernel, ragged tiles
    (257, 257, 128, (0b101, [70, 190]), 0, np.float16),      # causal / full / causal
    (200, 260, 64, (0b010, [50, 130]), 40, np.float16),      # full / causal / full, Tq < Tkv, window
    (90, 90, 48, (0b01, [33]), 0, np.float32),               # the generic tile path
    (128, 128, 64, (0b0, []), 0, np.float16),                # one full block: no mask
])
def test_scores_block_mask(gpu, tq, tkv, d, blocks, span, dt):
    rng = np.random.default_rng(tq)
    q = draw((2, tq, d), rng, dt)
    k = draw((2, tkv, d), rng, dt)
    print(f"scores blocks={blocks} tq={tq} tkv={tkv} d={d}", flush=True)
    got = run_scores(gpu, q, k, blocks=blocks, span=span)
    want = oracle.attn_scores(q, k, blocks=blocks, span=span)
    assert_close(got, want, FP32 if dt == np.float16 else TRANS)


def test_scores_block_mask_rejects(gpu):
    import ctypes
    D = gpu.DeviceArray
    q = D((1, 16, 64), np.float16)
    a = gpu.attn_scores_args(D((1, 16, 16), np.float32), q, q, blocks=(0b01, [8, 4]))   # ends must increase
    assert gpu.lib().vai_attn_scores_launch(ctypes.byref(a), None) == 1001
    a = gpu.attn_scores_args(D((1, 16, 16), np.float32), q, q, blocks=(0b01, [8]))
    a.causal = 1                                                                         # both at once
    assert gpu.lib().vai_attn_scores_launch(ctypes.byref(a), None) == 1001


def test_config4_attention_scores(gpu):
    """Q,K [8,1024,256] fp16, S = QK^T/16 causal; oracle on heads 0 and 7."""
    rng = np.random.default_rng(0)
    q = draw((8, 1024, 256), rng, np.float16)
    k = draw((8, 1024, 256), rng, np.float16)
    got = run_scores(gpu, q, k, scale=1.0 / 16, causal=True)
    i, j = np.indices((1024, 1024))
    assert np.isneginf(got[:, j > i]).all()
    for h in (0, 7):
        want = oracle.attn_scores(q[h:h + 1], k[h:h + 1], scale=1.0 / 16, causal=True)
        assert_close(got[h:h + 1], want, FP32)


@pytest.mark.parametrize("ci, co, ks, stride, hw, dt_in", [(40, 48, 3, 1, 19, np.float16), (64, 32, 1, 1, 24, np.float32),
                                                           (16, 24, 3, 2, 21, np.float16), (96, 40, 3, 2, 33, np.float32)])
def test_conv_packed_weight_reuse(gpu, ci, co, ks, stride, hw, dt_in):
    """A weight packed once (vai_conv2d_pack_weight) gives the same output as
    the per-call pack, on two different inputs."""
    rng = np.random.default_rng(2)
    w = draw(normal((co, ci, ks, ks), 0.1), rng, np.float16)
    b = draw(normal((co,), 0.1), rng, np.float16)
    D = gpu.DeviceArray.from_numpy
    dw, db = D(w), D(b)
    ho = (hw - 1) // stride + 1
    for seed in (0, 1):
        x = draw((2, ci, hw, hw), np.random.default_rng(seed), dt_in)
        dx = D(x)
        o1 = gpu.DeviceArray((2, co, ho, ho), np.float32)
        gpu.conv2d(o1, dx, dw, db, stride=stride, epi="SILU")
        a = gpu.conv2d_args(o1, dx, dw, db, stride=stride, epi="SILU")
        packed = gpu.conv2d_pack_weight(a)
        assert packed is not None
        o2 = gpu.DeviceArray((2, co, ho, ho), np.float32)
        gpu.conv2d(o2, dx, dw, db, stride=stride, epi="SILU", packed=packed)
        np.testing.assert_array_equal(o1.numpy(), o2.numpy())
        assert_close(o2.numpy(), oracle.conv2d(x, w, b, stride=stride, epi="SILU"), FP16)
