"""ctypes binding of include/vai_amd.h (libvai_amd.so, built in-tree).

This is the binding a Python caller of the C ABI writes; the tests and
bench.py drive the kernels through it. There is no fallback: if the library
is missing, every call raises.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libvai_amd.so")

F32, F16, NONE = 0, 1, 2
EPILOGUES = {"NONE": 0, "RELU": 1, "GELU": 2, "GELU_TANH": 3, "SILU": 4, "SIGMOID": 5}
RESIDUAL_ORDERS = {"AFTER_EPILOGUE": 0, "BEFORE_EPILOGUE": 1}
MAX_CAUSAL_BLOCKS = 32

# Every symbol include/vai_amd.h declares (checked by tests/test_capi_symbols.py).
EXPORTS = [
    "vai_linear_launch", "vai_linear_workspace_size", "vai_linear_plan", "vai_gated_mul_launch",
    "vai_linear_launch_noalloc",
    "vai_linear_packed_weight_size", "vai_linear_pack_weight",
    "vai_conv2d_launch", "vai_conv2d_workspace_size", "vai_conv2d_packed_weight_size", "vai_conv2d_pack_weight",
    "vai_attn_scores_launch", "vai_attention_launch", "vai_attention_workspace_size",
    "vai_device_count", "vai_set_device", "vai_malloc", "vai_free", "vai_memcpy_h2d", "vai_memcpy_d2h",
    "vai_memcpy_d2d", "vai_memset", "vai_stream_create", "vai_stream_destroy", "vai_stream_sync",
    "vai_device_sync", "vai_status_string", "vai_event_create", "vai_event_destroy", "vai_event_record",
    "vai_event_sync", "vai_event_elapsed_ms",
    "vai_graph_begin_capture", "vai_graph_end_capture", "vai_graph_launch", "vai_graph_destroy",
]


class LinearArgs(ctypes.Structure):
    _fields_ = [
        ("out", ctypes.c_void_p), ("inp", ctypes.c_void_p), ("weight", ctypes.c_void_p),
        ("bias", ctypes.c_void_p), ("residual", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
        ("M", ctypes.c_uint32), ("N", ctypes.c_uint32), ("K", ctypes.c_uint32),
        ("o_dtype", ctypes.c_int32), ("i_dtype", ctypes.c_int32), ("w_dtype", ctypes.c_int32),
        ("b_dtype", ctypes.c_int32),
        ("epilogue", ctypes.c_uint32), ("residual_order", ctypes.c_uint32),
        ("bias_repeat", ctypes.c_uint32), ("residual_repeat", ctypes.c_uint32),
        ("scalar_scale", ctypes.c_float), ("split_size", ctypes.c_uint32),
        ("gated", ctypes.c_uint32), ("gate_epilogue", ctypes.c_uint32),
        ("packed_weight", ctypes.c_void_p), ("acc_dtype", ctypes.c_int32),
    ]


class Conv2dArgs(ctypes.Structure):
    _fields_ = [
        ("out", ctypes.c_void_p), ("inp", ctypes.c_void_p), ("weight", ctypes.c_void_p),
        ("bias", ctypes.c_void_p), ("scale", ctypes.c_void_p), ("residual", ctypes.c_void_p),
        ("batch", ctypes.c_uint32), ("ci", ctypes.c_uint32), ("hi", ctypes.c_uint32), ("wi", ctypes.c_uint32),
        ("co", ctypes.c_uint32), ("kernel", ctypes.c_uint32), ("stride", ctypes.c_uint32),
        ("o_dtype", ctypes.c_int32), ("i_dtype", ctypes.c_int32), ("w_dtype", ctypes.c_int32),
        ("epilogue", ctypes.c_uint32), ("residual_order", ctypes.c_uint32),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
        ("packed_weight", ctypes.c_void_p),
    ]


class AttnScoresArgs(ctypes.Structure):
    _fields_ = [
        ("scores", ctypes.c_void_p), ("q", ctypes.c_void_p), ("k", ctypes.c_void_p),
        ("batch", ctypes.c_uint32), ("hq", ctypes.c_uint32), ("hkv", ctypes.c_uint32),
        ("tq", ctypes.c_uint32), ("tkv", ctypes.c_uint32), ("head_dim", ctypes.c_uint32),
        ("dtype", ctypes.c_int32), ("scale", ctypes.c_float), ("causal", ctypes.c_uint32),
        ("span", ctypes.c_uint32),
        ("mask_blocks", ctypes.c_uint32), ("mask_bits", ctypes.c_uint32),
        ("mask_block_end", ctypes.c_uint32 * (MAX_CAUSAL_BLOCKS - 1)),
    ]


class AttentionArgs(ctypes.Structure):
    _fields_ = [
        ("out", ctypes.c_void_p), ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("o_dtype", ctypes.c_int32), ("q_dtype", ctypes.c_int32), ("kv_dtype", ctypes.c_int32),
        ("batch", ctypes.c_uint32), ("hq", ctypes.c_uint32), ("hkv", ctypes.c_uint32),
        ("tq", ctypes.c_uint32), ("tkv", ctypes.c_uint32), ("head_dim", ctypes.c_uint32),
        ("scale", ctypes.c_float), ("causal", ctypes.c_uint32), ("span", ctypes.c_uint32),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
        ("mask_blocks", ctypes.c_uint32), ("mask_bits", ctypes.c_uint32),
        ("mask_block_end", ctypes.c_uint32 * (MAX_CAUSAL_BLOCKS - 1)),
        ("k_cache", ctypes.c_void_p), ("v_cache", ctypes.c_void_p), ("cache_count", ctypes.c_void_p),
        ("cache_size", ctypes.c_uint32), ("cache_dtype", ctypes.c_int32), ("cache_ring", ctypes.c_uint32),
    ]


class VaiError(RuntimeError):
    pass


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise VaiError(f"{LIB_PATH} is not built; run `python -m vai_amd.build`")
        L = ctypes.CDLL(LIB_PATH)
        vp, sz, u32, i32 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint32, ctypes.c_int32
        L.vai_linear_launch.argtypes = [ctypes.POINTER(LinearArgs), vp]
        L.vai_linear_launch_noalloc.argtypes = [ctypes.POINTER(LinearArgs), vp]
        L.vai_linear_workspace_size.argtypes = [ctypes.POINTER(LinearArgs)]
        L.vai_linear_workspace_size.restype = sz
        L.vai_linear_plan.argtypes = [ctypes.POINTER(LinearArgs), ctypes.c_char_p, sz, ctypes.POINTER(u32)]
        L.vai_gated_mul_launch.argtypes = [vp, i32, vp, i32, u32, u32, u32, vp]
        L.vai_linear_packed_weight_size.argtypes = [ctypes.POINTER(LinearArgs)]
        L.vai_linear_packed_weight_size.restype = sz
        L.vai_linear_pack_weight.argtypes = [ctypes.POINTER(LinearArgs), vp, sz, vp]
        L.vai_conv2d_launch.argtypes = [ctypes.POINTER(Conv2dArgs), vp]
        L.vai_conv2d_workspace_size.argtypes = [ctypes.POINTER(Conv2dArgs)]
        L.vai_conv2d_workspace_size.restype = sz
        L.vai_conv2d_packed_weight_size.argtypes = [ctypes.POINTER(Conv2dArgs)]
        L.vai_conv2d_packed_weight_size.restype = sz
        L.vai_conv2d_pack_weight.argtypes = [ctypes.POINTER(Conv2dArgs), vp, sz, vp]
        L.vai_attn_scores_launch.argtypes = [ctypes.POINTER(AttnScoresArgs), vp]
        L.vai_attention_launch.argtypes = [ctypes.POINTER(AttentionArgs), vp]
        L.vai_attention_workspace_size.argtypes = [ctypes.POINTER(AttentionArgs)]
        L.vai_attention_workspace_size.restype = sz
        L.vai_malloc.argtypes = [ctypes.POINTER(vp), sz]
        L.vai_free.argtypes = [vp]
        L.vai_memcpy_h2d.argtypes = [vp, vp, sz, vp]
        L.vai_memcpy_d2h.argtypes = [vp, vp, sz, vp]
        L.vai_memcpy_d2d.argtypes = [vp, vp, sz, vp]
        L.vai_memset.argtypes = [vp, ctypes.c_int, sz, vp]
        L.vai_stream_create.argtypes = [ctypes.POINTER(vp)]
        L.vai_stream_destroy.argtypes = [vp]
        L.vai_stream_sync.argtypes = [vp]
        L.vai_set_device.argtypes = [ctypes.c_int]
        L.vai_device_count.argtypes = [ctypes.POINTER(ctypes.c_int)]
        L.vai_status_string.restype = ctypes.c_char_p
        L.vai_status_string.argtypes = [ctypes.c_int]
        L.vai_event_create.argtypes = [ctypes.POINTER(vp)]
        L.vai_event_destroy.argtypes = [vp]
        L.vai_event_record.argtypes = [vp, vp]
        L.vai_event_sync.argtypes = [vp]
        L.vai_event_elapsed_ms.argtypes = [ctypes.POINTER(ctypes.c_float), vp, vp]
        L.vai_graph_begin_capture.argtypes = [vp]
        L.vai_graph_end_capture.argtypes = [vp, ctypes.POINTER(vp)]
        L.vai_graph_launch.argtypes = [vp, vp]
        L.vai_graph_destroy.argtypes = [vp]
        _lib = L
    return _lib


def check(status, what=""):
    if status != 0:
        msg = lib().vai_status_string(status).decode()
        raise VaiError(f"{what}: status {status} ({msg})")


def dtype_code(dt):
    dt = np.dtype(dt)
    if dt == np.float16:
        return F16
    if dt == np.float32:
        return F32
    raise VaiError(f"unsupported dtype {dt}")


class DeviceArray:
    """A hipMalloc'd buffer with a numpy shape and dtype (fp16 or fp32)."""

    def __init__(self, shape, dtype=np.float32):
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = ctypes.c_void_p()
        check(lib().vai_malloc(ctypes.byref(p), max(self.nbytes, 1)), "vai_malloc")
        self.ptr = p.value

    @classmethod
    def from_numpy(cls, a, stream=None):
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        check(lib().vai_memcpy_h2d(d.ptr, a.ctypes.data, a.nbytes, stream), "h2d")
        return d

    def numpy(self, stream=None):
        out = np.empty(self.shape, self.dtype)
        check(lib().vai_memcpy_d2h(out.ctypes.data, self.ptr, self.nbytes, stream), "d2h")
        return out

    def fill_(self, byte, stream=None):
        check(lib().vai_memset(self.ptr, byte, self.nbytes, stream), "memset")

    @property
    def code(self):
        return dtype_code(self.dtype)

    def free(self):
        if getattr(self, "ptr", None):
            lib().vai_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def _ptr(d):
    return None if d is None else d.ptr


def linear_args(out, inp, weight, bias=None, residual=None, *, epi="NONE", order="AFTER_EPILOGUE",
                scale=1.0, split_size=0, gated=False, gate_epi="SILU", workspace=None, acc=np.float32):
    K = weight.shape[-1]
    N = weight.shape[0]
    M = int(np.prod(inp.shape[:-1]))
    a = LinearArgs()
    a.out, a.inp, a.weight = out.ptr, inp.ptr, weight.ptr
    a.bias, a.residual = _ptr(bias), _ptr(residual)
    a.M, a.N, a.K = M, N, K
    a.o_dtype, a.i_dtype, a.w_dtype = out.code, inp.code, weight.code
    a.b_dtype = bias.code if bias is not None else NONE
    a.epilogue = EPILOGUES[epi]
    a.residual_order = RESIDUAL_ORDERS[order] if isinstance(order, str) else int(order)
    MN = M * N
    if bias is not None:
        n = int(np.prod(bias.shape))
        a.bias_repeat = 0 if n == MN else n
    if residual is not None:
        n = int(np.prod(residual.shape))
        a.residual_repeat = 0 if n == MN else n
    a.scalar_scale = scale
    a.split_size = split_size
    a.gated = 1 if gated else 0
    a.gate_epilogue = EPILOGUES[gate_epi]
    a.acc_dtype = dtype_code(acc)
    if workspace is not None:
        a.workspace, a.workspace_bytes = workspace.ptr, workspace.nbytes
    a._keep = (out, inp, weight, bias, residual, workspace)   # the buffers live as long as the args
    return a


def linear_workspace_size(args):
    return lib().vai_linear_workspace_size(ctypes.byref(args))


def linear_plan(args):
    buf = ctypes.create_string_buffer(64)
    n = ctypes.c_uint32()
    check(lib().vai_linear_plan(ctypes.byref(args), buf, 64, ctypes.byref(n)), "vai_linear_plan")
    return buf.value.decode(), n.value


def linear_pack_weight(args, stream=None):
    """Packs args' weight once for the prefill path; returns the packed
    buffer (None when the shape or dtypes have no packed path)."""
    n = lib().vai_linear_packed_weight_size(ctypes.byref(args))
    if not n:
        return None
    packed = DeviceArray((n,), np.uint8)
    check(lib().vai_linear_pack_weight(ctypes.byref(args), packed.ptr, packed.nbytes, stream), "linear_pack_weight")
    check(lib().vai_stream_sync(stream), "sync")   # args' weight buffer may go once this returns
    return packed


def linear(out, inp, weight, bias=None, residual=None, stream=None, packed=None, **kw):
    """Launches the Linear kernels; allocates the split-K workspace if needed.
    packed: a linear_pack_weight() result for the weight (prefill shapes)."""
    a = linear_args(out, inp, weight, bias, residual, **kw)
    if packed is not None:
        a.packed_weight = packed.ptr
    ws = None
    need = linear_workspace_size(a)
    if need and a.workspace_bytes < need:
        ws = DeviceArray((need,), np.uint8)
        a.workspace, a.workspace_bytes = ws.ptr, ws.nbytes
    check(lib().vai_linear_launch(ctypes.byref(a), stream), "vai_linear_launch")
    # wait for the kernels: the caller may drop its argument buffers on return
    check(lib().vai_stream_sync(stream), "sync")
    return out


def gated_mul(out, inp, epi="SILU", stream=None):
    H = out.shape[-1]
    rows = int(np.prod(out.shape[:-1]))
    check(lib().vai_gated_mul_launch(out.ptr, out.code, inp.ptr, inp.code, rows, H, EPILOGUES[epi], stream),
          "vai_gated_mul_launch")
    check(lib().vai_stream_sync(stream), "sync")   # the caller may drop its argument buffers on return
    return out


def conv2d_args(out, inp, weight, bias=None, scale=None, residual=None, *, stride=1, epi="NONE",
                order="AFTER_EPILOGUE"):
    Co, Ci, ks, _ = weight.shape
    Hi, Wi = inp.shape[-2:]
    a = Conv2dArgs()
    a.out, a.inp, a.weight = out.ptr, inp.ptr, weight.ptr
    a.bias, a.scale, a.residual = _ptr(bias), _ptr(scale), _ptr(residual)
    a.batch = int(np.prod(inp.shape[:-3]))
    a.ci, a.hi, a.wi, a.co, a.kernel, a.stride = Ci, Hi, Wi, Co, ks, stride
    a.o_dtype, a.i_dtype, a.w_dtype = out.code, inp.code, weight.code
    a.epilogue = EPILOGUES[epi]
    a.residual_order = RESIDUAL_ORDERS[order] if isinstance(order, str) else int(order)
    a._keep = (out, inp, weight, bias, scale, residual)
    return a


def conv2d_workspace_size(args):
    return lib().vai_conv2d_workspace_size(ctypes.byref(args))


def conv2d_pack_weight(args, stream=None):
    """Packs args' weight once; returns the packed buffer (or None on the fp32 path)."""
    n = lib().vai_conv2d_packed_weight_size(ctypes.byref(args))
    if not n:
        return None
    packed = DeviceArray((n,), np.uint8)
    check(lib().vai_conv2d_pack_weight(ctypes.byref(args), packed.ptr, packed.nbytes, stream), "pack_weight")
    check(lib().vai_stream_sync(stream), "sync")   # args' weight buffer may go once this returns
    return packed


def conv2d(out, inp, weight, bias=None, scale=None, residual=None, stream=None, packed=None, **kw):
    """Launches the convolution; allocates its packing workspace if needed.
    packed: a conv2d_pack_weight() result to skip the per-call weight pack."""
    a = conv2d_args(out, inp, weight, bias, scale, residual, **kw)
    if packed is not None:
        a.packed_weight = packed.ptr
    ws = None
    need = conv2d_workspace_size(a)
    if need:
        ws = DeviceArray((need,), np.uint8)
        a.workspace, a.workspace_bytes = ws.ptr, ws.nbytes
    check(lib().vai_conv2d_launch(ctypes.byref(a), stream), "vai_conv2d_launch")
    check(lib().vai_stream_sync(stream), "sync")   # the caller may drop its argument buffers on return
    return out


def _set_blocks(a, blocks):
    """blocks: None, or (bits, ends) -- the reference's block list: len(ends)+1
    blocks, bit (count-1-k) of bits marks block k causal, ends in query rows."""
    if blocks is None:
        return
    bits, ends = blocks
    a.causal = 0
    a.mask_blocks = len(ends) + 1
    a.mask_bits = bits
    for i, e in enumerate(ends):
        a.mask_block_end[i] = e


def attn_scores_args(scores, q, k, *, scale=None, causal=True, span=0, blocks=None):
    Hq, Tq, D = q.shape[-3:]
    Hkv, Tkv, _ = k.shape[-3:]
    a = AttnScoresArgs()
    a.scores, a.q, a.k = scores.ptr, q.ptr, k.ptr
    a.batch = int(np.prod(q.shape[:-3]))
    a.hq, a.hkv, a.tq, a.tkv, a.head_dim = Hq, Hkv, Tq, Tkv, D
    a.dtype = q.code
    a.scale = float(1.0 / np.sqrt(D)) if scale is None else float(scale)
    a.causal = 1 if causal else 0
    a.span = span
    _set_blocks(a, blocks)
    a._keep = (scores, q, k)
    return a


def attn_scores(scores, q, k, stream=None, **kw):
    a = attn_scores_args(scores, q, k, **kw)
    check(lib().vai_attn_scores_launch(ctypes.byref(a), stream), "vai_attn_scores_launch")
    check(lib().vai_stream_sync(stream), "sync")   # the caller may drop its argument buffers on return
    return scores


def attention_args(out, q, k, v, *, scale=None, causal=False, span=0, blocks=None, cache=None):
    """O token-major [..., Tq, Hq, D]; no mask unless causal / blocks ask for one.
    cache = (k_cache, v_cache, count, ring): the KV cache planes [Hkv, size, D]
    (DeviceArrays of one dtype) and a device uint32 DeviceArray holding the
    positions they held before the call; k / v may then be None (Tkv = 0)."""
    Hq, Tq, D = q.shape[-3:]
    a = AttentionArgs()
    a.out, a.q = out.ptr, q.ptr
    a.o_dtype, a.q_dtype = out.code, q.code
    a.batch = int(np.prod(q.shape[:-3]))
    if k is not None:
        Hkv, Tkv, _ = k.shape[-3:]
        a.k, a.v, a.kv_dtype = k.ptr, v.ptr, k.code
    else:
        Hkv, Tkv = cache[0].shape[-3], 0
    a.hq, a.hkv, a.tq, a.tkv, a.head_dim = Hq, Hkv, Tq, Tkv, D
    a.scale = 0.0 if scale is None else float(scale)
    a.causal = 1 if causal else 0
    a.span = span
    _set_blocks(a, blocks)
    if cache is not None:
        kc, vc, count, ring = cache
        a.k_cache, a.v_cache, a.cache_count = kc.ptr, vc.ptr, count.ptr
        a.cache_size, a.cache_dtype, a.cache_ring = kc.shape[-2], kc.code, 1 if ring else 0
    a._keep = (out, q, k, v, cache)
    return a


def attention(out, q, k, v, stream=None, **kw):
    a = attention_args(out, q, k, v, **kw)
    need = lib().vai_attention_workspace_size(ctypes.byref(a))
    ws = DeviceArray((need,), np.uint8) if need else None
    if ws is not None:
        a.workspace, a.workspace_bytes = ws.ptr, ws.nbytes
    check(lib().vai_attention_launch(ctypes.byref(a), stream), "vai_attention_launch")
    check(lib().vai_stream_sync(stream), "sync")   # the caller may drop its argument buffers on return
    return out


def synchronize():
    check(lib().vai_device_sync(), "sync")


class Event:
    def __init__(self):
        p = ctypes.c_void_p()
        check(lib().vai_event_create(ctypes.byref(p)), "event_create")
        self.ptr = p.value

    def record(self, stream=None):
        check(lib().vai_event_record(self.ptr, stream), "event_record")

    def synchronize(self):
        check(lib().vai_event_sync(self.ptr), "event_sync")

    def elapsed_ms(self, end):
        ms = ctypes.c_float()
        check(lib().vai_event_elapsed_ms(ctypes.byref(ms), self.ptr, end.ptr), "elapsed")
        return ms.value

    def __del__(self):
        try:
            lib().vai_event_destroy(self.ptr)
        except Exception:
            pass


def device_count():
    n = ctypes.c_int(0)
    st = lib().vai_device_count(ctypes.byref(n))
    return n.value if st == 0 else 0


class Stream:
    def __init__(self):
        p = ctypes.c_void_p()
        check(lib().vai_stream_create(ctypes.byref(p)), "stream_create")
        self.ptr = p.value

    def synchronize(self):
        check(lib().vai_stream_sync(self.ptr), "stream_sync")

    def __del__(self):
        try:
            lib().vai_stream_destroy(self.ptr)
        except Exception:
            pass


class Graph:
    """Captures whatever fn() launches on `stream` into a replayable HIP graph."""

    def __init__(self, stream, fn):
        self.stream = stream
        check(lib().vai_graph_begin_capture(stream.ptr), "begin_capture")
        try:
            fn()
        finally:
            g = ctypes.c_void_p()
            st = lib().vai_graph_end_capture(stream.ptr, ctypes.byref(g))
        check(st, "end_capture")
        self.ptr = g.value

    def launch(self):
        check(lib().vai_graph_launch(self.ptr, self.stream.ptr), "graph_launch")

    def __del__(self):
        try:
            lib().vai_graph_destroy(self.ptr)
        except Exception:
            pass
