"""ctypes front end of the C restatement in vai_oracle.c (test infrastructure).

Every entry point mirrors one reference kernel's numeric contract; see the
docstrings of vai_oracle.c for the reference file:line each follows.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libvai_oracle.so")
_lib = None

F32, F16 = 0, 1
EPILOGUES = {"NONE": 0, "RELU": 1, "GELU": 2, "GELU_TANH": 3, "SILU": 4, "SIGMOID": 5}


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _lib.orc_epilogue.restype = ctypes.c_float
        _lib.orc_epilogue.argtypes = [ctypes.c_float, ctypes.c_int]
        _lib.orc_f2h.restype = ctypes.c_uint16
        _lib.orc_h2f.restype = ctypes.c_float
        _lib.orc_num_threads.restype = ctypes.c_int
        _lib.orc_fma16.restype = ctypes.c_uint16
        _lib.orc_fma16.argtypes = [ctypes.c_uint16] * 3
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _dt(a):
    if a is None:
        return F32
    if a.dtype == np.float16:
        return F16
    assert a.dtype == np.float32, a.dtype
    return F32


def _c(a):
    return None if a is None else np.ascontiguousarray(a)


# ---- fp16 conversion (reference tensor.cpp:42-90) ---------------------------

def to_f16(x):
    """fp32 -> fp16 bits as the reference host does it: RNE, subnormals flush."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f32_to_f16(_p(x), _p(out), ctypes.c_size_t(x.size))
    return out.view(np.float16)


def from_f16(h):
    h = np.ascontiguousarray(h).view(np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().orc_f16_to_f32(_p(h), _p(out), ctypes.c_size_t(h.size))
    return out


def epilogue(x, epi):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().orc_epilogue_vec(_p(x), _p(y), ctypes.c_size_t(x.size), ctypes.c_int(EPILOGUES[epi]))
    return y


# ---- Linear -----------------------------------------------------------------

def linear(inp, weight, bias=None, residual=None, *, epi="NONE", order=0, scale=1.0,
           out_dtype=np.float32, stage="auto", split_size=0):
    """O = s*epi(I W^T + b) (+R). stage 'slab' (M <= 8) or 'tile' or 'auto'."""
    inp, weight, bias, residual = _c(inp), _c(weight), _c(bias), _c(residual)
    K = weight.shape[-1]
    N = weight.shape[0]
    M = inp.size // K
    if stage == "auto":
        stage = "slab" if M <= 8 else "tile"
    out = np.empty(inp.shape[:-1] + (N,), dtype=out_dtype)
    bias_rep = 0 if bias is None or bias.size == M * N else bias.size
    res_rep = 0 if residual is None or residual.size == M * N else residual.size
    lib().orc_linear(_p(out), _dt(out), _p(inp), _dt(inp), _p(weight), _dt(weight),
                     _p(bias), _dt(bias), ctypes.c_uint32(bias_rep),
                     _p(residual), ctypes.c_uint32(res_rep),
                     ctypes.c_uint32(M), ctypes.c_uint32(N), ctypes.c_uint32(K),
                     ctypes.c_int(EPILOGUES[epi]), ctypes.c_int(order), ctypes.c_float(scale),
                     ctypes.c_int(1 if stage == "tile" else 0), ctypes.c_uint32(split_size))
    return out


def linear_acc16(inp, weight, bias=None, residual=None, *, epi="NONE", order=0, scale=1.0,
                 out_dtype=np.float32, split_size=0, gated=False, gate_epi="SILU"):
    """The tile path with an fp16 accumulator (Linear::setAccDtype(Fp16)):
    fp16 sums in linear-tile.comp's fma order, clamped, finished in fp32."""
    inp, weight, bias, residual = _c(inp), _c(weight), _c(bias), _c(residual)
    K, N = weight.shape[-1], weight.shape[0]
    M = inp.size // K
    cols = N // 2 if gated else N
    out = np.empty(inp.shape[:-1] + (cols,), dtype=out_dtype)
    bias_rep = 0 if bias is None or bias.size == M * N else bias.size
    res_rep = 0 if residual is None or residual.size == M * N else residual.size
    lib().orc_linear_acc16(_p(out), _dt(out), _p(inp), _dt(inp), _p(weight), _dt(weight),
                           _p(bias), _dt(bias), ctypes.c_uint32(bias_rep), _p(residual), ctypes.c_uint32(res_rep),
                           ctypes.c_uint32(M), ctypes.c_uint32(N), ctypes.c_uint32(K),
                           ctypes.c_int(EPILOGUES[epi]), ctypes.c_int(order), ctypes.c_float(scale),
                           ctypes.c_uint32(split_size), ctypes.c_int(1 if gated else 0),
                           ctypes.c_int(EPILOGUES[gate_epi]))
    return out


def fma16(a, b, c):
    """fp16 fused multiply-add on fp16 arrays (one rounding), elementwise."""
    a, b, c = (np.ascontiguousarray(v, np.float16).view(np.uint16) for v in (a, b, c))
    f = np.vectorize(lambda x, y, z: lib().orc_fma16(int(x), int(y), int(z)), otypes=[np.uint16])
    return f(a, b, c).view(np.float16)


def gemm_f32(a, b):
    """Plain fp32 O = A B^T (CPU baseline kernel)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    M, K = a.shape
    N = b.shape[0]
    out = np.empty((M, N), dtype=np.float32)
    lib().orc_gemm_f32(_p(out), _p(a), _p(b), ctypes.c_uint32(M), ctypes.c_uint32(N), ctypes.c_uint32(K))
    return out


def linear_reduce(partials, bias=None, residual=None, *, epi="NONE", order=0, scale=1.0):
    partials = _c(partials)
    split, MN = partials.shape[0], partials[0].size
    out = np.empty(partials.shape[1:], dtype=partials.dtype)
    bias_rep = 0 if bias is None or bias.size == MN else bias.size
    res_rep = 0 if residual is None or residual.size == MN else residual.size
    bias, residual = _c(bias), _c(residual)
    lib().orc_linear_reduce(_p(out), _p(partials), _dt(partials), ctypes.c_uint32(split), ctypes.c_uint32(MN),
                            _p(bias), _dt(bias), ctypes.c_uint32(bias_rep), _p(residual), ctypes.c_uint32(res_rep),
                            ctypes.c_int(EPILOGUES[epi]), ctypes.c_int(order), ctypes.c_float(scale))
    return out


def gated_mul(inp, *, epi="SILU", out_dtype=np.float32):
    inp = _c(inp)
    H = inp.shape[-1] // 2
    rows = inp.size // (2 * H)
    out = np.empty(inp.shape[:-1] + (H,), dtype=out_dtype)
    lib().orc_gated_mul(_p(out), _dt(out), _p(inp), _dt(inp), ctypes.c_uint32(rows), ctypes.c_uint32(H),
                        ctypes.c_int(EPILOGUES[epi]))
    return out


def conv2d(x, weight, bias=None, scale=None, residual=None, *, stride=1, epi="NONE", order=0,
           out_dtype=np.float32):
    """Same-padded odd-kernel conv, x [..., Ci, Hi, Wi], weight [Co, Ci, k, k]."""
    x, weight, bias, scale, residual = _c(x), _c(weight), _c(bias), _c(scale), _c(residual)
    Co, Ci, ks, _ = weight.shape
    Hi, Wi = x.shape[-2:]
    batch = x.size // (Ci * Hi * Wi)
    Ho, Wo = (Hi - 1) // stride + 1, (Wi - 1) // stride + 1
    out = np.empty(x.shape[:-3] + (Co, Ho, Wo), dtype=out_dtype)
    lib().orc_conv2d(_p(out), _dt(out), _p(x), _dt(x), _p(weight), _dt(weight), _p(bias), _p(scale), _p(residual),
                     ctypes.c_uint32(batch), ctypes.c_uint32(Ci), ctypes.c_uint32(Hi), ctypes.c_uint32(Wi),
                     ctypes.c_uint32(Co), ctypes.c_uint32(ks), ctypes.c_uint32(stride),
                     ctypes.c_int(EPILOGUES[epi]), ctypes.c_int(order))
    return out


def attn_scores(q, k, *, scale=None, causal=True, span=0, blocks=None):
    """S = scale * Q K^T per head, -inf where the mask hides a key. blocks:
    None, or (bits, ends) -- the reference's block list (len(ends) + 1 blocks,
    bit (count-1-k) of bits marks block k causal; causal is then ignored)."""
    q, k = _c(q), _c(k)
    assert q.dtype == k.dtype
    Hq, Tq, D = q.shape[-3:]
    Hkv, Tkv, _ = k.shape[-3:]
    lead = q.size // (Hq * Tq * D)
    if scale is None:
        scale = 1.0 / np.sqrt(D)
    out = np.empty(q.shape[:-1] + (Tkv,), dtype=np.float32)
    nb, bits, ends = 0, 0, None
    if blocks is not None:
        bits, e = blocks
        nb = len(e) + 1
        ends = np.ascontiguousarray(np.asarray(list(e) + [0], np.uint32))
        causal = False
    lib().orc_attn_scores_blocks(_p(out), _p(q), _p(k), _dt(q), ctypes.c_uint32(Hq * lead),
                                 ctypes.c_uint32(Hkv * lead), ctypes.c_uint32(Tq), ctypes.c_uint32(Tkv),
                                 ctypes.c_uint32(D), ctypes.c_float(scale), ctypes.c_int(1 if causal else 0),
                                 ctypes.c_uint32(span), ctypes.c_uint32(nb), ctypes.c_uint32(bits), _p(ends))
    return out


def attention(q, k, v, *, scale=None, causal=False, span=0, out_dtype=np.float32, blocks=None):
    """The reference's Attention node without a KV cache: O[..., i, h, :] =
    sum_j softmax_j(S[..., h, i, :]) V[..., h / g, j, :], S = attn_scores(q, k)
    (the mask's -inf entries drop out), evaluated in float64 from the
    operands' exact values. Q [..., Hq, Tq, D], K / V [..., Hkv, Tkv, D], each
    fp32 or fp16; O is token-major [..., Tq, Hq, D]
    (/root/reference/vai/shaders/attention-fa.comp:8,96; nodes/attention.h:
    1220-1223). No mask unless one is asked for (attention.h:129: a null mask
    binds no mask); a row with no visible key gives 0 (attention-fa.comp:889).
    The fused pass of attention-fa.comp (scores at :581-591, online softmax,
    P.V); this restatement takes the exact softmax, the limit that the
    reference's fp32 sweep approximates."""
    q, k, v = _c(q), _c(k), _c(v)
    if q.dtype != k.dtype:   # the scores oracle reads one dtype: fp32 holds fp16 values exactly
        q, k = q.astype(np.float32), k.astype(np.float32)
    S = attn_scores(q, k, scale=scale, causal=causal, span=span, blocks=blocks).astype(np.float64)
    Hq, Tq, D = q.shape[-3:]
    Hkv, Tkv, _ = k.shape[-3:]
    g = Hq // Hkv
    vv = np.repeat(v.astype(np.float64).reshape((-1, Hkv, Tkv, D)), g, axis=1).reshape(q.shape[:-2] + (Tkv, D))
    finite = np.isfinite(S)
    m = np.where(finite, S, -np.inf).max(axis=-1, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    P = np.where(finite, np.exp(S - m), 0.0)
    l = P.sum(axis=-1, keepdims=True)
    O = np.einsum("...ij,...jd->...id", P, vv)
    O = np.where(l > 0, O / np.where(l > 0, l, 1.0), 0.0)   # [..., Hq, Tq, D]
    return np.ascontiguousarray(np.swapaxes(O, -3, -2)).astype(out_dtype)


def _new_token_end(t, tq, causal, blocks):
    """common/causal_mask.h:25-38: the new tokens query t may read (no mask:
    all Tq; a causal block: up to itself; a full block: to its end)."""
    if blocks is None:
        return t + 1 if causal else tq
    bits, ends = blocks
    nb = len(ends) + 1
    k, end = 0, tq
    while k + 1 < nb:
        e = min(ends[k], tq)
        if t < e:
            end = e
            break
        k += 1
    return t + 1 if (bits >> (nb - 1 - k)) & 1 else end


def attention_cached(q, k, v, k_cache, v_cache, count, *, ring=False, scale=None, causal=False, span=0,
                     blocks=None, out_dtype=np.float32):
    """The reference's Attention with its KV cache, restated from its formulas
    (one sequence): the tkv new K / V rows are appended at positions count ..
    count + tkv - 1, row p of the cache planes [Hkv, size, D] (p % size for
    a ring), rounded to the cache dtype (attention-fa.comp:344-400); query t
    sits at position keyPos(t) = count + max(t + tkv - tq, 0) and reads the
    positions [keyStart(keyPos(t)), count + keyEnd(t)), keyEnd(t) =
    max(newTokenEnd(t) + tkv - tq, 0) (attention-fa.comp:137-146, 470-478;
    causal_mask.h:42-45), position j at its cache row. Exact softmax in
    float64 as attention() takes it. k / v may be None (tkv = 0). Returns
    (O token-major [Tq, Hq, D], the updated K cache, the updated V cache)."""
    q = _c(q)
    kc, vc = np.array(k_cache, copy=True), np.array(v_cache, copy=True)
    Hkv, size, D = kc.shape
    Hq, tq, _ = q.shape[-3:]
    q = q.reshape(Hq, tq, D)
    tkv = 0 if k is None else k.shape[-2]
    for tok in range(tkv):
        pos = count + tok
        if not ring and pos >= size:
            continue
        row = pos % size if ring else pos
        kc[:, row] = np.asarray(k, np.float32).reshape(Hkv, tkv, D)[:, tok].astype(kc.dtype)
        vc[:, row] = np.asarray(v, np.float32).reshape(Hkv, tkv, D)[:, tok].astype(vc.dtype)
    if scale is None:
        scale = 1.0 / np.sqrt(D)
    g = Hq // Hkv
    O = np.zeros((tq, Hq, D))
    for t in range(tq):
        end = count + max(_new_token_end(t, tq, causal, blocks) + tkv - tq, 0)
        p = count + max(t + tkv - tq, 0)
        start = 0 if span == 0 or p < span else p + 1 - span
        js = np.arange(start, end)
        if js.size == 0:
            continue
        rows = js % size if ring else js
        for h in range(Hq):
            kk = kc[h // g, rows].astype(np.float64)
            vv = vc[h // g, rows].astype(np.float64)
            s = scale * (kk @ q[h, t].astype(np.float64))
            e = np.exp(s - s.max())
            O[t, h] = (e @ vv) / e.sum()
    return O.astype(out_dtype), kc, vc


# ---- CPU baseline (cpu_baseline.c): the timed CPU restatement bench.py reports ----

def _f32_or_none(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


def cpu_linear(x, w, bias=None, *, epi="NONE", gated=False, gate_epi="SILU", out=None):
    """fp32 O = epi(x w^T + b) (gated: gate_epi(g) * u over W = [gate; up]),
    x and w fp32 or fp16; M <= 8 takes the streaming GEMV."""
    x, w, bias = _c(x), _c(w), _f32_or_none(bias)
    K, N = w.shape[-1], w.shape[0]
    M = x.size // K
    if out is None:
        out = np.empty((M, N // 2 if gated else N), np.float32)
    lib().cpb_linear(_p(out), _p(x), _dt(x), _p(w), _dt(w), _p(bias), ctypes.c_uint32(M), ctypes.c_uint32(N),
                     ctypes.c_uint32(K), ctypes.c_int(EPILOGUES[epi]), ctypes.c_int(1 if gated else 0),
                     ctypes.c_int(EPILOGUES[gate_epi]))
    return out


def cpu_conv2d(x, w, bias=None, *, stride=1, epi="NONE", out=None):
    """One image x [Ci,Hi,Wi] (or [1,Ci,Hi,Wi]), w [Co,Ci,k,k]: fp32 same-padded conv."""
    x, w, bias = _c(x), _c(w), _f32_or_none(bias)
    Co, Ci, ks, _ = w.shape
    Hi, Wi = x.shape[-2:]
    assert x.size == Ci * Hi * Wi
    Ho, Wo = (Hi - 1) // stride + 1, (Wi - 1) // stride + 1
    if out is None:
        out = np.empty((Co, Ho, Wo), np.float32)
    lib().cpb_conv2d(_p(out), _p(x), _dt(x), _p(w), _dt(w), _p(bias), ctypes.c_uint32(Ci), ctypes.c_uint32(Hi),
                     ctypes.c_uint32(Wi), ctypes.c_uint32(Co), ctypes.c_uint32(ks), ctypes.c_uint32(stride),
                     ctypes.c_int(EPILOGUES[epi]))
    return out


def cpu_attn_scores(q, k, *, scale, causal=True, out=None):
    """fp16 q [H,Tq,D], k [H,Tkv,D] -> fp32 S [H,Tq,Tkv], -inf where hidden."""
    q, k = _c(q), _c(k)
    assert q.dtype == np.float16 and k.dtype == np.float16
    H, Tq, D = q.shape
    Tkv = k.shape[1]
    if out is None:
        out = np.empty((H, Tq, Tkv), np.float32)
    lib().cpb_attn_scores(_p(out), _p(q), _p(k), ctypes.c_uint32(H), ctypes.c_uint32(Tq), ctypes.c_uint32(Tkv),
                          ctypes.c_uint32(D), ctypes.c_float(scale), ctypes.c_int(1 if causal else 0))
    return out


def cpu_attention(q, k, v, *, scale, causal=True, out=None):
    """fp16 q [H,Tq,D], k and v [H,Tkv,D] -> fp32 softmax(scale q k^T + mask) v."""
    q, k, v = _c(q), _c(k), _c(v)
    assert q.dtype == k.dtype == v.dtype == np.float16
    H, Tq, D = q.shape
    Tkv = k.shape[1]
    if out is None:
        out = np.empty((H, Tq, D), np.float32)
    lib().cpb_attention(_p(out), _p(q), _p(k), _p(v), ctypes.c_uint32(H), ctypes.c_uint32(Tq), ctypes.c_uint32(Tkv),
                        ctypes.c_uint32(D), ctypes.c_float(scale), ctypes.c_int(1 if causal else 0))
    return out


def num_threads():
    return lib().orc_num_threads()
