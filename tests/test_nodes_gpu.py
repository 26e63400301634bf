"""Nodes through the engine on the MI355X, as the reference tests them
(/root/reference/python/tests/nodes/test_linear.py:11-84,
test_convolution.py:12-87, test_gated_mul.py): one-node nets built with the
`-` wiring DSL, float64 expectations, a bit-identical replayed second forward,
and a rerun on other shapes. Plus what is new here: the record-once/replay
graph, the Linear -> GatedMul fusion, the attention-scores node.
"""
import numpy as np
import pytest

from helpers import FP16, FP32, TRANS, assert_close, draw, normal, np_epilogue, uniform
from node_check import build_net, check_node, forward, pyvai
from oracle import oracle

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize(
    "m, k, n, has_bias, epilogue, split_size, tol, alt_m",
    [
        (1, 64, 32, True, "NONE", 0, FP32, 33),   # rerun: slab -> tile
        (8, 96, 40, False, "NONE", 0, FP32, None),
        (33, 96, 48, True, "RELU", 0, FP32, None),
        (64, 128, 100, False, "GELU_TANH", 0, TRANS, None),
        (16, 256, 64, True, "NONE", 64, FP32, None),
        (33, 1000, 100, True, "NONE", 0, FP32, None),
        (33, 100, 48, False, "NONE", 0, FP32, None),
        (33, 102, 48, False, "NONE", 0, FP32, None),
        (33, 101, 48, False, "NONE", 0, FP32, None),
        (16, 2050, 64, True, "NONE", 0, FP32, None),
        (33, 1000, 48, False, "NONE", 100, FP32, None),
    ],
)
def test_linear_node(gpu, m, k, n, has_bias, epilogue, split_size, tol, alt_m):
    pv = pyvai()
    params = {"weight": normal((n, k), 1.0 / np.sqrt(k))}
    if has_bias:
        params["bias"] = (n,)

    def ref(in0, weight, bias=None):
        y = in0.astype(np.float64) @ weight.astype(np.float64).T
        if bias is not None:
            y = y + bias
        return np_epilogue(epilogue, y)

    check_node(lambda: pv.nodes.LinearNode(in_dim=k, out_dim=n, epilogue=getattr(pv.Epilogue, epilogue),
                                           split_size=split_size),
               {"in0": (m, k)}, ref, params=params, tol=tol,
               alt_inputs={"in0": (alt_m, k)} if alt_m else None)


@pytest.mark.parametrize("m, order", [(4, "AFTER_EPILOGUE"), (4, "BEFORE_EPILOGUE"),
                                      (33, "AFTER_EPILOGUE"), (33, "BEFORE_EPILOGUE")])
def test_linear_node_residual(gpu, m, order):
    pv = pyvai()
    k, n = 64, 48

    def ref(in0, residual, weight, bias):
        y = in0.astype(np.float64) @ weight.astype(np.float64).T + bias
        if order == "BEFORE_EPILOGUE":
            return np.maximum(y + residual, 0)
        return np.maximum(y, 0) + residual

    check_node(lambda: pv.nodes.LinearNode(in_dim=k, out_dim=n, accept_residual=True,
                                           residual_order=getattr(pv.ResidualOrder, order), epilogue=pv.Epilogue.RELU),
               {"in0": (m, k), "residual": (m, n)}, ref,
               params={"weight": normal((n, k), 1.0 / np.sqrt(k)), "bias": (n,)}, tol=FP32)


@pytest.mark.parametrize("ci, co, ks, stride, hw, epi, w16", [
    (16, 32, 1, 1, 12, "NONE", False), (8, 16, 3, 1, 12, "RELU", False), (8, 16, 3, 1, 28, "SILU", False),
    (8, 16, 3, 2, 13, "NONE", False), (4, 8, 5, 1, 11, "GELU", False), (32, 48, 3, 1, 20, "SILU", True),
    (24, 40, 1, 1, 17, "SIGMOID", True)])
def test_convolution_node(gpu, ci, co, ks, stride, hw, epi, w16):
    pv = pyvai()
    dts = {"weight": np.float16, "bias": np.float16, "in0": np.float16} if w16 else {}

    def ref(in0, weight, bias):
        return np.asarray(oracle.conv2d(in0, weight, bias, stride=stride, epi=epi), np.float64)

    check_node(lambda: pv.nodes.ConvolutionNode(in_channels=ci, out_channels=co, kernel_size=ks, stride=stride,
                                                epilogue=getattr(pv.Epilogue, epi)),
               {"in0": (2, ci, hw, hw)}, ref,
               params={"weight": normal((co, ci, ks, ks), 1.0 / np.sqrt(ci * ks * ks)), "bias": normal((co,), 0.1)},
               tol=FP16 if w16 else TRANS, input_dtypes=dts,
               alt_inputs={"in0": (1, ci, hw + 2, hw + 1)},
               net_kw={"w_dtype": "F16" if w16 else "F32"})


def test_gated_mul_node(gpu):
    pv = pyvai()
    check_node(lambda: pv.nodes.GatedMulNode(activation=pv.Epilogue.GELU), {"in0": (5, 2 * 24)},
               lambda in0: np_epilogue("GELU", in0[:, :24]) * in0[:, 24:], tol=TRANS)


def _ffn_net(pv, k, h, fuse):
    class Net(pv.NeuralNet):
        def __init__(self):
            super().__init__(w_default_dtype=pv.Dtype.F16, fuse_gated_linear=fuse)
            self.gate_up = pv.nodes.LinearNode(in_dim=k, out_dim=2 * h)
            self.glu = pv.nodes.GatedMulNode(activation=pv.Epilogue.SILU)
            self.input("in0") - self.gate_up - self.glu - self.output("out0")
    return Net()


@pytest.mark.parametrize("m, k, h", [(6, 256, 96), (300, 512, 160), (1024, 512, 512)])
def test_gated_ffn_fusion(gpu, m, k, h):
    """gate/up Linear -> GatedMul (gated-feed-forward.h:37-46): fused at record
    time into one gated GEMM; same result as the two-kernel path."""
    pv = pyvai()
    rng = np.random.default_rng(0)
    w = draw(normal((2 * h, k), 0.05), rng, np.float16)
    b = draw(normal((2 * h,), 0.05), rng, np.float16)
    x = draw((m, k), rng, np.float16)
    outs = {}
    for fuse in (True, False):
        net = _ffn_net(pv, k, h, fuse)
        net.gate_up["weight"] = pv.Tensor.from_numpy(w)
        net.gate_up["bias"] = pv.Tensor.from_numpy(b)
        outs[fuse] = forward(net, {"in0": x})
        assert net.gate_up.fused == fuse
    want = oracle.gated_mul(oracle.linear(x, w, b), epi="SILU")
    assert_close(outs[True], want, TRANS)
    assert_close(outs[False], want, TRANS)


def test_replay_and_rerecord(gpu):
    """Same shapes replay the recorded HIP graph; a new shape records again."""
    pv = pyvai()
    rng = np.random.default_rng(0)
    w = draw(normal((64, 128), 0.1), rng)
    net = build_net(lambda: pv.nodes.LinearNode(in_dim=128, out_dim=64, epilogue=pv.Epilogue.SILU), ["in0"],
                    {"weight": w})
    x1, x2, x3 = (draw((40, 128), rng) for _ in range(3))
    y1 = forward(net, {"in0": x1})
    assert net.record_count == 1
    y2 = forward(net, {"in0": x2})                   # new data, same shape: replay
    assert net.record_count == 1
    assert_close(y2, oracle.linear(x2, w, epi="SILU"), TRANS)
    y3 = forward(net, {"in0": x3[:7]})               # new shape: record again (and the slab path)
    assert net.record_count == 2
    assert_close(y3, oracle.linear(x3[:7], w, epi="SILU"), TRANS)
    assert_close(y1, oracle.linear(x1, w, epi="SILU"), TRANS)
    assert net.submit_count == 3


@pytest.mark.parametrize("hq, hkv, tq, tkv, d, causal", [(4, 4, 64, 64, 64, True), (4, 2, 50, 80, 128, True),
                                                         (2, 1, 33, 33, 32, False)])
def test_attention_scores_node(gpu, hq, hkv, tq, tkv, d, causal):
    pv = pyvai()
    rng = np.random.default_rng(0)
    q = draw((2, hq, tq, d), rng, np.float16)
    k = draw((2, hkv, tkv, d), rng, np.float16)
    net = build_net(lambda: pv.nodes.AttentionScoresNode(num_q_heads=hq, head_dim=d, num_kv_heads=hkv, causal=causal),
                    ["in0", "K"], {})
    got = forward(net, {"in0": q, "K": k})
    assert_close(got, oracle.attn_scores(q, k, causal=causal), FP32)


@pytest.mark.parametrize("hq, hkv, tq, tkv, d, causal, span, qdt, kvdt", [
    (4, 2, 100, 100, 128, True, 0, np.float16, np.float16),
    (2, 2, 64, 1000, 64, False, 0, np.float16, np.float16),
    (2, 1, 257, 257, 64, True, 50, np.float16, np.float16),
    (16, 16, 729, 729, 72, False, 0, np.float32, np.float32),   # SigLIP: Dh 72, fp32 Linear outputs, no mask
    (4, 2, 90, 90, 128, True, 0, np.float32, np.float16),       # fp32 Q, K / V in the cache dtype
    (2, 2, 30, 30, 20, True, 0, np.float32, np.float32),        # Dh 20: the plain kernel
])
def test_attention_node(gpu, hq, hkv, tq, tkv, d, causal, span, qdt, kvdt):
    """The engine's Attention node (Q, K, V -> out0 [..., Tq, Hq, D]) with the
    reference's Config and setCausalMask; the key-split partials and fp16
    K / V copies bind to the "partialO" temporary when the launch needs them."""
    pv = pyvai()
    rng = np.random.default_rng(3)
    q = draw((1, hq, tq, d), rng, qdt)
    k = draw((1, hkv, tkv, d), rng, kvdt)
    v = draw((1, hkv, tkv, d), rng, kvdt)
    net = build_net(lambda: pv.nodes.AttentionNode(num_q_heads=hq, head_dim=d, num_kv_heads=hkv), ["Q", "K", "V"], {})
    if causal or span:
        net.node.set_causal_mask(1 if causal else 0, [], span=span)
    got = forward(net, {"Q": q, "K": k, "V": v}).astype(np.float32)
    assert got.shape == (1, tq, hq, d)
    assert_close(got, oracle.attention(q, k, v, causal=causal, span=span, out_dtype=np.float32), FP16)


def test_attention_node_no_mask_by_default(gpu):
    """Without setCausalMask every query attends every key (attention.h:129):
    the first query's output is not V's first row."""
    pv = pyvai()
    rng = np.random.default_rng(8)
    q, k, v = (draw((1, 2, 40, 64), rng, np.float16) for _ in range(3))
    net = build_net(lambda: pv.nodes.AttentionNode(num_q_heads=2, head_dim=64), ["Q", "K", "V"], {})
    got = forward(net, {"Q": q, "K": k, "V": v}).astype(np.float32)
    assert_close(got, oracle.attention(q, k, v, out_dtype=np.float32), FP16)
    assert not np.allclose(got[0, 0, 0], v[0, 0, 0], atol=1e-2)


def test_attention_node_block_mask(gpu):
    """setCausalMask on the Attention and AttentionScores nodes: a prefix-LM
    mask, then a three-block mask set after the first forward (re-records)."""
    pv = pyvai()
    rng = np.random.default_rng(5)
    hq, tq, d = 2, 150, 64
    q = draw((1, hq, tq, d), rng, np.float16)
    k = draw((1, hq, tq, d), rng, np.float16)
    v = draw((1, hq, tq, d), rng, np.float16)
    net = build_net(lambda: pv.nodes.AttentionNode(num_q_heads=hq, head_dim=d), ["Q", "K", "V"], {})
    net.node.set_causal_mask(0b01, [40])
    got = forward(net, {"Q": q, "K": k, "V": v})
    assert_close(got, oracle.attention(q, k, v, blocks=(0b01, [40]), out_dtype=np.float32), FP16)
    net.node.set_causal_mask(0b101, [30, 90], span=70)
    got = forward(net, {"Q": q, "K": k, "V": v})
    assert_close(got, oracle.attention(q, k, v, blocks=(0b101, [30, 90]), span=70, out_dtype=np.float32), FP16)
    sn = build_net(lambda: pv.nodes.AttentionScoresNode(num_q_heads=hq, head_dim=d), ["in0", "K"], {})
    sn.node.set_causal_mask(0b01, [40])
    got = forward(sn, {"in0": q[0], "K": k[0]})
    assert_close(got, oracle.attn_scores(q[0], k[0], blocks=(0b01, [40])), FP32)


def test_gpt2_cfc_through_the_engine(gpu):
    """BASELINE config 1 via input - linear - output."""
    import os, sys
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
    import configs as C
    G = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "baseline_configs.npz"))
    pv = pyvai()
    x, w, b = C.cfg1()
    net = build_net(lambda: pv.nodes.LinearNode(in_dim=768, out_dim=3072, epilogue=pv.Epilogue.GELU_TANH), ["in0"],
                    {"weight": w, "bias": b})
    got = forward(net, {"in0": x})
    assert net.node.plan.startswith("tile_f32")
    assert_close(got[C.CFG1_ROWS], G["cfg1_rows"], FP32)


def test_linear_node_packs_prefill_weight(gpu):
    """A prefill-sized fp16 Linear packs its weight once at prepare and runs
    the packed-weight GEMM; decode-sized inputs on the same net take the
    GEMV; a new weight tensor is packed again."""
    pv = pyvai()
    rng = np.random.default_rng(0)
    m, k, n = 1024, 512, 8192
    w = draw(normal((n, k), 0.05), rng, np.float16)
    b = draw(normal((n,), 0.05), rng, np.float16)
    x = draw((m, k), rng, np.float16)
    net = build_net(lambda: pv.nodes.LinearNode(in_dim=k, out_dim=n, epilogue=pv.Epilogue.GELU_TANH),
                    ["in0"], {"weight": w, "bias": b}, w_dtype="F16")
    got = forward(net, {"in0": x})
    assert net.node.plan == "tile_f16_256x256_packed", net.node.plan
    rows = np.unique(np.concatenate([np.arange(4), np.arange(m - 4, m), rng.choice(m, 16, replace=False)]))
    assert_close(got[rows], oracle.linear(x[rows], w, b, epi="GELU_TANH", stage="tile"), TRANS)
    # decode shape on the same net: the slab GEMV on the unpacked weight
    xs = draw((2, k), rng, np.float16)
    got_s = forward(net, {"in0": xs})
    assert net.node.plan.startswith("slab"), net.node.plan
    assert_close(got_s, oracle.linear(xs, w, b, epi="GELU_TANH"), TRANS)
    # a new weight is packed again
    w2 = draw(normal((n, k), 0.05), rng, np.float16)
    net.node["weight"] = pv.Tensor.from_numpy(w2)
    got2 = forward(net, {"in0": x})
    assert net.node.plan == "tile_f16_256x256_packed"
    assert_close(got2[rows], oracle.linear(x[rows], w2, b, epi="GELU_TANH", stage="tile"), TRANS)


def test_gated_ffn_packed_fusion(gpu):
    """The fused gate/up GEMM at prefill size runs on the packed weight (the
    gated layout), equal to the unfused two-kernel path bit for bit."""
    pv = pyvai()
    rng = np.random.default_rng(0)
    m, k, h = 2048, 512, 4096
    w = draw(normal((2 * h, k), 0.05), rng, np.float16)
    x = draw((m, k), rng, np.float16)
    outs = {}
    for fuse in (True, False):
        net = _ffn_net(pv, k, h, fuse)
        net.gate_up["weight"] = pv.Tensor.from_numpy(w)
        outs[fuse] = forward(net, {"in0": x})
        assert net.gate_up.plan == ("tile_f16_256x256_packed_gated" if fuse else "tile_f16_256x256_packed")
    rows = np.unique(np.concatenate([np.arange(4), np.arange(m - 4, m), rng.choice(m, 16, replace=False)]))
    want = oracle.gated_mul(oracle.linear(x[rows], w, stage="tile"), epi="SILU")
    assert_close(outs[True][rows], want, TRANS)
    assert_close(outs[False][rows], want, TRANS)


def test_linear_node_acc16(gpu):
    """Linear::setAccDtype(Fp16) through the engine: the node's plan switches to
    the fp16-accumulating kernel and its output equals the oracle's fma chain."""
    pv = pyvai()
    rng = np.random.default_rng(0)
    m, k, n = 40, 320, 72
    w = draw(normal((n, k), 0.05), rng, np.float16)
    b = draw((n,), rng)
    x = draw((m, k), rng, np.float16)
    net = build_net(lambda: pv.nodes.LinearNode(in_dim=k, out_dim=n), ["in0"], {"weight": w, "bias": b}, w_dtype="F16")
    net.set_acc_dtype(net.node, pv.Dtype.F16)
    got = forward(net, {"in0": x})
    assert net.node.plan == "tile_acc16_64x64"
    assert np.array_equal(got, oracle.linear_acc16(x, w, b))
    net.set_acc_dtype(net.node, pv.Dtype.F32)   # back to fp32: re-records with the MFMA tile
    got = forward(net, {"in0": x})
    assert net.node.plan.startswith("tile_f16")
    assert_close(got, oracle.linear(x, w, b, stage="tile"), FP32)


def test_attention_node_kv_cache(gpu):
    """The Attention node with its KV cache, run as a decoder runs it
    (attention.h:108-140, 242-246): a prompt, then one-token steps, the model
    rewriting the counter before each forward. The second one-token forward
    has the first's shapes, so it replays the recorded launches: the count the
    kernels read is the live one. Each output matches the reference's
    formulas over the cache the earlier forwards left, and the node's cache
    holds every appended K / V row."""
    pv = pyvai()
    rng = np.random.default_rng(21)
    hq, hkv, d, size = 8, 4, 128, 256
    net = build_net(lambda: pv.nodes.AttentionNode(num_q_heads=hq, head_dim=d, num_kv_heads=hkv, kv_cache_size=size,
                                                   kv_cache_dtype=pv.Dtype.F16), ["Q", "K", "V"], {})
    net.node.set_causal_mask(1, [])
    counter = gpu.DeviceArray((1,), np.uint32)
    net.node.set_kv_cache_counter(counter.ptr)
    kc = np.full((hkv, size, d), np.nan, np.float16)
    vc = kc.copy()
    count = 0
    for t in (20, 1, 1, 3):
        gpu.lib().vai_memcpy_h2d(counter.ptr, np.array([count], np.uint32).ctypes.data, 4, None)
        q = draw((1, hq, t, d), rng, np.float16)
        k = draw((1, hkv, t, d), rng, np.float16)
        v = draw((1, hkv, t, d), rng, np.float16)
        print(f"kv cache node: count {count}, {t} new tokens", flush=True)
        got = forward(net, {"Q": q, "K": k, "V": v}).astype(np.float32)
        want, kc, vc = oracle.attention_cached(q[0], k, v, kc, vc, count, causal=True)
        assert_close(got[0], want, FP16)
        count += t
    np.testing.assert_array_equal(net.node["K_cache"].to_numpy()[:, :count], kc[:, :count])
    np.testing.assert_array_equal(net.node["V_cache"].to_numpy()[:, :count], vc[:, :count])


def test_attention_node_kv_cache_alone_and_ring(gpu):
    """K / V unwired: the node attends the cache alone (Tkv = 0,
    attention.h:1001-1004); a ring rounds its size up to 256 (kvRingAlign)."""
    pv = pyvai()
    rng = np.random.default_rng(22)
    hq, d = 4, 64
    ring = build_net(lambda: pv.nodes.AttentionNode(num_q_heads=hq, head_dim=d, kv_cache_size=100,
                                                    kv_cache_dtype=pv.Dtype.F16, kv_cache_ring=True), ["Q", "K", "V"], {})
    assert ring.node.kv_cache_size == 256
    assert ring.node["K_cache"].shape == [hq, 256, d]
    net = build_net(lambda: pv.nodes.AttentionNode(num_q_heads=hq, head_dim=d, kv_cache_size=64,
                                                   kv_cache_dtype=pv.Dtype.F32), ["Q"], {})
    counter = gpu.DeviceArray.from_numpy(np.array([0], np.uint32))
    net.node.set_kv_cache_counter(counter.ptr)
    # the cache planes set directly (a persistent slot, uploaded at the next
    # forward), then a forward that attends 37 cached rows
    kc = draw((hq, 64, d), rng, np.float32)
    vc = draw((hq, 64, d), rng, np.float32)
    net.node["K_cache"] = pv.Tensor.from_numpy(kc)
    net.node["V_cache"] = pv.Tensor.from_numpy(vc)
    gpu.lib().vai_memcpy_h2d(counter.ptr, np.array([37], np.uint32).ctypes.data, 4, None)
    q = draw((1, hq, 2, d), rng, np.float16)
    got = forward(net, {"Q": q}).astype(np.float32)
    want, _, _ = oracle.attention_cached(q[0], None, None, kc, vc, 37)
    assert_close(got[0], want, FP16)
