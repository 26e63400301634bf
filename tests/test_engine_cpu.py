"""The engine's host side without a GPU: wiring errors, config checks, host
tensors (the reference's failure paths: neural-net.cpp:341,353 throw on a
cycle or a fan-in; node constructors reject bad configs)."""
import numpy as np
import pytest

from oracle import oracle


@pytest.fixture(scope="module")
def pv():
    from vai_amd import _pyvai
    return _pyvai


def test_cycle_is_rejected(pv):
    class Net(pv.NeuralNet):
        def __init__(self):
            super().__init__()
            self.a = pv.nodes.LinearNode(in_dim=4, out_dim=4)
            self.b = pv.nodes.GatedMulNode()
            self.input("x")
            self.a - self.b
            self.b - self.a
            self.a - self.output("out0")
    net = Net()
    with pytest.raises(RuntimeError, match="cycle"):
        net(x=pv.Tensor.from_numpy(np.zeros((1, 4), np.float32)))


def test_fan_in_is_rejected(pv):
    class Net(pv.NeuralNet):
        def __init__(self):
            super().__init__()
            self.a = pv.nodes.LinearNode(in_dim=4, out_dim=4)
            self.b = pv.nodes.LinearNode(in_dim=4, out_dim=4)
            self.c = pv.nodes.LinearNode(in_dim=4, out_dim=4)
            self.input("x") - self.a - self.c - self.output("out0")
            self.input("y") - self.b - self.c
    net = Net()
    with pytest.raises(RuntimeError, match="more than one producer"):
        net(x=pv.Tensor.from_numpy(np.zeros((1, 4), np.float32)))


def test_only_output_to_input_connections(pv):
    class Net(pv.NeuralNet):
        def __init__(self):
            super().__init__()
            self.a = pv.nodes.LinearNode(in_dim=4, out_dim=4)
    net = Net()
    with pytest.raises(RuntimeError, match="no slot named out0"):
        net.output("o") - net.a            # an OutputNode has no output slot
    with pytest.raises(RuntimeError, match="output slot feeds an input slot"):
        ("in0" / net.a) - ("weight" / net.a)   # in0 is not an output, weight is not an input


@pytest.mark.parametrize("make, msg", [
    (lambda pv: pv.nodes.ConvolutionNode(in_channels=3, out_channels=4, kernel_size=2), "odd"),
    (lambda pv: pv.nodes.ConvolutionNode(in_channels=0, out_channels=4, kernel_size=3), "positive"),
    (lambda pv: pv.nodes.ConvolutionNode(in_channels=3, out_channels=4, kernel_size=3, stride=0), "stride"),
    (lambda pv: pv.nodes.LinearNode(in_dim=0, out_dim=3), "positive"),
    (lambda pv: pv.nodes.AttentionScoresNode(num_q_heads=3, head_dim=8, num_kv_heads=2), "multiple"),
    (lambda pv: pv.nodes.AttentionNode(num_q_heads=3, head_dim=8, num_kv_heads=2), "multiple"),
])
def test_config_checks(pv, make, msg):
    class Net(pv.NeuralNet):
        def __init__(self):
            super().__init__()
            self.n = make(pv)
    with pytest.raises(RuntimeError, match=msg):
        Net()


def test_node_outside_a_net_is_rejected(pv):
    # nodes bind to the net under construction (the reference's thread-local current net)
    import gc
    gc.collect()
    # a fresh thread has no current net
    import threading
    err = []

    def make():
        try:
            pv.nodes.LinearNode(in_dim=2, out_dim=2)
        except RuntimeError as e:
            err.append(str(e))
    t = threading.Thread(target=make)
    t.start()
    t.join()
    assert err and "NeuralNet" in err[0]


def test_host_tensor_roundtrip_and_fp16_rounding(pv):
    x = np.random.default_rng(0).standard_normal((3, 5)).astype(np.float32) * np.float32(3e-5)
    t = pv.Tensor.from_numpy(x)
    assert t.shape == [3, 5] and t.dtype == pv.Dtype.F32
    np.testing.assert_array_equal(t.to_numpy(), x)
    h = pv.Tensor.from_numpy(x, pv.Dtype.F16)
    assert h.dtype == pv.Dtype.F16
    np.testing.assert_array_equal(h.to_numpy().view(np.uint16), oracle.to_f16(x).view(np.uint16))
