"""One-node-net checks through the engine (vai_amd._pyvai), the way the
reference checks its nodes (/root/reference/python/tests/node_check.py:51-96):
draw parameters then inputs from default_rng(seed) as float32, build a net
input -> node -> output, run it, compare with an expected value, check that a
second (replayed) forward is bit-identical and that nothing is NaN/Inf, and
optionally rerun on other inputs (which re-records).
"""
import numpy as np

from helpers import assert_close, draw


def pyvai():
    from vai_amd import _pyvai
    return _pyvai


def build_net(make, slots, params, w_dtype="F32", **net_kw):
    pv = pyvai()

    class Net(pv.NeuralNet):
        def __init__(self):
            super().__init__(w_default_dtype=getattr(pv.Dtype, w_dtype), **net_kw)
            self.node = make()
            self.input(slots[0]) - (slots[0] / self.node) - self.output("out0")
            for slot in slots[1:]:
                self.input(slot) - (slot / self.node)

    net = Net()
    for slot, array in params.items():
        net.node[slot] = pv.Tensor.from_numpy(array)
    return net


def forward(net, fed):
    pv = pyvai()
    out = net(**{slot: pv.Tensor.from_numpy(a) for slot, a in fed.items()})
    return out.to_numpy()


def check_node(make, inputs, ref, *, params=None, tol, input_dtypes=None, alt_inputs=None, seed=0, net_kw=None):
    """inputs/params: {slot: shape or generator}; ref(**fed, **params) -> expected out0.
    input_dtypes: {slot: np.float16} to feed fp16 (rounded as the reference host does)."""
    rng = np.random.default_rng(seed)
    input_dtypes = input_dtypes or {}
    params = {s: draw(g, rng, input_dtypes.get(s, np.float32)) for s, g in (params or {}).items()}
    net = build_net(make, list(inputs), params, **(net_kw or {}))
    fed = {s: draw(g, rng, input_dtypes.get(s, np.float32)) for s, g in inputs.items()}
    got = forward(net, fed)
    assert_close(got.astype(np.float32), ref(**fed, **params), tol, "out0 vs the reference")
    again = forward(net, fed)
    np.testing.assert_array_equal(again, got, err_msg="the second forward differs from the first")
    assert np.isfinite(got.astype(np.float64)).all(), "out0 has NaN or Inf"
    if alt_inputs:
        fed = {s: draw(g, rng, input_dtypes.get(s, np.float32)) for s, g in alt_inputs.items()}
        assert_close(forward(net, fed).astype(np.float32), ref(**fed, **params), tol, "rerun on alt_inputs")
    return net
