"""The engine driven from C++ as a model net drives it: tests/cpp/gated_ffn_net
builds `input - Linear(K -> 2H, bias) - GatedMul(SiLU) - output` with the
reference's member-node style (gated-feed-forward.h:23-54), runs it twice
(record, then replay), and the result is checked against the oracle.
"""
import os
import subprocess

import numpy as np
import pytest

from helpers import TRANS, assert_close, draw, normal
from oracle import oracle

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "_bin", "gated_ffn_net")


def test_cpp_program_is_built():
    assert os.access(BIN, os.X_OK), "tests/cpp/_bin/gated_ffn_net missing: run __graft_entry__.build()"


@pytest.mark.gpu
@pytest.mark.parametrize("m, k, h, plan", [(4, 256, 96, "slab"), (300, 512, 160, "tile"), (1024, 1024, 1024, "tile")])
def test_gated_ffn_net_from_cpp(gpu, tmp_path, m, k, h, plan):
    rng = np.random.default_rng(0)
    w = draw(normal((2 * h, k), 0.05), rng, np.float16)
    b = draw(normal((2 * h,), 0.05), rng, np.float16)
    x = draw((m, k), rng, np.float16)
    for name, a in (("x", x), ("w", w), ("b", b)):
        a.astype(np.float32).tofile(tmp_path / f"{name}.f32")
    print(f"gated_ffn_net M={m} K={k} H={h}", flush=True)
    r = subprocess.run([BIN, str(tmp_path), str(m), str(k), str(h)], capture_output=True, text=True, timeout=100)
    assert r.returncode == 0, r.stderr
    info = dict(kv.split("=") for kv in r.stdout.split())
    assert info["plan"].startswith(plan), info
    assert info["fused"] == "1" and info["records"] == "1" and info["submits"] == "2", info
    got = np.fromfile(tmp_path / "y.f32", np.float32).reshape(m, h)
    want = oracle.gated_mul(oracle.linear(x, w, b), epi="SILU")
    assert_close(got, want, TRANS)


@pytest.mark.gpu
def test_mfma_rate_program(gpu):
    """tests/cpp/mfma_rate measures the fp16 MFMA ceiling with constant and
    with random operands (the roofline figures in the bench notes come from
    it); here it runs briefly and must report six positive rates."""
    exe = os.path.join(os.path.dirname(BIN), "mfma_rate")
    r = subprocess.run([exe, "200"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    rates = [float(l.split(",")[1].split()[0]) for l in r.stdout.splitlines() if "TFLOP/s" in l]
    assert len(rates) == 12 and all(v > 0 for v in rates), r.stdout
