"""The engine driven from C++ as a model net drives it: tests/cpp/gated_ffn_net
builds `input - Linear(K -> 2H, bias) - GatedMul(SiLU) - output` with the
reference's member-node style (gated-feed-forward.h:23-54), runs it twice
(record, then replay), and the result is checked against the oracle.
"""
import os
import subprocess

import numpy as np
import pytest

from helpers import FP16, TRANS, assert_close, draw, normal
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


BLOCK = os.path.join(os.path.dirname(BIN), "gated_ffn_block")


@pytest.mark.gpu
@pytest.mark.parametrize("m, k, h, n, residual, act, odt, plans", [
    (4, 256, 128, 96, True, "silu", "f32", ("slab", "slab")),
    (64, 256, 192, 160, False, "gelu_tanh", "f32", ("tile", "tile")),
    (300, 512, 256, 384, True, "silu", "f16", ("tile", "tile")),
    (2048, 3072, 8192, 3072, True, "silu", "f16", ("tile_f16_256x256", "tile")),   # Llama-3.2-3B FFN
])
def test_gated_ffn_block_from_cpp(gpu, tmp_path, m, k, h, n, residual, act, odt, plans):
    """vai::group::GatedFeedForward (gated-feed-forward.h:23-54): fused
    gate/value projection + GLU, then the output projection with the skip add
    folded in, recorded once and replayed; vs the oracle on sampled rows."""
    rng = np.random.default_rng(0)
    w1 = draw(normal((2 * h, k), 0.05), rng, np.float16)
    w2 = draw(normal((n, h), 0.05), rng, np.float16)
    x = draw((m, k), rng, np.float16)
    out_dt = np.float16 if odt == "f16" else np.float32
    r = draw((m, n), rng, out_dt) if residual else None
    for name, a in (("x", x), ("w1", w1), ("w2", w2), ("r", r)):
        if a is not None:
            a.astype(np.float32).tofile(tmp_path / f"{name}.f32")
    args = [BLOCK, str(tmp_path), str(m), str(k), str(h), str(n), str(int(residual)), act, odt]
    print(" ".join(args[2:]), flush=True)
    p = subprocess.run(args, capture_output=True, text=True, timeout=100)
    assert p.returncode == 0, p.stderr
    info = dict(kv.split("=") for kv in p.stdout.split())
    assert info["plan1"].startswith(plans[0]) and info["plan2"].startswith(plans[1]), info
    assert info["fused"] == "1" and info["records"] == "1" and info["submits"] == "2", info
    got = np.fromfile(tmp_path / "y.f32", np.float32).reshape(m, n)
    rows = np.arange(m) if m <= 300 else np.unique(np.concatenate(
        [np.arange(4), np.arange(m - 4, m), np.random.default_rng(1).choice(m, 24, replace=False)]))
    epi = "SILU" if act == "silu" else "GELU_TANH"
    hid = oracle.gated_mul(oracle.linear(x[rows], w1, stage="tile" if m > 8 else "slab"), epi=epi, out_dtype=out_dt)
    want = oracle.linear(hid, w2, None, r[rows] if residual else None, out_dtype=out_dt,
                         stage="tile" if m > 8 else "slab")
    # Past the slab path the output projection stages its fp32 input as fp16
    # (linear-tile.comp); the GLU's transcendental rounding (TRANS) can then
    # move a staged value by one fp16 ulp, so those cases take the fp16 tier.
    assert_close(got[rows], want.astype(np.float32), FP16 if (odt == "f16" or m > 8) else TRANS)


def test_cpp_block_program_is_built():
    assert os.access(BLOCK, os.X_OK), "tests/cpp/_bin/gated_ffn_block missing: run __graft_entry__.build()"


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_gated_ffn_block_from_checkpoint(gpu, tmp_path, dtype):
    """Weights ingested from a sharded .safetensors checkpoint (Llama MLP
    names, bf16 or fp16 as published) into the GatedFeedForward block, then
    run on the GPU; vs the oracle on the weights as the engine stores them
    (fp16)."""
    import torch
    from safetensors.torch import save_file
    m, k, h, n = 256, 512, 768, 384
    rng = np.random.default_rng(4)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    g = torch.from_numpy(rng.standard_normal((h, k)).astype(np.float32) * 0.05).to(tdt)
    u = torch.from_numpy(rng.standard_normal((h, k)).astype(np.float32) * 0.05).to(tdt)
    dn = torch.from_numpy(rng.standard_normal((n, h)).astype(np.float32) * 0.05).to(tdt)
    ck = tmp_path / "ckpt"
    ck.mkdir()
    save_file({"mlp.gate_proj.weight": g, "mlp.up_proj.weight": u}, str(ck / "model-00001-of-00002.safetensors"))
    save_file({"mlp.down_proj.weight": dn}, str(ck / "model-00002-of-00002.safetensors"))
    x = draw((m, k), rng, np.float16)
    x.astype(np.float32).tofile(tmp_path / "x.f32")
    args = [BLOCK, str(tmp_path), str(m), str(k), str(h), str(n), "0", "silu", "f16", str(ck)]
    print(" ".join(args[2:]), flush=True)
    p = subprocess.run(args, capture_output=True, text=True, timeout=100)
    assert p.returncode == 0, p.stderr
    got = np.fromfile(tmp_path / "y.f32", np.float32).reshape(m, n)
    # the engine holds the weights as fp16: bf16 values round to nearest even
    as16 = lambda t: t.to(torch.float32).numpy().astype(np.float16)
    w1 = np.concatenate([as16(g), as16(u)], 0)
    hid = oracle.gated_mul(oracle.linear(x, w1, stage="tile"), epi="SILU", out_dtype=np.float16)
    want = oracle.linear(hid, as16(dn), out_dtype=np.float16, stage="tile")
    assert_close(got, want.astype(np.float32), FP16)
