"""Checkpoint ingest (the reference's vai/engine/safetensors-parser.*,
weights.h:38-70) on the host: tests/cpp/safetensors_read opens a checkpoint
folder of .safetensors shards written here by the safetensors package, loads
every tensor as an engine Tensor and writes its values back; they must equal
what was saved (exactly for same-width or widening conversions, the engine's
fp32 -> fp16 rounding for narrowing). Malformed files must be refused with
the reference's error wording.
"""
import json
import os
import struct
import subprocess

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "_bin", "safetensors_read")


def run(ckpt, out, dt):
    return subprocess.run([BIN, str(ckpt), str(out), dt], capture_output=True, text=True, timeout=60)


@pytest.fixture
def ckpt(tmp_path):
    rng = np.random.default_rng(0)
    d = tmp_path / "ckpt"
    d.mkdir()
    t = {
        "a.weight": torch.from_numpy(rng.standard_normal((48, 32)).astype(np.float16)),
        "a.bias": torch.from_numpy(rng.standard_normal(48).astype(np.float32)),
    }
    u = {
        "b.weight": torch.from_numpy(rng.standard_normal((16, 8)).astype(np.float32)).to(torch.bfloat16),
        "scale": torch.tensor(0.5, dtype=torch.float32),
    }
    save_file(t, str(d / "model-00001-of-00002.safetensors"), metadata={"format": "pt"})
    save_file(u, str(d / "model-00002-of-00002.safetensors"))
    (d / "notes.txt").write_text("not a shard")
    return d, {**t, **u}


def test_program_is_built():
    assert os.access(BIN, os.X_OK), "tests/cpp/_bin/safetensors_read missing: run __graft_entry__.build()"


@pytest.mark.parametrize("dt", ["f32", "f16"])
def test_checkpoint_roundtrip(ckpt, tmp_path, dt):
    d, saved = ckpt
    out = tmp_path / "out"
    out.mkdir()
    r = run(d, out, dt)
    assert r.returncode == 0, r.stderr
    lines = r.stdout.splitlines()
    listed = {l.split()[1]: l.split()[2:] for l in lines if l.startswith("tensor ")}
    assert sorted(listed) == sorted(saved)
    assert listed["a.weight"] == ["F16", "48x32", str(48 * 32 * 2)]
    assert listed["b.weight"] == ["BF16", "16x8", str(16 * 8 * 2)]
    assert listed["scale"] == ["F32", "scalar", "4"]
    assert "partial=ok" in lines and "overrun=refused" in lines
    assert any(l.startswith("missing=") and "no.such.tensor" in l for l in lines)
    for name, t in saved.items():
        got = np.fromfile(out / f"{name}.f32", np.float32)
        want = t.to(torch.float32).numpy().reshape(-1)
        if dt == "f16":
            # the engine rounds fp32 -> fp16 to nearest even (values here are normal fp16)
            want = want.astype(np.float16).astype(np.float32)
        np.testing.assert_array_equal(got, want, err_msg=name)


def write_raw(path, header, data):
    h = json.dumps(header).encode()
    path.write_bytes(struct.pack("<Q", len(h)) + h + data)


@pytest.mark.parametrize("case, msg", [
    ("header_past_end", "Failed to read header string"),
    ("size_mismatch", "Data size mismatch"),
    ("bad_json", "Invalid Safetensors header"),
    ("bad_offsets", "bad data_offsets"),
])
def test_malformed_files_are_refused(tmp_path, case, msg):
    d = tmp_path / "bad"
    d.mkdir()
    f = d / "x.safetensors"
    if case == "header_past_end":
        f.write_bytes(struct.pack("<Q", 1 << 20) + b"{}")
    elif case == "size_mismatch":
        write_raw(f, {"w": {"dtype": "F32", "shape": [4, 4], "data_offsets": [0, 60]}}, bytes(60))
    elif case == "bad_json":
        h = b'{"w": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]'   # unterminated
        f.write_bytes(struct.pack("<Q", len(h)) + h + bytes(8))
    else:
        write_raw(f, {"w": {"dtype": "F32", "shape": [2], "data_offsets": [8, 0]}}, bytes(8))
    r = run(d, tmp_path, "f32")
    assert r.returncode == 1 and msg in r.stderr, (r.returncode, r.stderr)


def test_empty_folder_is_refused(tmp_path):
    r = run(tmp_path, tmp_path, "f32")
    assert r.returncode == 1 and "no *.safetensors" in r.stderr
