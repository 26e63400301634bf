"""Writes tests/golden/baseline_configs.npz: expected outputs of the five
BASELINE configs in float64 closed form (numpy only; no oracle, no reference).

    python tests/golden/gen_golden.py
"""
import math
import os
import sys

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import configs as C  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "baseline_configs.npz")


def gelu_tanh(y):
    return 0.5 * y * (1 + np.tanh(math.sqrt(2 / math.pi) * (y + 0.044715 * y ** 3)))


def silu(y):
    return y / (1 + np.exp(-y))


def main():
    g = {}
    x, w, b = C.cfg1()
    y = gelu_tanh(x.astype(np.float64) @ w.astype(np.float64).T + b)
    g["cfg1_rows"] = y[C.CFG1_ROWS]
    g["cfg1_rowsum"] = y.sum(axis=1)

    x, w = C.cfg2()
    y = x.astype(np.float64) @ w.astype(np.float64).T
    g["cfg2_out"] = y                      # [8, 8192]; M=1 and M=4 are its leading rows

    x, w = C.cfg3()
    y = x.astype(np.float64) @ w.astype(np.float64).T
    o = silu(y[:, :8192]) * y[:, 8192:]
    g["cfg3_rows"] = o[C.CFG3_ROWS]
    g["cfg3_rowsum"] = o.sum(axis=1)
    del y, o

    q, k = C.cfg4()
    i, j = np.indices((1024, 1024))
    rows, sums = [], []
    for h in range(8):
        s = (q[h].astype(np.float64) @ k[h].astype(np.float64).T) / 16.0
        sums.append(np.where(j <= i, s, 0.0).sum(axis=1))
        if h in C.CFG4_HEADS:
            rows.append(np.where(j <= i, s, -np.inf)[C.CFG4_QROWS])
    g["cfg4_rows"] = np.stack(rows)
    g["cfg4_visible_rowsum"] = np.stack(sums)

    x, w, b = C.cfg5()
    xp = np.pad(x[0].astype(np.float64), ((0, 0), (1, 1), (1, 1)))
    out = np.zeros((128, 80, 80))
    w64 = w.astype(np.float64)
    for kh in range(3):
        for kw in range(3):
            out += np.einsum("oc,chw->ohw", w64[:, :, kh, kw], xp[:, kh:kh + 80, kw:kw + 80])
    out = silu(out + b.astype(np.float64)[:, None, None])
    g["cfg5_channels"] = out[C.CFG5_CHANNELS]
    g["cfg5_chansum"] = out.sum(axis=(1, 2))

    np.savez_compressed(OUT, **g)
    print("wrote", OUT, {k: v.shape for k, v in g.items()})


if __name__ == "__main__":
    main()
