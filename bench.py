#!/usr/bin/env python3
"""Benchmark of vAi's matmul hot path on one MI355X (BASELINE.json's metric).

A "step" is one pass of the hot path over one batch of synthetic input: one
launch of the configuration's kernel(s) through the C ABI. K steps are
captured into one HIP graph (the replay form of the reference's recorded
command buffer) and timed with HIP events on the stream they run on, with
inputs already resident in HBM. Bandwidth-bound configurations rotate through
enough copies of their streamed operand (>= 384 MB) that the 256 MB Infinity
Cache cannot hold them between launches.

`value` is configs[1] of BASELINE.json -- the Llama-3.2-1B decode GEMV at
M=1, in HBM GB/s; the prefill GEMM TFLOP/s (config 3) and the other configs
are reported under "configs" with their own rooflines.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "Linear GEMM TFLOP/s (% MFMA peak) + decode GEMV HBM GB/s (% peak)"
HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2500.0
FP32_PEAK_TFLOPS = 157.3
ROTATE_BYTES = 384 << 20
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "l2_miss_traffic.tsv")
# rocprofv3 counter scale factors on gfx950, measured with GatedMul over a
# [4096, 4096] fp32 input (reads exactly 64 MiB, writes 32 MiB): FETCH_SIZE
# reports half the bytes read, WRITE_SIZE reports the bytes written.
FETCH_FACTOR = 2.0
WRITE_FACTOR = 1.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--configs", default="1,2,3,4,5,ffn,attn,5/k1s1,5/k3s2")
    ap.add_argument("--cpu-seconds", type=float, default=20.0, help="budget of the CPU-baseline leg (all configs)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--repeats", type=int, default=3)
    ap.add_argument("--traffic-probe", type=int, default=0, metavar="REPS",
                    help="counter-collection mode: a calibration kernel of known traffic, then REPS "
                         "untimed launches of each workload; prints nothing else")
    return ap.parse_args()


def f16(a):
    return np.asarray(a, np.float32).astype(np.float16)


class Case:
    """One configuration: device buffers, one step's launches, its work."""

    def __init__(self, name, unit, work, bound, peak, launch_fn, kernel, flops, bytes_, dtype, tkey):
        self.name, self.unit, self.work, self.bound, self.peak = name, unit, work, bound, peak
        self.launch = launch_fn      # launch(step_index) -> None, on the bench stream
        self.kernel, self.flops, self.bytes, self.dtype = kernel, flops, bytes_, dtype
        self.tkey = tkey             # row of the traffic table for this workload


def load_traffic():
    """L2-miss bytes per launch (HBM plus Infinity Cache hits) from the committed
    rocprofv3 counter table:
    workload key -> FETCH_FACTOR * FETCH_SIZE + WRITE_FACTOR * WRITE_SIZE, summed
    over the rows of one key (a split-K GEMM and its reduce are one step)."""
    out = {}
    if not os.path.exists(TRAFFIC_FILE):
        return out
    for ln in open(TRAFFIC_FILE):
        if ln.startswith("#") or not ln.strip():
            continue
        key, _kernel, fetch_kib, write_kib = ln.rstrip("\n").split("\t")
        out[key] = out.get(key, 0) + round((FETCH_FACTOR * float(fetch_kib) + WRITE_FACTOR * float(write_kib)) * 1024)
    return out


def build_cases(capi, stream, which):
    import ctypes
    lib = capi.lib()
    D = capi.DeviceArray.from_numpy
    rng = np.random.default_rng(0)
    cases = {}

    def linear_case(x, ws, bias=None, epi="NONE", gated=False, odt=np.float32, pack=False):
        N = ws[0].shape[0] // 2 if gated else ws[0].shape[0]
        out = capi.DeviceArray(x.shape[:-1] + (N,), odt)
        args = [capi.linear_args(out, x, w, bias, epi=epi, gated=gated, gate_epi="SILU") for w in ws]
        keep = [out, x, ws, bias]
        if pack:
            # prefill weights are packed once, as the engine's Linear does at prepare
            for a in args:
                packed = capi.linear_pack_weight(a, stream.ptr)
                if packed is not None:
                    a.packed_weight = packed.ptr
                    keep.append(packed)
            stream.synchronize()
        need = capi.linear_workspace_size(args[0])
        if need:
            wsp = capi.DeviceArray((need,), np.uint8)
            keep.append(wsp)
            for a in args:
                a.workspace, a.workspace_bytes = wsp.ptr, wsp.nbytes
        refs = [ctypes.byref(a) for a in args]

        def launch(i):
            capi.check(lib.vai_linear_launch(refs[i % len(refs)], stream.ptr), "linear")
        launch.keep = keep + args
        return launch, capi.linear_plan(args[0])[0]

    if "1" in which:   # GPT-2 small c_fc, fp32
        w = (rng.standard_normal((768, 3072)).astype(np.float32) * np.float32(0.02)).T.copy()
        b = rng.standard_normal(3072).astype(np.float32) * np.float32(0.02)
        x = rng.standard_normal((128, 768)).astype(np.float32)
        fn, kern = linear_case(D(x), [D(w)], D(b), epi="GELU_TANH")
        flops = 2 * 128 * 768 * 3072
        cases["1"] = Case("GPT-2 c_fc Linear fp32 X[128,768] W[3072,768] +bias GELU-tanh", "TFLOP/s",
                          flops / 1e12, "mfma", FP32_PEAK_TFLOPS, fn, kern, flops, 11415552, "f32", "1")

    if "2" in which:   # decode GEMV, M in {1,4,8}; rotate W copies past the MALL
        w0 = f16(rng.standard_normal((2048, 8192)) * 0.02).T.copy()
        copies = max(2, ROTATE_BYTES // w0.nbytes)
        ws = [D(w0) for _ in range(copies)]
        for m in (1, 4, 8):
            x = D(f16(np.random.default_rng(m).standard_normal((m, 2048))))
            # each W copy packed once, as the engine's Linear does at prepare (M >= 3 reads it)
            fn, kern = linear_case(x, ws, pack=True)
            byts = 2048 * 8192 * 2 + m * 2048 * 2 + m * 8192 * 4
            cases[f"2/M={m}"] = Case(f"decode GEMV M={m} K=2048 N=8192 fp16 W, fp32 acc/out", "GB/s",
                                     byts / 1e9, "hbm", HBM_PEAK_GBS, fn, kern, 2 * m * 2048 * 8192, byts, "f16", f"2/M={m}")

    if "3" in which:   # prefill gate/up, fused SiLU(g)*u
        wg = f16(rng.standard_normal((3072, 8192)) * 0.02).T
        wu = f16(rng.standard_normal((3072, 8192)) * 0.02).T
        w = np.ascontiguousarray(np.concatenate([wg, wu], 0))
        x = D(f16(rng.standard_normal((2048, 3072))))
        fn, kern = linear_case(x, [D(w)], gated=True, pack=True)
        flops = 2 * 2048 * 3072 * 16384
        cases["3"] = Case("prefill gate/up X[2048,3072] W[2x8192,3072] fp16, SiLU(g)*u fused, fp32 out",
                          "TFLOP/s", flops / 1e12, "mfma", FP16_PEAK_TFLOPS, fn, kern, flops, 180355072, "f16", "3")

    if "ffn" in which:   # the whole gated MLP block at config 3's shape (Llama-3.2-3B FFN), fp16 between nodes
        wg = f16(rng.standard_normal((3072, 8192)) * 0.02).T
        wu = f16(rng.standard_normal((3072, 8192)) * 0.02).T
        w1 = D(np.ascontiguousarray(np.concatenate([wg, wu], 0)))
        w2 = D(f16(rng.standard_normal((8192, 3072)) * 0.02).T.copy())
        x = D(f16(rng.standard_normal((2048, 3072))))
        res = D(f16(rng.standard_normal((2048, 3072))))
        hid = capi.DeviceArray((2048, 8192), np.float16)
        y = capi.DeviceArray((2048, 3072), np.float16)
        a1 = capi.linear_args(hid, x, w1, gated=True, gate_epi="SILU")
        a2 = capi.linear_args(y, hid, w2, None, res)
        keep = [w1, w2, x, res, hid, y, a1, a2]
        for a in (a1, a2):
            packed = capi.linear_pack_weight(a, stream.ptr)
            if packed is not None:
                a.packed_weight = packed.ptr
                keep.append(packed)
            need = capi.linear_workspace_size(a)
            if need:
                wsp = capi.DeviceArray((need,), np.uint8)
                keep.append(wsp)
                a.workspace, a.workspace_bytes = wsp.ptr, wsp.nbytes
        stream.synchronize()
        r1, r2 = ctypes.byref(a1), ctypes.byref(a2)

        def fnf(i):
            capi.check(lib.vai_linear_launch(r1, stream.ptr), "ffn gate/value")
            capi.check(lib.vai_linear_launch(r2, stream.ptr), "ffn out")
        fnf.keep = keep
        flops = 2 * 2048 * 3072 * 16384 + 2 * 2048 * 8192 * 3072
        kern = capi.linear_plan(a1)[0] + " + " + capi.linear_plan(a2)[0]
        cases["ffn"] = Case("gated MLP block X[2048,3072] -> SiLU(g)*u [2048,8192] -> out [2048,3072] + residual, fp16",
                            "TFLOP/s", flops / 1e12, "mfma", FP16_PEAK_TFLOPS, fnf, kern, flops,
                            2048 * 3072 * 2 + 16384 * 3072 * 2 + 2048 * 8192 * 2 * 2 + 3072 * 8192 * 2 + 2048 * 3072 * 2 * 2,
                            "f16", "ffn")

    if "4" in which:   # attention scores; rotate Q, K and S together past the MALL
        n4 = ROTATE_BYTES // (8 << 22) + 1
        q0 = f16(rng.standard_normal((8, 1024, 256)))
        k0 = f16(rng.standard_normal((8, 1024, 256)))
        qs = [D(q0) for _ in range(n4)]
        ks = [D(k0) for _ in range(n4)]
        outs = [capi.DeviceArray((8, 1024, 1024), np.float32) for _ in range(n4)]
        args = [capi.attn_scores_args(o, q, k, scale=1.0 / 16, causal=True) for o, q, k in zip(outs, qs, ks)]
        refs = [ctypes.byref(a) for a in args]

        def fn4(i):
            capi.check(lib.vai_attn_scores_launch(refs[i % len(refs)], stream.ptr), "scores")
        fn4.keep = [qs, ks, outs, args]
        cases["4"] = Case("attention scores Q,K[8,1024,256] fp16, S=QK^T/16 fp32 causal", "GB/s",
                          41943040 / 1e9, "hbm", HBM_PEAK_GBS, fn4, "scores_strip_kernel<256> (64-row strips x 4 column classes, Q in registers, K tiles by DMA, hidden tiles stored as -inf, register epilogue)", 2 * 8 * 1024 * 1024 * 256,
                          41943040, "f16", "4")

    if "attn" in which:   # the whole attention at config 4's shape: scores, softmax and P.V fused
        q = D(f16(rng.standard_normal((8, 1024, 256))))
        k = D(f16(rng.standard_normal((8, 1024, 256))))
        v = D(f16(rng.standard_normal((8, 1024, 256))))
        o = capi.DeviceArray((8, 1024, 256), np.float16)
        aa = capi.attention_args(o, q, k, v, scale=1.0 / 16, causal=True)
        need = lib.vai_attention_workspace_size(ctypes.byref(aa))
        wsa = capi.DeviceArray((max(need, 1),), np.uint8)
        if need:
            aa.workspace, aa.workspace_bytes = wsa.ptr, wsa.nbytes
        ra = ctypes.byref(aa)

        def fna(i):
            capi.check(lib.vai_attention_launch(ra, stream.ptr), "attention")
        fna.keep = [q, k, v, o, aa, wsa]
        flops = 4 * 8 * 256 * (1024 * 1025 // 2)   # QK^T and P.V over the visible (causal) pairs
        cases["attn"] = Case("attention Q,K,V[8,1024,256] fp16 causal, O = softmax(QK^T/16) V fp16 (fused)", "TFLOP/s",
                             flops / 1e12, "mfma", FP16_PEAK_TFLOPS, fna, "attention_fwd_kernel<256> + attention_merge_kernel<256> (key range split over workgroups, merged by a second pass)", flops,
                             4 * 8 * 1024 * 256 * 2, "f16", "attn")

    if "5" in which:   # YOLOX 3x3 conv, bias + SiLU
        wt = D(f16(rng.standard_normal((128, 128, 3, 3)) * 0.03))
        bias = D(f16(rng.standard_normal(128) * 0.02))
        x = D(f16(rng.uniform(-1, 1, (1, 128, 80, 80))))
        out = capi.DeviceArray((1, 128, 80, 80), np.float32)
        a5 = capi.conv2d_args(out, x, wt, bias, epi="SILU")
        # the weight is packed once, as the reference's Convolution transforms it once at prepare
        ws5 = capi.conv2d_pack_weight(a5, stream.ptr)
        stream.synchronize()
        a5.packed_weight = ws5.ptr if ws5 is not None else None
        r5 = ctypes.byref(a5)

        def fn5(i):
            capi.check(lib.vai_conv2d_launch(r5, stream.ptr), "conv")
        fn5.keep = [wt, bias, x, out, a5, ws5]
        flops = 2 * 6400 * 128 * 1152
        cases["5"] = Case("YOLOX-s 3x3 conv in[1,128,80,80] W[128,128,3,3] fp16 +bias SiLU, fp32 out",
                          "TFLOP/s", flops / 1e12, "mfma", FP16_PEAK_TFLOPS, fn5, "conv3_pipe_kernel<5,4,4> (implicit GEMM, NCHW rows transposed by the LDS read, packed weight; 4 waves x 16 output channels x one row over all 4 channel blocks, block-pipelined copies, SiLU epilogue stored per fragment during the last block)", flops, 5210368, "f16", "5")
    for key, (ci, co, ks, st, hw) in {"5/k1s1": (256, 128, 1, 1, 40), "5/k3s2": (128, 256, 3, 2, 80)}.items():
        if key not in which:
            continue
        # the other YOLOX-s conv plans: a CSP pointwise conv and the 3x3 stride-2 downsample
        wt = D(f16(rng.standard_normal((co, ci, ks, ks)) * 0.03))
        bias = D(f16(rng.standard_normal(co) * 0.02))
        x = D(f16(rng.uniform(-1, 1, (1, ci, hw, hw))))
        ho = (hw - 1) // st + 1
        out = capi.DeviceArray((1, co, ho, ho), np.float32)
        ac = capi.conv2d_args(out, x, wt, bias, stride=st, epi="SILU")
        wsc = capi.conv2d_pack_weight(ac, stream.ptr)
        stream.synchronize()
        ac.packed_weight = wsc.ptr if wsc is not None else None
        rc = ctypes.byref(ac)

        def fnc(i, rc=rc):
            capi.check(lib.vai_conv2d_launch(rc, stream.ptr), "conv")
        fnc.keep = [wt, bias, x, out, ac, wsc]
        flops = 2 * ho * ho * co * ci * ks * ks
        byts = ci * hw * hw * 2 + co * ci * ks * ks * 2 + co * 2 + co * ho * ho * 4
        cases[key] = Case(f"YOLOX-s {ks}x{ks}/s{st} conv in[1,{ci},{hw},{hw}] W[{co},{ci},{ks},{ks}] fp16 +bias SiLU, fp32 out",
                          "TFLOP/s", flops / 1e12, "mfma", FP16_PEAK_TFLOPS, fnc,
                          "conv1_pipe_kernel<8,4> (pointwise: 16 flat positions x 64 output channels per workgroup, branch-free SiLU epilogue, one 16-byte store per lane)" if ks == 1
                          else f"conv_kernel<{ks}> (implicit GEMM, packed weight)",
                          flops, byts, "f16", key)
    if "read" in which or "empty" in which or "write" in which:
        # the ceiling for config 2: a plain read of W's 32 MiB, rotated like the
        # GEMV's W copies (vai_amd/probe/read_ceiling.hip), and an empty launch
        probe = ctypes.CDLL(os.path.join(ROOT, "vai_amd", "libvai_probe.so"))
        probe.vai_probe_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_void_p, ctypes.c_void_p]
        probe.vai_probe_empty.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
        sink = capi.DeviceArray((1,), np.float32)
        nbytes = 2048 * 8192 * 2
        bufs = [capi.DeviceArray((nbytes,), np.uint8) for _ in range(max(2, ROTATE_BYTES // nbytes))]
        for b in bufs:
            b.fill_(0)
        variants = [(v, g, t, l) for v, (g, t, l) in READ_VARIANTS.items()] if "read" in which else []
        for name, g, t, l in variants:
            def fnr(i, g=g, t=t, l=l):
                capi.check(probe.vai_probe_read(bufs[i % len(bufs)].ptr, nbytes, g, t, l, sink.ptr, stream.ptr), "read")
            fnr.keep = [bufs, sink, probe]
            cases[f"read/{name}"] = Case(f"plain read of 32 MiB ({g} workgroups x {t} threads, {l} x 16 B loads per lane "
                                         f"in flight), rotating {len(bufs)} buffers", "GB/s", nbytes / 1e9, "hbm",
                                         HBM_PEAK_GBS, fnr, "read_kernel (vai_amd/probe)", 0, nbytes, "f16", "read")
        if "write" in which:
            # the ceiling for config 4: writing S's 32 MiB, rotated the same way
            probe.vai_probe_write.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                              ctypes.c_void_p]
            for name, (g, t, l) in WRITE_VARIANTS.items():
                def fnw(i, g=g, t=t, l=l):
                    capi.check(probe.vai_probe_write(bufs[i % len(bufs)].ptr, nbytes, g, t, l, stream.ptr), "write")
                fnw.keep = [bufs, probe]
                cases[f"write/{name}"] = Case(f"plain write of 32 MiB ({g} workgroups x {t} threads, {l} x 16 B "
                                              f"non-temporal stores per lane), rotating {len(bufs)} buffers", "GB/s",
                                              nbytes / 1e9, "hbm", HBM_PEAK_GBS, fnw, "write_kernel (vai_amd/probe)", 0,
                                              nbytes, "f32", "write")
        if "empty" in which:
            for g in (1, 256, 1024):
                def fne(i, g=g):
                    capi.check(probe.vai_probe_empty(g, 256, sink.ptr, stream.ptr), "empty")
                fne.keep = [sink, probe]
                cases[f"empty/{g}"] = Case(f"empty kernel, {g} workgroups of 256", "us", 0.0, "hbm", HBM_PEAK_GBS, fne,
                                           "empty_kernel (vai_amd/probe)", 0, 0, "-", "empty")
    return cases


# plain-write variants: name -> (workgroups, threads per workgroup, stores per lane)
WRITE_VARIANTS = {
    "2048x256x4": (2048, 256, 4),
    "1024x256x8": (1024, 256, 8),
    "512x256x16": (512, 256, 16),
    "256x1024x8": (256, 1024, 8),
}


# plain-read variants: name -> (workgroups, threads per workgroup, loads per lane)
READ_VARIANTS = {
    "gemv_shape": (1024, 256, 8),      # the M=1 GEMV's grid: 4096 waves of 8 KB
    "wg512": (512, 512, 8),
    "wg1024x256thr": (256, 1024, 8),
    "16loads": (512, 256, 16),
    "32loads": (256, 256, 32),
    "4loads": (2048, 256, 4),
}


def time_case(capi, stream, case, steps, warmup, repeats):
    for i in range(warmup):
        case.launch(i)
    stream.synchronize()
    graph = capi.Graph(stream, lambda: [case.launch(i) for i in range(steps)])
    graph.launch()
    stream.synchronize()
    t0, t1 = capi.Event(), capi.Event()
    per_step = []
    for _ in range(repeats):
        t0.record(stream.ptr)
        graph.launch()
        t1.record(stream.ptr)
        t1.synchronize()
        per_step.append(t0.elapsed_ms(t1) / steps)
    return float(np.median(per_step))


def cpu_samples(keys):
    """The CPU baseline's bounded sample of each configuration: key ->
    (call(i), work per call in the GPU line's unit, unit, description). The
    calls run the OpenMP restatement in oracle/cpu_baseline.c on the same
    shapes and dtypes (fp16 operands stay fp16 in memory and are widened by
    F16C); GEMV bytes are the bytes each call really reads and writes."""
    from oracle import oracle
    rng = np.random.default_rng(0)
    out = {}
    for key in keys:
        if key == "1":
            w = (rng.standard_normal((3072, 768)) * 0.02).astype(np.float32)
            b = (rng.standard_normal(3072) * 0.02).astype(np.float32)
            x = rng.standard_normal((128, 768)).astype(np.float32)
            o = np.empty((128, 3072), np.float32)
            out[key] = (lambda i, x=x, w=w, b=b, o=o: oracle.cpu_linear(x, w, b, epi="GELU_TANH", out=o),
                        2 * 128 * 768 * 3072 / 1e12, "TFLOP/s", "full config 1 (fp32 blocked GEMM + bias + GELU-tanh)")
        elif key.startswith("2/M="):
            m = int(key[4:])
            w0 = f16(rng.standard_normal((8192, 2048)) * 0.02)
            ws = [w0.copy() for _ in range(max(2, ROTATE_BYTES // w0.nbytes))]
            x = f16(rng.standard_normal((m, 2048)))
            o = np.empty((m, 8192), np.float32)
            byts = 2048 * 8192 * 2 + m * 2048 * 2 + m * 8192 * 4
            out[key] = (lambda i, x=x, ws=ws, o=o: oracle.cpu_linear(x, ws[i % len(ws)], out=o), byts / 1e9, "GB/s",
                        f"full config 2 M={m} (fp16 W read as fp16 via F16C), rotating {len(ws)} W copies "
                        f"({len(ws) * w0.nbytes >> 20} MiB) past the host caches")
        elif key in ("3", "ffn"):
            rows = 128
            wg = f16(rng.standard_normal((8192, 3072)) * 0.02)
            wu = f16(rng.standard_normal((8192, 3072)) * 0.02)
            w = np.ascontiguousarray(np.concatenate([wg, wu], 0))
            x = f16(rng.standard_normal((rows, 3072)))
            o = np.empty((rows, 8192), np.float32)
            if key == "3":
                out[key] = (lambda i, x=x, w=w, o=o: oracle.cpu_linear(x, w, gated=True, gate_epi="SILU", out=o),
                            2 * rows * 3072 * 16384 / 1e12, "TFLOP/s",
                            f"config 3 on {rows} of the 2048 rows of X against the full gate/up weight")
            else:
                w2 = f16(rng.standard_normal((3072, 8192)) * 0.02)
                o2 = np.empty((rows, 3072), np.float32)

                def ffn(i, x=x, w=w, w2=w2, o=o, o2=o2):
                    oracle.cpu_linear(x, w, gated=True, gate_epi="SILU", out=o)
                    oracle.cpu_linear(o, w2, out=o2)
                out[key] = (ffn, (2 * rows * 3072 * 16384 + 2 * rows * 8192 * 3072) / 1e12, "TFLOP/s",
                            f"the FFN block on {rows} of the 2048 rows (fp32 activations between the two GEMMs)")
        elif key in ("4", "attn"):
            q = f16(rng.standard_normal((8, 1024, 256)))
            k = f16(rng.standard_normal((8, 1024, 256)))
            if key == "4":
                s = np.empty((8, 1024, 1024), np.float32)
                out[key] = (lambda i, q=q, k=k, s=s: oracle.cpu_attn_scores(q, k, scale=1 / 16, causal=True, out=s),
                            41943040 / 1e9, "GB/s", "full config 4 (bytes counted as the GPU line's: Q, K, S)")
            else:
                v = f16(rng.standard_normal((8, 1024, 256)))
                o = np.empty((8, 1024, 256), np.float32)
                out[key] = (lambda i, q=q, k=k, v=v, o=o: oracle.cpu_attention(q, k, v, scale=1 / 16, causal=True, out=o),
                            4 * 8 * 256 * (1024 * 1025 // 2) / 1e12, "TFLOP/s",
                            "full config-4 attention (blocked scores, fp32 softmax, P.V; causal pairs only)")
        elif key.startswith("5"):
            ci, co, ks, st, hw = {"5": (128, 128, 3, 1, 80), "5/k1s1": (256, 128, 1, 1, 40),
                                  "5/k3s2": (128, 256, 3, 2, 80)}[key]
            w = f16(rng.standard_normal((co, ci, ks, ks)) * 0.03)
            b = f16(rng.standard_normal(co) * 0.02).astype(np.float32)
            x = f16(rng.uniform(-1, 1, (ci, hw, hw)))
            ho = (hw - 1) // st + 1
            o = np.empty((co, ho, ho), np.float32)
            out[key] = (lambda i, x=x, w=w, b=b, st=st, o=o: oracle.cpu_conv2d(x, w, b, stride=st, epi="SILU", out=o),
                        2 * ho * ho * co * ci * ks * ks / 1e12, "TFLOP/s",
                        f"full {ks}x{ks}/s{st} conv (implicit GEMM per output row, K order c*k*k + kh*k + kw)")
    return out


def cpu_baseline(keys, budget_s):
    """Each sample above run repeatedly for its share of budget_s (at least
    one call) on the host cores, after one untimed call."""
    from oracle import oracle
    samples = cpu_samples(keys)
    share = budget_s / max(1, len(samples))
    res = {}
    for key, (call, work, unit, desc) in samples.items():
        call(0)
        n, t0 = 0, time.perf_counter()
        while n == 0 or time.perf_counter() - t0 < share:
            call(n + 1)
            n += 1
        dt = (time.perf_counter() - t0) / n
        res[key] = {"value": round(work / dt, 4 if unit == "TFLOP/s" else 3), "unit": unit,
                    "cores": oracle.num_threads(), "kind": "port",
                    "sample": f"oracle/cpu_baseline.c, {desc}; {n} calls in {dt * n:.1f} s"}
        print(f"# cpu {key}: {res[key]['value']} {unit} ({n} calls)", file=sys.stderr, flush=True)
    return res


def traffic_probe(capi, stream, cases, reps):
    """Launches for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs: first the
    calibration kernel (GatedMul over [4096, 4096] fp32 -> [4096, 2048]: reads
    64 MiB, writes 32 MiB), then `reps` launches of every workload."""
    gin = capi.DeviceArray((4096, 4096), np.float32)
    gin.fill_(0)
    gout = capi.DeviceArray((4096, 2048), np.float32)
    for _ in range(5):
        capi.gated_mul(gout, gin, "NONE", stream=stream.ptr)
    stream.synchronize()
    for key, case in cases.items():
        for i in range(reps):
            case.launch(i)
        stream.synchronize()
        print(f"# traffic probe: {key} x{reps}", file=sys.stderr, flush=True)


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                                   "(multi-GPU sharding of this path is design-only)"}))
        sys.exit(2)
    from vai_amd import _capi as capi
    capi.check(capi.lib().vai_set_device(0), "set_device")
    stream = capi.Stream()
    cases = build_cases(capi, stream, set(args.configs.split(",")))
    if args.traffic_probe:
        traffic_probe(capi, stream, cases, args.traffic_probe)
        return
    traffic = load_traffic()
    report = {}
    for key, case in cases.items():
        ms = time_case(capi, stream, case, args.steps, args.warmup, args.repeats)
        if case.unit == "us":   # empty-launch probe: the per-step time is the figure
            report[key] = {"workload": case.name, "kernel": case.kernel, "value": round(ms * 1e3, 3), "unit": "us",
                           "ms_per_step": round(ms, 6), "dtype": case.dtype}
            print(f"# {key}: {case.name}: {ms*1e3:.2f} us/step", file=sys.stderr, flush=True)
            continue
        rate = case.work / (ms * 1e-3)
        achieved = (case.bytes / 1e9 if case.bound == "hbm" else case.flops / 1e12) / (ms * 1e-3)
        report[key] = {
            "workload": case.name, "kernel": case.kernel, "value": round(rate, 3), "unit": case.unit,
            "ms_per_step": round(ms, 6), "dtype": case.dtype,
            "roofline": {"bound": case.bound, "achieved": round(achieved, 3), "peak": case.peak,
                         "unit": "GB/s" if case.bound == "hbm" else "TFLOP/s",
                         "frac": round(achieved / case.peak, 4), "traffic": traffic.get(case.tkey)},
        }
        print(f"# cfg {key}: {case.name}: {ms*1e3:.2f} us/step, {rate:.1f} {case.unit}, "
              f"{100*achieved/case.peak:.1f}% of {case.bound} peak [{case.kernel}]", file=sys.stderr, flush=True)
    if not args.no_cpu:
        for key, cb in cpu_baseline([k for k in report if not k.startswith(("read", "empty", "write"))],
                                    args.cpu_seconds).items():
            report[key]["cpu_baseline"] = cb
    prim = report.get("2/M=1") or next(iter(report.values()))
    line = {
        "metric": METRIC, "value": prim["value"], "unit": prim["unit"], "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": prim["ms_per_step"], "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": prim["dtype"], "data": "synthetic",
        "config": {"workload": prim["workload"], "kernel": prim["kernel"]},
        "roofline": prim["roofline"],
        "cpu_baseline": prim.get("cpu_baseline"),
        "configs": report,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
