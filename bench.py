"""Benchmark: quantized-matmul hot path on one MI355X.

Headline (BASELINE.json metric "qmv HBM GB/s (% of peak) at M=1"): one step =
the Llama-3-8B MLP decode projections at M=1, 4-bit affine, group 64:
gate (N=14336, K=4096), up (same) and down (N=4096, K=14336), three qmv
launches of 33,067,008 algorithmic bytes each (packed W + bf16 scales +
bf16 biases + x + y).  Weights rotate across 8 distinct layers (~793 MB) so
every launch streams from HBM, not the 256 MB MALL.  The steps of the 8
layers are one HIP graph (as a decode step's graph holds every layer), so the
timed region holds GPU work only; `value` = algorithmic bytes / time over
exactly K timed steps (HIP events on the replay stream).
`roofline` is the gate kernel alone: bytes per launch / its average launch
duration, timed the same way; `roofline.read_ceiling` is the fastest plain
streaming read of the same bytes per launch on this device, timed the same
way (the practical bound at this size).

Also reported (extra): the M in {1,2,4,8,16} x {4,8}-bit decode sweep, the
qmm prefill configs, mxfp4 gather_qmm (gpt-oss-20b MoE shapes), the fused
decode MoE (Qwen3-30B-A3B experts) against its gather_qmm chain, end-to-end
decode of a Qwen3-8B-shaped model, the general kernel (float16/float32,
3-bit, transpose=false), the measured device copy ceiling, and the
single-core CPU baseline (the oracle's restatement of MLX's CPU `_qmm_t`,
overlays/cpu/mlx/backend/cpu/quantized.cpp:199-257).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-extra] [--no-cpu]
                       [--extras copy,c1,sweep,qmm,gather,moe,e2e,general]
       python bench.py --traffic-probe   (under rocprofv3 --pmc: copy calibration + gate and gather launches)
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import mlxcel_amd as mq  # noqa: E402

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0  # dense
MALL_BYTES = 256 << 20
SETTLE_MS = 60.0  # untimed replays before each prefill measurement (see timed)
GATE_REPLAYS = 12  # replays of the 8-launch gate graph behind `roofline` (>= 96 launches)
# HBM bytes per gate launch from rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE on
# `bench.py --traffic-probe`, each counter scaled by what it reads for a
# device copy of exactly 256 MiB (FETCH_SIZE x 1.999800, WRITE_SIZE x 1.0):
# 16207.6 KiB fetched + 56 KiB written per launch of qmv_rs_dense_kernel
# (profiles/qmv_rs_gate_m1_traffic.txt, build 827e1df), 1.0054 x the
# algorithmic bytes.  Re-measure when qmv_rs.hip or common.hpp changes.
TRAFFIC_GATE = 33_247_110


def qmv_bytes(M, N, K, bits, gs):
    return N * K * bits // 8 + N * (K // gs) * 4 + M * K * 2 + M * N * 2


def make_affine(N, K, bits, gs, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = (torch.randn(N, K, device="cuda", generator=g, dtype=torch.float32) * 0.02).to(torch.bfloat16)
    return mq.quantize(w, gs, bits)


def make_mxfp4(E, N, K, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = (torch.randn(E, N, K, device="cuda", generator=g, dtype=torch.float32) * 0.02).to(torch.bfloat16)
    return mq.quantize(w, 32, 4, "mxfp4")


def randn_bf16(shape, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randn(*shape, device="cuda", generator=g, dtype=torch.float32).to(torch.bfloat16)


def timed(fn, iters, warmup, settle_ms=0.0):
    """ms per call of fn(i), HIP events on the current stream around `iters`
    calls, after `warmup` calls and then more untimed calls until `settle_ms`
    of wall time has passed.  (A freshly captured prefill graph replays ~5-15%
    slower for its first few milliseconds on MI355X; the extra sections settle,
    the headline keeps exactly its W warm-up steps.)"""
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    t_end = time.perf_counter() + settle_ms * 1e-3
    i = warmup
    while time.perf_counter() < t_end:
        fn(i)
        i += 1
        torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for i in range(iters):
        fn(i)
    t1.record(stream)
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / iters


def capture(fn):
    """HIP graph of fn() (launches only).  The library keeps scratch per
    (device, stream), so the warm-up runs on the stream that is captured."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        fn()
    torch.cuda.synchronize()
    return g


def timed_graphs(graphs, iters, warmup, settle_ms=0.0):
    """ms per replay, replaying graphs[i % len(graphs)] for i < iters."""
    return timed(lambda i: graphs[i % len(graphs)].replay(), iters, warmup, settle_ms)


# ---- headline: MLP decode step ----------------------------------------------

def headline(steps, warmup, layers=8):
    """One step = gate, up and down of one layer; steps rotate over `layers`
    layers so every launch streams its weights from HBM.  The timed region
    replays HIP graphs only (GPU work only).  Returns (GB/s, ms per step, avg
    us per launch, bytes per launch, gate us per launch, one gate matrix)."""
    K1, N1 = 4096, 14336
    mlp = []
    for l in range(layers):
        gate = make_affine(N1, K1, 4, 64, 1000 + 3 * l)
        up = make_affine(N1, K1, 4, 64, 1001 + 3 * l)
        down = make_affine(K1, N1, 4, 64, 1002 + 3 * l)
        mlp.append((gate, up, down))
    x = randn_bf16((1, K1), 7)
    h = randn_bf16((1, N1), 8)
    out_g = torch.empty(1, N1, dtype=torch.bfloat16, device="cuda")
    out_u = torch.empty_like(out_g)
    out_d = torch.empty(1, K1, dtype=torch.bfloat16, device="cuda")

    def step_fn(l):
        gate, up, down = mlp[l]

        def f():
            mq.quantized_matmul(x, *gate, True, 64, 4, out=out_g)
            mq.quantized_matmul(x, *up, True, 64, 4, out=out_u)
            mq.quantized_matmul(h, *down, True, 64, 4, out=out_d)
        return f

    # one graph runs the steps of all `layers` layers back to back, as a decode
    # step's graph runs every layer; a second graph holds the first
    # steps % layers of them, so exactly `steps` steps are timed
    def run(n):
        def f():
            for l in range(n):
                step_fn(l)()
        return f

    full = capture(run(layers))
    rem = steps % layers
    part = capture(run(rem)) if rem else None
    for _ in range(max(1, warmup // layers)):
        full.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for _ in range(steps // layers):
        full.replay()
    if part is not None:
        part.replay()
    t1.record(stream)
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps
    per_launch = qmv_bytes(1, N1, K1, 4, 64)
    assert per_launch == qmv_bytes(1, K1, N1, 4, 64) == 33_067_008
    value = 3 * per_launch / (ms * 1e-3) / 1e9
    # the dominant kernel alone: the gate projection (row-streaming qmv), one
    # graph of `layers` back-to-back launches over distinct weights, timed on
    # the replay stream (rocprofv3's kernel trace of the same command gives the
    # kernel bodies alone; the two agree within ~2%)
    gate_graph = capture(lambda: [mq.quantized_matmul(x, *mlp[l][0], True, 64, 4, out=out_g) for l in range(layers)])
    # a fixed >= 96 launches (>= 12 replays of the 8-launch graph) whatever
    # --steps is, after ~60 ms of untimed replays, so the figure does not
    # depend on the driver's step count
    reps = max(GATE_REPLAYS, steps // layers)
    gate_us = timed_graphs([gate_graph], reps, max(2, warmup // layers), SETTLE_MS) * 1e3 / layers
    # the same steps with gate and up as one quantized_matmul_multi launch
    # (two launches per step instead of three; same bytes)
    def multi_step(l):
        gate, up, down = mlp[l]
        mq.quantized_matmul_multi(x, [gate[0], up[0]], [gate[1], up[1]], [gate[2], up[2]], 64, 4,
                                  out=[out_g, out_u])
        mq.quantized_matmul(h, *down, True, 64, 4, out=out_d)

    multi_graph = capture(lambda: [multi_step(l) for l in range(layers)])
    multi_ms = timed_graphs([multi_graph], reps, max(2, warmup // layers), SETTLE_MS) / layers
    multi_value = 3 * per_launch / (multi_ms * 1e-3) / 1e9
    return value, ms, ms * 1e3 / 3, per_launch, gate_us, mlp[0][0], multi_value, multi_ms


# ---- extras -------------------------------------------------------------------

def read_ceiling(nbytes=33_067_008, reps=40):
    """Fastest streaming read of `nbytes` per launch on this device: a plain
    16-byte-load kernel (mlxcel_amd/csrc/bench_read.hip) that folds what it
    reads with xor and writes nothing, timed like the gate kernel (one graph
    of back-to-back launches over distinct buffers that together overflow the
    MALL).  The best of a few launch shapes is the practical HBM bound for a
    decode projection of that size; it sits well below the 8 TB/s spec."""
    lib = ctypes.CDLL(os.path.join(ROOT, "mlxcel_amd", "libmlxq_bench.so"))
    lib.mlxq_bench_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_void_p]
    lib.mlxq_bench_read.restype = ctypes.c_int
    copies = max(2, math.ceil(2.4 * MALL_BYTES / nbytes))
    bufs = [torch.full((nbytes,), c + 1, dtype=torch.uint8, device="cuda") for c in range(copies)]
    sink = torch.zeros(1 << 16, dtype=torch.int32, device="cuda")
    best = None
    for wgs, thr in ((1024, 256), (2048, 256), (1024, 512), (4096, 512)):
        def launch_all(wgs=wgs, thr=thr):
            st = torch.cuda.current_stream().cuda_stream
            for b in bufs:
                rc = lib.mlxq_bench_read(b.data_ptr(), nbytes, sink.data_ptr(), wgs, thr, st)
                if rc != 0:
                    raise RuntimeError(f"mlxq_bench_read failed: {rc}")
        g = capture(launch_all)
        us = timed_graphs([g], reps, 3) * 1e3 / copies
        if best is None or us < best[0]:
            best = (us, wgs, thr)
        del g
    del bufs
    us, wgs, thr = best
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"bytes": nbytes, "us": round(us, 3), "GBps": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 3),
            "workgroups": wgs, "threads": thr}


def n_sweep(iters=240):
    """The M=1 gate-shape qmv (K=4096, 4-bit g64) over N, beside the plain
    streaming read of the same bytes (read_ceiling), both graph-timed on
    rotated copies: a least-squares line time = fixed + bytes / rate for
    each, so the fixed cost per launch and the streaming rate separate."""
    K = 4096
    rows = []
    for N in (2048, 4096, 7168, 14336, 28672, 57344):
        b = qmv_bytes(1, N, K, 4, 64)
        copies = max(2, math.ceil(2.4 * MALL_BYTES / qmv_bytes(0, N, K, 4, 64)))
        ws = [make_affine(N, K, 4, 64, 300 + c) for c in range(copies)]
        x = randn_bf16((1, K), 301)
        out = torch.empty(1, N, dtype=torch.bfloat16, device="cuda")
        g = capture(lambda: [mq.quantized_matmul(x, *w, True, 64, 4, out=out) for w in ws])
        us = timed_graphs([g], max(4, iters // copies), 2, SETTLE_MS) * 1e3 / copies
        del g, ws
        rd = read_ceiling(b)
        rows.append({"N": N, "bytes": b, "qmv_us": round(us, 3), "read_us": rd["us"]})
    fit = {}
    for key in ("qmv_us", "read_us"):
        xs = np.array([r["bytes"] for r in rows], np.float64)
        ys = np.array([r[key] for r in rows], np.float64)
        slope, icpt = np.polyfit(xs, ys, 1)
        fit[key] = {"fixed_us": round(float(icpt), 3), "rate_GBps": round(float(1e-3 / slope), 1)}
    return {"rows": rows, "fit": fit}


def route_audit(bits_list=(4, 8), rows_list=(1, 2, 3, 4, 5, 8, 12, 16)):
    """Decode routing audit: the default route beside every kernel the
    library can be forced to (MLXQ_QMV_KERNEL), at 7-8B projection shapes,
    the gpt-oss expert shape and a 151936-row LM head; 4/8-bit g64, graph
    timing over enough weight copies to stream from HBM.  A row whose best
    kernel beats the default by 5% or more is marked."""
    from mlxcel_amd import _lib
    shapes = [(4096, 4096), (1024, 4096), (12288, 4096), (4096, 12288), (14336, 4096), (4096, 14336),
              (2880, 2880), (151936, 4096)]
    kernels = ["", "rs", "b4", "mr", "kq", "mid", "mfma"]
    saved = os.environ.get("MLXQ_QMV_KERNEL")
    res = []
    for bits in bits_list:
        for N, K in shapes:
            L = max(2, min(64, int(2.4 * MALL_BYTES / (N * K * bits // 8)) + 1))
            ws = [make_affine(N, K, bits, 64, 500 + i) for i in range(L)]
            for M in rows_list:
                x = randn_bf16((M, K), 7)
                out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
                row = {"bits": bits, "N": N, "K": K, "M": M}
                for k in kernels:
                    os.environ.pop("MLXQ_QMV_KERNEL", None)
                    if k:
                        os.environ["MLXQ_QMV_KERNEL"] = k
                    _lib.load().mlxq_reload_options()
                    try:
                        g = capture(lambda: [mq.quantized_matmul(x, *w, True, 64, bits, out=out) for w in ws])
                    except (RuntimeError, ValueError):  # a forced kernel that does not take this shape
                        row[k or "default"] = None
                        continue
                    row[k or "default"] = round(timed_graphs([g], 6, 1, SETTLE_MS) * 1e3 / L, 2)
                    del g
                best = min((k for k in kernels[1:] if row[k] is not None), key=lambda k: row[k])
                row["best"] = best
                row["default_vs_best"] = round(row["default"] / row[best], 3)
                res.append(row)
                print(("!! " if row["default_vs_best"] > 1 / 0.95 else "   ") + json.dumps(row),
                      file=sys.stderr, flush=True)
            del ws
            torch.cuda.empty_cache()
    os.environ.pop("MLXQ_QMV_KERNEL", None)
    if saved is not None:
        os.environ["MLXQ_QMV_KERNEL"] = saved
    _lib.load().mlxq_reload_options()
    return res


def copy_ceiling():
    n = 1 << 30
    src = torch.empty(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    ms = timed(lambda i: dst.copy_(src), 20, 3)
    return 2 * n / (ms * 1e-3) / 1e9


def qmv_sweep(iters=200):
    """Decode sweep: M in {1,2,4,8} x {4,8}-bit at the
    Llama-3-8B MLP shapes, plus M=16 (the batch-16 decode of configs[4]); one
    graph launches every weight copy once."""
    res = []
    for bits in (4, 8):
        for (N, K, name) in ((14336, 4096, "gate_up"), (4096, 14336, "down")):
            wbytes = qmv_bytes(0, N, K, bits, 64)
            copies = max(2, math.ceil(2.4 * MALL_BYTES / wbytes))
            ws = [make_affine(N, K, bits, 64, 50 + c) for c in range(copies)]
            for M in (1, 2, 4, 8, 16):
                x = randn_bf16((M, K), 9)
                out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
                g = capture(lambda: [mq.quantized_matmul(x, *w, True, 64, bits, out=out) for w in ws])
                ms = timed_graphs([g], max(1, iters // copies), 2) / copies
                b = qmv_bytes(M, N, K, bits, 64)
                res.append({"bits": bits, "shape": name, "N": N, "K": K, "M": M, "us": round(ms * 1e3, 2),
                            "GBps": round(b / (ms * 1e-3) / 1e9, 1),
                            "frac_hbm": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 3)})
                del g
            del ws
    return res


def qmm_prefill(iters=20):
    """Prefill GEMM: M in {512, 2048}, 4/8-bit, the
    Llama-3-8B gate/up and down shapes; TFLOPS = 2 M N K / time.  Beside
    each, timed the same way in the same run:
    - `ref_route`: the reference's CDNA prefill route on this device, the
      quantized weights dequantized to bf16 (this library's bit-exact
      `dequantize`, the role of affine_dequantize_packed_kernel,
      rocm/quantized/qmm.hip:1376-1617) then torch's bf16 GEMM (hipBLASLt)
      x @ W^T, both in one graph per weight copy;
    - `dense_bf16`: the GEMM alone on already-dequantized [K, N] weights."""
    res = []
    for bits in (4, 8):
        for (N, K, name) in ((14336, 4096, "gate_up"), (4096, 14336, "down")):
            ws = [make_affine(N, K, bits, 64, 80 + c) for c in range(3)]
            # [K, N] contiguous bf16 copies of the dequantized weights
            wts = [mq.dequantize(*w, 64, bits).t().contiguous() for w in ws]
            wdq = torch.empty(N, K, dtype=torch.bfloat16, device="cuda")  # the route's dequantized matrix

            def ref_route(w, x, out):
                mq.dequantize(*w, 64, bits, out=wdq)
                torch.nn.functional.linear(x, wdq, out=out)

            for M in (512, 2048):
                x = randn_bf16((M, K), 13)
                out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
                g = capture(lambda: [mq.quantized_matmul(x, *w, True, 64, bits, out=out) for w in ws])
                ms = timed_graphs([g], max(1, iters // len(ws)), 1, SETTLE_MS) / len(ws)
                del g
                gr = capture(lambda: [ref_route(w, x, out) for w in ws])
                ms_r = timed_graphs([gr], max(1, iters // len(ws)), 1, SETTLE_MS) / len(ws)
                del gr
                gd = capture(lambda: [torch.mm(x, wt, out=out) for wt in wts])
                ms_d = timed_graphs([gd], max(1, iters // len(wts)), 1, SETTLE_MS) / len(wts)
                del gd
                fl = 2.0 * M * N * K
                tf, tf_r, tf_d = (fl / (t * 1e-3) / 1e12 for t in (ms, ms_r, ms_d))
                res.append({"bits": bits, "shape": name, "M": M, "N": N, "K": K, "us": round(ms * 1e3, 1),
                            "TFLOPS": round(tf, 1), "frac_mfma": round(tf / BF16_PEAK_TFLOPS, 3),
                            "ref_route": {"us": round(ms_r * 1e3, 1), "TFLOPS": round(tf_r, 1),
                                          "frac_mfma": round(tf_r / BF16_PEAK_TFLOPS, 3)},
                            "vs_ref_route": round(ms_r / ms, 3),
                            "dense_bf16": {"us": round(ms_d * 1e3, 1), "TFLOPS": round(tf_d, 1),
                                           "frac_mfma": round(tf_d / BF16_PEAK_TFLOPS, 3)},
                            "vs_dense": round(ms_d / ms, 3)})
            del ws, wts, wdq
    return res


def c1_qmv(iters=400, cpu_budget_s=5.0, with_cpu=True):
    """one 4-bit g64 qmv, N = K = 4096, M = 1 (the
    reference's CPU-runnable case), on the GPU (weights rotated over enough
    copies to overflow the MALL, one graph) and with the single-core oracle
    `_qmm_t` on the host (a bounded sample of calls)."""
    N = K = 4096
    b = qmv_bytes(1, N, K, 4, 64)
    assert b == 9_453_568
    copies = max(2, math.ceil(2.4 * MALL_BYTES / qmv_bytes(0, N, K, 4, 64)))
    ws = [make_affine(N, K, 4, 64, 150 + c) for c in range(copies)]
    x = randn_bf16((1, K), 151)
    out = torch.empty(1, N, dtype=torch.bfloat16, device="cuda")
    g = capture(lambda: [mq.quantized_matmul(x, *w, True, 64, 4, out=out) for w in ws])
    ms = timed_graphs([g], max(4, iters // copies), 2, SETTLE_MS) / copies
    del g
    res = {"workload": "C1: x [1,4096] bf16, w [4096,512] u32 (4-bit g64), transpose=true",
           "bytes": b, "us": round(ms * 1e3, 3), "GBps": round(b / (ms * 1e-3) / 1e9, 1),
           "frac_hbm": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 3)}
    if with_cpu:
        res["cpu"] = cpu_time(ws[0], x, N, K, cpu_budget_s)
    del ws
    return res


def general_path(iters=10):
    """The general kernel (qmm_gen.hip) and the float16 decode route at the
    gate shape (N=14336, K=4096, g64): float16 / float32 activations and
    scales, 3-bit codes, transpose=false; weights are random codes (the
    arithmetic does not depend on their values)."""
    N, K, gs = 14336, 4096, 64
    res = []
    cases = (("float16", 4, True), ("float32", 4, True), ("bfloat16", 3, True), ("bfloat16", 4, False))
    for dtn, bits, tr in cases:
        dt = getattr(torch, dtn)
        rows, cols = (N, K) if tr else (K, N)
        g = torch.Generator(device="cuda").manual_seed(90 + bits)
        for M in (1, 2048):
            # decode rotates enough weight copies to stream from HBM, not the MALL
            nl = max(2, int(2.4 * MALL_BYTES / (N * K * bits // 8)) + 1) if M == 1 else 2
            ws = []
            for _ in range(nl):
                wq = torch.randint(0, 2 ** 31 - 1, (rows, cols * bits // 32), device="cuda", generator=g,
                                   dtype=torch.int64).to(torch.int32).view(torch.uint32)
                s_ = (torch.rand(rows, cols // gs, device="cuda", generator=g) * 0.02).to(dt)
                b_ = (torch.rand(rows, cols // gs, device="cuda", generator=g) * 0.02 - 0.01).to(dt)
                ws.append((wq, s_, b_))
            x = torch.randn(M, K, device="cuda", generator=g).to(dt)
            out = torch.empty(M, N, dtype=dt, device="cuda")
            gr = capture(lambda: [mq.quantized_matmul(x, *w, tr, gs, bits, out=out) for w in ws])
            ms = timed_graphs([gr], max(2, iters), 1) / nl
            del gr
            res.append({"dtype": dtn, "bits": bits, "transpose": tr, "M": M, "us": round(ms * 1e3, 2),
                        "weight_GBps": round(N * K * bits / 8 / (ms * 1e-3) / 1e9, 1),
                        "TFLOPS": round(2.0 * M * N * K / (ms * 1e-3) / 1e12, 1)})
            del ws
    return res


def gather_moe(iters=100):
    """gpt-oss-20b-like MoE: 32 experts, gate/up fused [5760, 2880], down [2880, 2880], top-4."""
    E, H, I2 = 32, 2880, 5760
    copies = 2
    gu = [make_mxfp4(E, I2, H, 60 + c) for c in range(copies)]
    dn = [make_mxfp4(E, H, H, 70 + c) for c in range(copies)]
    per_expert = (I2 * H // 2 + I2 * H // 32) + (H * H // 2 + H * H // 32)
    res = []
    rng = np.random.default_rng(5)
    for T in (1, 16, 256):
        nsets = 16
        ids = [np.stack([rng.permutation(E)[:4] for _ in range(T)]).astype(np.int32) for _ in range(nsets)]
        sorted_mode = T * 4 >= 64  # src/models/gpt_oss.rs:322
        x = randn_bf16((T, 1, 1, H), 11)
        if sorted_mode:
            orders = [np.argsort(i.reshape(-1), kind="stable") for i in ids]
            rhs = [torch.from_numpy(i.reshape(-1)[o].astype(np.int32)).cuda() for i, o in zip(ids, orders)]
            xs = [x.reshape(T, 1, H)[torch.from_numpy(o // 4).cuda()] for o in orders]
        else:
            rhs = [torch.from_numpy(i).cuda() for i in ids]
        touched = [len(np.unique(i)) for i in ids]
        # down-projection input: the SwiGLU output per (token, expert) row
        hidden = randn_bf16((T * 4, 1, H), 12) if sorted_mode else randn_bf16((T, 4, 1, H), 12)

        def step(j):
            c = j % copies
            s = j % nsets
            if sorted_mode:
                mq.gather_qmm(xs[s], *gu[c], None, None, rhs[s], True, 32, 4, "mxfp4", sorted_indices=True)
                mq.gather_qmm(hidden, *dn[c], None, None, rhs[s], True, 32, 4, "mxfp4", sorted_indices=True)
            else:
                # x [T,1,1,H] with rhs [T,4]; the down input [T,4,1,H] pairs with rhs through lhs = arange
                mq.gather_qmm(x, *gu[c], None, None, rhs[s], True, 32, 4, "mxfp4")
                mq.gather_qmm(hidden, *dn[c], None, None, rhs[s], True, 32, 4, "mxfp4")

        def all_steps():  # every routing set in one graph: no per-call graph launch
            for j in range(nsets):
                step(j)

        g = capture(all_steps)
        ms = timed_graphs([g], max(iters // nsets, 4), 2) / nsets
        avg_touched = float(np.mean(touched))
        b = avg_touched * per_expert + T * H * 2 + T * 4 * I2 * 2 + T * 4 * H * 2 * 2
        res.append({"T": T, "sorted": sorted_mode, "experts_touched": round(avg_touched, 2), "us": round(ms * 1e3, 2),
                    "GBps": round(b / (ms * 1e-3) / 1e9, 1), "frac_hbm": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 3)})
    return res


def fused_moe(iters=200):
    """Fused single-token decode MoE (mlxq_fused_moe_expert) on Qwen3-30B-A3B
    experts: 128 experts, hidden 2048, expert intermediate 768, top-8, 4-bit
    affine g64; two copies of the expert stacks and 16 routing sets rotate so
    the selected experts stream from HBM.  Compared with the reference's
    fallback on this library: gather_qmm for gate, up and down, torch for
    SiLU * up and the score-weighted sum."""
    E, din, dff, k, gs, bits = 128, 2048, 768, 8, 64, 4
    copies, nsets = 2, 16
    stacks = []
    for c in range(copies):
        stacks.append([make_affine(E * dff, din, bits, gs, 80 + 3 * c), make_affine(E * dff, din, bits, gs, 81 + 3 * c),
                       make_affine(E * din, dff, bits, gs, 82 + 3 * c)])
        g, u, d = stacks[-1]
        stacks[-1] = [tuple(t.view(E, dff, -1) for t in g), tuple(t.view(E, dff, -1) for t in u),
                      tuple(t.view(E, din, -1) for t in d)]
    rng = np.random.default_rng(9)
    ids = [torch.from_numpy(rng.permutation(E)[:k].astype(np.int32)).cuda() for _ in range(nsets)]
    scs = [torch.softmax(torch.randn(k, device="cuda"), 0) for _ in range(nsets)]
    x = randn_bf16((din,), 13)
    out = torch.empty(din, dtype=torch.bfloat16, device="cuda")
    per_expert = 2 * (dff * din * bits // 8 + dff * (din // gs) * 4) + din * dff * bits // 8 + din * (dff // gs) * 4
    nbytes = k * per_expert + 2 * din * 2

    def fused(j):
        g, u, d = stacks[j % copies]
        s = j % nsets
        mq.fused_moe_expert(x, ids[s], *g, *u, *d, scs[s], din, dff, k, bits, bits, gs, out=out)

    def chain(j):
        g, u, d = stacks[j % copies]
        s = j % nsets
        x4 = x.view(1, 1, 1, din)
        rhs = ids[s].view(1, k)
        gt = mq.gather_qmm(x4, *g, None, rhs, True, gs, bits)
        ut = mq.gather_qmm(x4, *u, None, rhs, True, gs, bits)
        a = torch.nn.functional.silu(gt) * ut
        dt = mq.gather_qmm(a, *d, None, rhs, True, gs, bits)
        out.copy_((dt.view(k, din).float() * scs[s].view(k, 1)).sum(0))

    res = {"workload": "qwen3-30b-a3b experts: E=128, din=2048, dff=768, top-8, 4-bit g64, one token",
           "bytes_per_call": nbytes}
    calls = copies * nsets  # one graph holds every (copy, routing set) call: no per-call graph launch
    for name, fn in (("fused", fused), ("gather_chain", chain)):
        def all_calls(fn=fn):
            for j in range(calls):
                fn(j)

        g = capture(all_calls)
        ms = timed_graphs([g], max(iters // calls, 4), 2) / calls
        res[name] = {"us": round(ms * 1e3, 2), "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1),
                     "frac_hbm": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 3)}
    return res


# ---- end-to-end decode --------------------------------
#
# A Qwen3-8B-shaped decoder (36 layers, hidden 4096, 32 query / 8 key-value
# heads of 128, SwiGLU intermediate 12288, vocabulary 151936) with random
# weights ~N(0, 0.02), every linear layer (q/k/v/o, gate/up/down, lm_head)
# 4-bit affine g64 and run through this library's quantized_matmul; the
# glue (RMSNorm, per-head q/k RMSNorm, rotary embedding, grouped-query
# attention over a bf16 KV cache, SwiGLU, residuals, greedy argmax) is
# torch.  The reference measures the same through `mlxcel generate`; MLX is
# not available here, so this driver stands in for mlxcel's model code.
# Attention products keep every right-hand operand contiguous.


class QwenShape:
    def __init__(self, layers=36, hidden=4096, nq=32, nkv=8, hd=128, inter=12288, vocab=151936,
                 eps=1e-6, theta=1.0e6):
        self.layers, self.hidden, self.nq, self.nkv, self.hd = layers, hidden, nq, nkv, hd
        self.inter, self.vocab, self.eps, self.theta = inter, vocab, eps, theta


class QuantDecoder:
    """Random-weight quantized decoder; decode steps capture into HIP graphs."""

    def __init__(self, shape: QwenShape, batch: int, max_ctx: int, seed: int = 0, gs: int = 64, bits: int = 4,
                 multi: bool = True):
        self.c, self.B, self.T, self.gs, self.bits = shape, batch, max_ctx, gs, bits
        self.multi = multi  # q/k/v and gate/up through quantized_matmul_multi
        c = shape
        dev = "cuda"
        gen = torch.Generator(device=dev).manual_seed(seed)

        def lin(out_f, in_f):
            w = (torch.randn(out_f, in_f, device=dev, generator=gen) * 0.02).to(torch.bfloat16)
            q = mq.quantize(w, gs, bits)
            del w
            return q

        def norm(n):
            return (1.0 + 0.02 * torch.randn(n, device=dev, generator=gen)).to(torch.bfloat16)

        self.layers = []
        for _ in range(c.layers):
            self.layers.append(dict(
                q=lin(c.nq * c.hd, c.hidden), k=lin(c.nkv * c.hd, c.hidden), v=lin(c.nkv * c.hd, c.hidden),
                o=lin(c.hidden, c.nq * c.hd), g=lin(c.inter, c.hidden), u=lin(c.inter, c.hidden),
                d=lin(c.hidden, c.inter), n1=norm(c.hidden), n2=norm(c.hidden), qn=norm(c.hd), kn=norm(c.hd)))
        self.embed = (torch.randn(c.vocab, c.hidden, device=dev, generator=gen) * 0.02).to(torch.bfloat16)
        self.lm = lin(c.vocab, c.hidden)
        self.nf = norm(c.hidden)
        self.kc = [torch.zeros(batch, c.nkv, max_ctx, c.hd, dtype=torch.bfloat16, device=dev) for _ in self.layers]
        self.vc = [torch.zeros_like(k) for k in self.kc]
        inv = 1.0 / (c.theta ** (torch.arange(0, c.hd, 2, device=dev, dtype=torch.float32) / c.hd))
        ang = torch.arange(max_ctx, device=dev, dtype=torch.float32)[:, None] * inv[None, :]
        self.cos = torch.cat([ang.cos(), ang.cos()], -1)  # [T, hd]
        self.sin = torch.cat([ang.sin(), ang.sin()], -1)
        self.weight_bytes = sum(t.numel() * t.element_size() for L in self.layers for k in "qkvogud" for t in L[k])
        self.weight_bytes += sum(t.numel() * t.element_size() for t in self.lm)

    def qmm(self, x, w):
        return mq.quantized_matmul(x, *w, True, self.gs, self.bits)

    def qmm_n(self, x, ws):
        if self.multi:
            return mq.quantized_matmul_multi(x, [w[0] for w in ws], [w[1] for w in ws], [w[2] for w in ws],
                                             self.gs, self.bits)
        return [self.qmm(x, w) for w in ws]

    def rms(self, x, w):
        xf = x.float()
        return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.c.eps) * w.float()).to(torch.bfloat16)

    def rope(self, x, cos, sin):
        # x [..., S, heads, hd] (bf16); cos/sin [S, hd]
        xf = x.float()
        h = xf.shape[-1] // 2
        rot = torch.cat([-xf[..., h:], xf[..., :h]], -1)
        return (xf * cos[:, None, :] + rot * sin[:, None, :]).to(torch.bfloat16)

    def attend(self, q, kc, vc, mask):
        # q [B, nkv, G*S, hd]; kc/vc [B, nkv, T, hd] (rows contiguous); mask [G*S, T]
        # additive.  Scores are formed as kc @ q^T so the cache is never a
        # transposed right-hand operand; only small tensors are transposed.
        qt = q.transpose(-1, -2).contiguous()
        st = torch.matmul(kc, qt).float() * (1.0 / math.sqrt(self.c.hd)) + mask.transpose(0, 1)
        p = torch.softmax(st, -2).to(torch.bfloat16).transpose(-1, -2).contiguous()
        return torch.matmul(p, vc)

    def layer(self, L, i, h, pos0, S, T, mask):
        """h [B*S, hidden] at positions pos0 .. pos0+S-1 (pos0: device scalar)."""
        c, B = self.c, self.B
        x = self.rms(h, L["n1"])
        q, k, v = self.qmm_n(x, [L["q"], L["k"], L["v"]])
        q, k, v = q.view(B, S, c.nq, c.hd), k.view(B, S, c.nkv, c.hd), v.view(B, S, c.nkv, c.hd)
        q, k = self.rms(q, L["qn"]), self.rms(k, L["kn"])
        idx = pos0 + torch.arange(S, device=h.device)
        cos, sin = self.cos.index_select(0, idx), self.sin.index_select(0, idx)
        q, k = self.rope(q, cos, sin), self.rope(k, cos, sin)
        self.kc[i].index_copy_(2, idx, k.transpose(1, 2))
        self.vc[i].index_copy_(2, idx, v.transpose(1, 2))
        G = c.nq // c.nkv
        qg = q.view(B, S, c.nkv, G, c.hd).permute(0, 2, 3, 1, 4).reshape(B, c.nkv, G * S, c.hd)
        o = self.attend(qg, self.kc[i][:, :, :T], self.vc[i][:, :, :T], mask)
        o = o.view(B, c.nkv, G, S, c.hd).permute(0, 3, 1, 2, 4).reshape(B * S, c.nq * c.hd)
        h = h + self.qmm(o, L["o"])
        x = self.rms(h, L["n2"])
        gt, ut = self.qmm_n(x, [L["g"], L["u"]])
        a = torch.nn.functional.silu(gt.float()) * ut.float()
        return h + self.qmm(a.to(torch.bfloat16), L["d"])

    def forward(self, tokens, pos0, S, T, mask):
        h = self.embed.index_select(0, tokens.reshape(-1))
        for i, L in enumerate(self.layers):
            h = self.layer(L, i, h, pos0, S, T, mask)
        return self.qmm(self.rms(h.view(self.B, S, -1)[:, -1], self.nf), self.lm)  # logits of the last position

    def prefill(self, prompt):
        """prompt [B, S] int64 -> logits [B, vocab] of the last position (causal attention)."""
        S = prompt.shape[1]
        G = self.c.nq // self.c.nkv
        causal = torch.full((S, S), float("-inf"), device=prompt.device).triu(1)
        mask = causal.repeat(G, 1)  # rows (g, s)
        return self.forward(prompt, torch.zeros((), dtype=torch.int64, device=prompt.device), S, S, mask)

    def decode_graph(self, T):
        """Graph of one greedy decode step attending to cache positions < T:
        reads self.tok [B] and self.pos (device), writes the next token into
        self.tok and advances self.pos."""
        dev = self.embed.device
        G = self.c.nq // self.c.nkv

        if getattr(self, "logits", None) is None:
            self.logits = torch.empty(self.B, self.c.vocab, dtype=torch.bfloat16, device=dev)

        def step():
            ar = torch.arange(T, device=dev)
            mask = torch.where(ar[None, :] <= self.pos, 0.0, float("-inf")).expand(G, T)
            logits = self.forward(self.tok, self.pos, 1, T, mask)
            self.logits.copy_(logits)
            self.tok.copy_(torch.argmax(logits, -1))
            self.pos.add_(1)

        saved = (self.tok.clone(), self.pos.clone())
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            step()  # warm-up on the capture stream (library workspace, allocator pools)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            step()
        torch.cuda.synchronize()
        self.tok.copy_(saved[0])
        self.pos.copy_(saved[1])
        return g

    def projections_graph(self):
        """Graph of one decode step's quantized projections alone (every
        layer's q/k/v, o, gate/up and down, then the LM head) on fixed
        activations of the step's shapes: the library's share of a step."""
        c, B = self.c, self.B
        xh = randn_bf16((B, c.hidden), 21)
        xo = randn_bf16((B, c.nq * c.hd), 22)
        xi = randn_bf16((B, c.inter), 23)

        def run():
            for L in self.layers:
                self.qmm_n(xh, [L["q"], L["k"], L["v"]])
                self.qmm(xo, L["o"])
                self.qmm_n(xh, [L["g"], L["u"]])
                self.qmm(xi, L["d"])
            self.qmm(xh, self.lm)

        return capture(run)

    def generate(self, prompt, steps, bucket=64):
        """Greedy decode `steps` tokens after `prompt`; returns (tokens [B, steps],
        prefill seconds, decode seconds).  Each step replays the graph of the
        smallest cache bucket covering its position."""
        B, S = prompt.shape
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        logits = self.prefill(prompt)
        torch.cuda.synchronize()
        t_pre = time.perf_counter() - t0
        self.tok = torch.argmax(logits, -1)
        self.pos = torch.full((), S, dtype=torch.int64, device=prompt.device)
        graphs = {}
        for p in range(S, S + steps):
            T = min(self.T, ((p + 1 + bucket - 1) // bucket) * bucket)
            if T not in graphs:
                graphs[T] = self.decode_graph(T)
        out = torch.empty(B, steps, dtype=torch.int64, device=prompt.device)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i, p in enumerate(range(S, S + steps)):
            out[:, i] = self.tok
            T = min(self.T, ((p + 1 + bucket - 1) // bucket) * bucket)
            graphs[T].replay()
        torch.cuda.synchronize()
        return out, t_pre, time.perf_counter() - t0


def e2e_decode(batches=(1, 16), prompt_len=512, steps=256, layers=36, separate_at=(1,)):
    """Decode tokens/s of the Qwen3-8B-shaped 4-bit model at each batch (q/k/v
    and gate/up through quantized_matmul_multi; at the batches in
    `separate_at` also with one quantized_matmul call per projection)."""
    res = []
    runs = [(B, True) for B in batches] + [(B, False) for B in separate_at]
    for B, multi in runs:
        model = QuantDecoder(QwenShape(layers=layers), B, prompt_len + steps, seed=11, multi=multi)
        g = torch.Generator(device="cuda").manual_seed(12)
        prompt = torch.randint(0, model.c.vocab, (B, prompt_len), device="cuda", generator=g)
        model.generate(prompt[:, :64], 8)  # warm-up (kernels, allocator)
        toks, t_pre, t_dec = model.generate(prompt, steps)
        # the same step's quantized projections alone, replayed back to back
        lib_ms = timed_graphs([model.projections_graph()], 20, 3)
        step_ms = t_dec / steps * 1e3
        res.append({"batch": B, "multi_projection": multi, "prompt": prompt_len, "decode_tokens": steps,
                    "decode_tok_s": round(B * steps / t_dec, 1), "ms_per_step": round(step_ms, 3),
                    "library_ms_per_step": round(lib_ms, 3), "library_share": round(lib_ms / step_ms, 3),
                    "prefill_tok_s": round(B * prompt_len / t_pre, 1),
                    "weight_GB": round(model.weight_bytes / 1e9, 3),
                    "weight_stream_GBps": round(model.weight_bytes / (t_dec / steps) / 1e9, 1),
                    "library_weight_stream_GBps": round(model.weight_bytes / (lib_ms * 1e-3) / 1e9, 1)})
        del model
        torch.cuda.empty_cache()
    return res


def host_facts():
    """The host the CPU baseline runs on: logical CPUs (and those this
    process may use), the CPU model, and how the oracle was compiled."""
    import oracle as orc

    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count()
    return {"nproc": os.cpu_count(), "nproc_usable": usable, "cpu_model": model, **orc.build_info()}


def cpu_time(w, x, N, K, budget_s):
    """Seconds per call of the single-core oracle `_qmm_t` (the restatement of
    MLX's CPU path, overlays/cpu/mlx/backend/cpu/quantized.cpp:199-257) on
    the weights `w` and activation row `x`, over calls filling `budget_s`."""
    import oracle as orc

    wq, s, b = w
    wq_h = wq.cpu().numpy()
    s_h = s.cpu().view(torch.int16).numpy().astype(np.uint16)
    b_h = b.cpu().view(torch.int16).numpy().astype(np.uint16)
    x_h = x.cpu().view(torch.int16).numpy().astype(np.uint16).reshape(1, K)
    orc.qmm_t_affine(x_h, wq_h, s_h, b_h, 64, 4)  # warm
    n, t0 = 0, time.perf_counter()
    while True:
        orc.qmm_t_affine(x_h, wq_h, s_h, b_h, 64, 4)
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    per = el / n
    return {"GBps": round(qmv_bytes(1, N, K, 4, 64) / per / 1e9, 3), "ms_per_call": round(per * 1e3, 2),
            "calls": n, "cores": 1}


def cpu_baseline(gate, budget_s=10.0):
    """Single-core oracle `_qmm_t` on the gate projection (same bytes as the GPU launch)."""
    x = randn_bf16((1, 4096), 99)
    t = cpu_time(gate, x, 14336, 4096, budget_s)
    return {"value": t["GBps"], "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{t['calls']} calls of the gate projection (N=14336, K=4096, 4-bit g64, M=1), "
                      f"{t['ms_per_call']:.1f} ms/call, oracle restatement of MLX CPU _qmm_t (scalar, 1 thread)",
            **host_facts()}


def traffic_probe():
    """Dispatches whose HBM counters calibrate and measure traffic: a device
    copy of exactly 256 MiB (reads 256 MiB, writes 256 MiB), the gate
    projection over 5 distinct weight sets (33,067,008 algorithmic bytes each),
    then 5 sorted mxfp4 MoE gathers at T=256 (gate/up, 299,704,320 bytes each)."""
    n = 256 << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    gates = [make_affine(14336, 4096, 4, 64, 2000 + c) for c in range(5)]
    x = randn_bf16((1, 4096), 7)
    out = torch.empty(1, 14336, dtype=torch.bfloat16, device="cuda")
    torch.cuda.synchronize()
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    for g in gates:
        mq.quantized_matmul(x, *g, True, 64, 4, out=out)
    torch.cuda.synchronize()
    del gates
    # the sorted MoE gather at T=256 (gate/up, 32 mxfp4 experts, top-4): 5
    # launches of qmm_group_mxfp4_kernel over one weight set
    E, H, I2, T = 32, 2880, 5760, 256
    gu = make_mxfp4(E, I2, H, 60)
    ids = np.stack([np.random.default_rng(5 + t).permutation(E)[:4] for t in range(T)]).reshape(-1)
    order = np.argsort(ids, kind="stable")
    rhs = torch.from_numpy(ids[order].astype(np.int32)).cuda()
    xg = randn_bf16((T, 1, H), 11)[torch.from_numpy(order // 4).cuda()]
    torch.cuda.synchronize()
    for _ in range(5):
        mq.gather_qmm(xg, *gu, None, None, rhs, True, 32, 4, "mxfp4", sorted_indices=True)
    torch.cuda.synchronize()
    gather_bytes = E * (I2 * H // 2 + I2 * H // 32) + T * 4 * (H + I2) * 2
    print(json.dumps({"traffic_probe": {"copy_bytes": n, "gate_algorithmic_bytes": qmv_bytes(1, 14336, 4096, 4, 64),
                                        "gather_t256_gate_up_algorithmic_bytes": gather_bytes}}))


def prefill_probe():
    """Dispatches for rocprofv3 counter passes over the prefill GEMM: the 8
    configs[2] cases (4/8-bit x gate/up and down x M=512/2048), two launches
    each on distinct weights, in the order printed."""
    cases = []
    for bits in (4, 8):
        for (N, K, name) in ((14336, 4096, "gate_up"), (4096, 14336, "down")):
            ws = [make_affine(N, K, bits, 64, 90 + c) for c in range(2)]
            for M in (512, 2048):
                x = randn_bf16((M, K), 13)
                out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
                torch.cuda.synchronize()
                for w in ws:
                    mq.quantized_matmul(x, *w, True, 64, bits, out=out)
                torch.cuda.synchronize()
                cases.append({"bits": bits, "shape": name, "M": M, "N": N, "K": K, "launches": len(ws)})
            del ws
    print(json.dumps({"prefill_probe": cases}))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--extras", default="copy,c1,sweep,qmm,gather,moe,e2e,general",
                    help="comma-separated extra sections: copy, c1, sweep, qmm, gather, moe, e2e, general "
                         "(and nsweep, routes, not in the default set)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="run 5 copies of 256 MiB and 5 gate launches, eager, for rocprofv3 --pmc")
    ap.add_argument("--prefill-probe", action="store_true",
                    help="run the 8 prefill GEMM configs twice each, eager, for rocprofv3 --pmc")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build runs the quantized-matmul kernels on a single "
              "MI355X; sharding across GPUs is a design, not a run.", file=sys.stderr)
        sys.exit(2)
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.set_device(0)
    mq.load_library()
    if args.traffic_probe:
        traffic_probe()
        return
    if args.prefill_probe:
        prefill_probe()
        return

    value, ms, launch_us, per_launch, gate_us, gate, multi_value, multi_ms = headline(args.steps, args.warmup)
    achieved = per_launch / (gate_us * 1e-6) / 1e9
    ceiling = read_ceiling(per_launch)
    line = {
        "metric": "qmv HBM GB/s at M=1 (4-bit affine g64, Llama-3-8B MLP decode projections)",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: x ~ N(0,1) bf16, W ~ N(0,0.02) bf16 quantized MLX-style (affine 4-bit, g64)",
        "config": {"workload": "llama3-8b MLP decode qmv: gate+up (N=14336,K=4096) + down (N=4096,K=14336), M=1",
                   "bits": 4, "group_size": 64, "M": 1, "layers_rotated": 8,
                   "bytes_per_step": 3 * per_launch, "avg_us_per_launch": round(launch_us, 3)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": TRAFFIC_GATE,
                     "kernel": "qmv_rs_dense_kernel<AFF4, MR=1, R=8, CPW=1, UPW=4> (gate, N=14336 K=4096 M=1)",
                     "timing": "graph replay of 8 back-to-back launches, HIP events on the replay stream; "
                               "per-launch time includes the dispatch gap between dependent kernels",
                     "bytes_per_launch": per_launch, "avg_launch_us": round(gate_us, 3),
                     "read_ceiling": ceiling, "frac_of_read_ceiling": round(achieved / ceiling["GBps"], 3)},
    }
    if not args.no_extra:
        want = set(args.extras.split(","))
        extra = {"mlp_step_gate_up_multi": {"GBps": round(multi_value, 1), "ms_per_step": round(multi_ms, 5),
                                            "note": "the headline step with gate+up as one quantized_matmul_multi "
                                                    "launch (2 launches per step instead of 3)"}}
        if "copy" in want:
            extra["copy_ceiling_GBps"] = round(copy_ceiling(), 1)
        if "c1" in want:
            extra["c1_qmv_4096"] = c1_qmv(with_cpu=not args.no_cpu)
        if "nsweep" in want:
            extra["qmv_n_sweep"] = n_sweep()
        if "routes" in want:
            extra["qmv_route_audit"] = route_audit()
        if "sweep" in want:
            extra["qmv_sweep"] = qmv_sweep()
        if "qmm" in want:
            extra["qmm_prefill"] = qmm_prefill()
        if "gather" in want:
            extra["gather_mxfp4_moe"] = gather_moe()
        if "moe" in want:
            extra["fused_moe_decode"] = fused_moe()
        if "e2e" in want:
            extra["e2e_decode_qwen3_8b_shape"] = e2e_decode()
        if "general" in want:
            extra["general_path"] = general_path()
        line["extra"] = extra
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(gate)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
