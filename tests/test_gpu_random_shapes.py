"""GPU parity over seeded random shapes: each case draws a route's inputs
(rows 1-513 across every routing boundary, ragged N, K any multiple of the
group size, 4/8-bit affine at group sizes 32/64/128, mxfp4, float16 and
float32 activations, 2-6-bit codes, batched weights, gathers with several
rows per entry and explicit lhs, transpose=false, strided activations,
dequantize) and checks the library against the oracle: the C restatement of
MLX's `_qmm_t` / `fp_qmm_t` (overlays/cpu/mlx/backend/cpu/quantized.cpp:
199-257, 550-597) for bfloat16, the float64 numpy restatement
(oracle/generic.py) otherwise, max|y - y_ref| / max|y_ref| <= 1e-2 (1e-4 for
float32 results).  Fixed seeds: the same cases every run.  Cases like these
found two defects that the fixed-shape tests had missed: the tile kernel's
last output column when the scale rows end inside a dword, and calls of
17-64 rows per matrix at 4-bit g128 that were refused.
"""
import numpy as np
import pytest
import torch

import mlxcel_amd as mq
import oracle as orc
from oracle import generic as og
from helpers import affine_case, announce, dev_bf16, dev_u32, dev_u8, host_u16, max_rel, mxfp4_case

pytestmark = pytest.mark.gpu

ROWS = [1, 2, 3, 4, 5, 6, 8, 9, 12, 15, 16, 17, 24, 33, 64, 65, 128, 129, 200, 257, 300, 513]
TD = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}


def _dev(rng, shape, dt, lo=None, hi=None):
    vals = rng.standard_normal(shape) if lo is None else rng.uniform(lo, hi, size=shape)
    t = torch.from_numpy(np.asarray(vals, dtype=np.float32)).to(TD[dt]).cuda()
    return t, t.float().cpu().numpy().astype(np.float64)


def _rel(y, want64, dt):
    got = y.float().cpu().numpy().astype(np.float64)
    want = og.round_to(want64, dt)
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-30))


def _weights(rng, lead, cols, bits, gs, dt, mode):
    if mode == "mxfp4":
        wq = og.pack_codes(rng.integers(0, 16, size=lead + (cols,)), 4)
        sc = rng.integers(118, 126, size=lead + (cols // 32,)).astype(np.uint8)
        return (dev_u32(wq), torch.from_numpy(sc).cuda(), None), (wq, sc.astype(np.float64), None)
    wq = og.pack_codes(rng.integers(0, 1 << bits, size=lead + (cols,)), bits)
    s, sv = _dev(rng, lead + (cols // gs,), dt, 0.002, 0.02)
    b, bv = _dev(rng, lead + (cols // gs,), dt, -0.1, 0.1)
    return (dev_u32(wq), s, b), (wq, sv, bv)


def _dense_case(rng):
    """bfloat16 4/8-bit affine or mxfp4, transpose=true, 2-D weights: the specialised routes."""
    while True:
        kind = rng.choice(["aff", "aff", "mx"])
        M = int(rng.choice(ROWS))
        N = int(rng.integers(1, 3000)) if rng.random() < 0.5 else int(rng.choice([64, 256, 1000, 2880, 4096]))
        if kind == "aff":
            bits, gs = int(rng.choice([4, 8])), int(rng.choice([32, 64, 128]))
            K = gs * int(rng.integers(1, max(2, 6144 // gs)))
        else:
            bits, gs = 4, 32
            K = 32 * int(rng.integers(1, 160))
        if M * N * K <= 1.5e8:
            return kind, bits, gs, M, N, K


@pytest.mark.parametrize("seed", range(60))
def test_random_dense_routes(seed):
    rng = np.random.default_rng(9000 + seed)
    kind, bits, gs, M, N, K = _dense_case(rng)
    announce("random_dense", seed, kind, bits, gs, M, N, K)
    if kind == "aff":
        x, wq, s, b = affine_case(M, N, K, gs, bits, int(rng.integers(1 << 30)))
        y = host_u16(mq.quantized_matmul(dev_bf16(x), dev_u32(wq), dev_bf16(s), dev_bf16(b), True, gs, bits))
        want = orc.qmm_t_affine(x, wq, s, b, gs, bits)
    else:
        x, wq, sc = mxfp4_case(M, N, K, int(rng.integers(1 << 30)))
        y = host_u16(mq.quantized_matmul(dev_bf16(x), dev_u32(wq), dev_u8(sc), None, True, 32, 4, "mxfp4"))
        want = orc.fp_qmm_t_mxfp4(x, wq, sc)
    assert max_rel(y, want) <= 1e-2


@pytest.mark.parametrize("seed", range(40))
def test_random_general_routes(seed):
    rng = np.random.default_rng(9500 + seed)
    kind = ["gather_rows", "batched", "no_transpose", "float32", "strided"][seed % 5]
    mode = "mxfp4" if rng.random() < 0.25 else "affine"
    bits = 4 if mode == "mxfp4" else int(rng.choice([2, 3, 4, 5, 6, 8]))
    gs = 32 if mode == "mxfp4" else int(rng.choice([32, 64, 128]))
    dt = "float32" if kind == "float32" else ("bfloat16" if mode == "mxfp4" or rng.random() < 0.7 else "float16")
    if kind == "gather_rows":
        E, X, M = int(rng.integers(1, 12)), int(rng.integers(1, 6)), int(rng.choice([1, 2, 5, 16, 40, 64]))
        B, N, K = int(rng.choice([1, 3, 8, 33])), int(rng.choice([64, 200, 577])), gs * int(rng.integers(1, 40))
        announce("random_general", seed, kind, mode, bits, gs, dt, E, X, M, B, N, K)
        x, xv = _dev(rng, (X, M, K), dt)
        (wq, s, b), (wqn, sv, bv) = _weights(rng, (E, N), K, bits, gs, dt, mode)
        lhs, rhs = rng.integers(0, X, B), rng.integers(0, E, B)
        srt = bool(rng.random() < 0.3)
        if srt:
            o = np.argsort(rhs, kind="stable")
            lhs, rhs = lhs[o], rhs[o]
        y = mq.gather_qmm(x, wq, s, b, torch.from_numpy(lhs.astype(np.int32)).cuda(),
                          torch.from_numpy(rhs.astype(np.int32)).cuda(), True, gs, bits, mode, sorted_indices=srt)
        want = og.gather_qmm(xv, wqn, sv, bv, lhs, rhs, True, gs, bits, mode)
    elif kind == "batched":
        E, M, N, K = int(rng.integers(1, 5)), int(rng.choice([1, 2, 9, 17, 64])), int(rng.choice([64, 200])), gs * int(rng.integers(1, 30))
        announce("random_general", seed, kind, mode, bits, gs, dt, E, M, N, K)
        x, xv = _dev(rng, (E, M, K), dt)
        (wq, s, b), (wqn, sv, bv) = _weights(rng, (E, N), K, bits, gs, dt, mode)
        y = mq.quantized_matmul(x, wq, s, b, True, gs, bits, mode)
        want = np.stack([og.qmm(xv[e], wqn[e], sv[e], None if bv is None else bv[e], True, gs, bits, mode)
                         for e in range(E)])
    elif kind in ("no_transpose", "float32"):
        tr = kind == "float32" and rng.random() < 0.5
        M, N, K = int(rng.choice([1, 2, 5, 16, 33])), gs * int(rng.integers(1, 16)), gs * int(rng.integers(1, 16))
        announce("random_general", seed, kind, mode, bits, gs, dt, M, N, K, tr)
        x, xv = _dev(rng, (M, K), dt)
        rows, cols = (N, K) if tr else (K, N)
        (wq, s, b), (wqn, sv, bv) = _weights(rng, (rows,), cols, bits, gs, dt, mode)
        y = mq.quantized_matmul(x, wq, s, b, tr, gs, bits, mode)
        want = og.qmm(xv, wqn, sv, bv, tr, gs, bits, mode)
    else:
        if mode == "affine":
            bits = int(rng.choice([4, 8]))
        M, N, K = int(rng.choice([1, 3, 8, 20, 70])), int(rng.choice([64, 130, 256])), gs * int(rng.integers(1, 30))
        announce("random_general", seed, kind, mode, bits, gs, dt, M, N, K)
        wide, wv = _dev(rng, (M, 2 * K), dt)
        (wq, s, b), (wqn, sv, bv) = _weights(rng, (N,), K, bits, gs, dt, mode)
        y = mq.quantized_matmul(wide[:, ::2], wq, s, b, True, gs, bits, mode)
        want = og.qmm(wv[:, ::2], wqn, sv, bv, True, gs, bits, mode)
    assert _rel(y, want, dt) <= (1e-4 if dt == "float32" else 1e-2)


@pytest.mark.parametrize("seed", range(10))
def test_random_dequantize(seed):
    rng = np.random.default_rng(9800 + seed)
    mode = "mxfp4" if seed % 3 == 0 else "affine"
    bits = 4 if mode == "mxfp4" else int(rng.choice([2, 3, 4, 5, 6, 8]))
    gs = 32 if mode == "mxfp4" else int(rng.choice([32, 64, 128]))
    dt = "bfloat16" if mode == "mxfp4" else str(rng.choice(["bfloat16", "float16"]))
    N, K = int(rng.integers(1, 300)), gs * int(rng.integers(1, 40))
    announce("random_dequantize", seed, mode, bits, gs, dt, N, K)
    (wq, s, b), (wqn, sv, bv) = _weights(rng, (N,), K, bits, gs, dt, mode)
    y = mq.dequantize(wq, s, b, gs, bits, mode)
    assert _rel(y, og.dequantize(wqn, sv, bv, gs, bits, K, mode), dt) <= 1e-2
