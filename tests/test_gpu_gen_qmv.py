"""GPU parity of the general path's decode kernels (qmm_gen.hip):
`qmv_gen_kernel` (transpose=true, 1-4 activation rows per weight matrix)
and `qmv_gen_t_kernel` (transpose=false, 1-2 rows, codes packed along N, K
split over workgroups): affine codes of 1-6 and 8 bits read as MLX's little-endian
bit stream (overlays/cpu/mlx/backend/cpu/quantized.cpp:107-137), any element
type of x / scales / biases, 2-D weights, batched weights and gather
segments.

Checked against the float64 numpy restatement of MLX's CPU `_qmm_t`
(oracle/generic.py) at max|y - y_ref| / max|y_ref| <= 1e-2 for 16-bit results
and <= 1e-4 for float32 results, and against the tile kernel it replaces for
these shapes (MLXQ_GEN_QMV=0) at the same bounds.  Ragged N (not a multiple
of the 32 rows a workgroup covers), K from one 32-position piece to more than
64 pieces per lane pass, and every group size.
"""
import numpy as np
import pytest
import torch

import mlxcel_amd as mq
from oracle import generic as og
from helpers import announce, dev_u32, setknob

pytestmark = pytest.mark.gpu

TD = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}


def _dev(vals, dt):
    t = torch.from_numpy(np.asarray(vals, dtype=np.float32)).to(TD[dt]).cuda()
    return t, t.float().cpu().numpy().astype(np.float64)


def _rel(y, want64, dt):
    assert y.dtype == TD[dt]
    got = y.float().cpu().numpy().astype(np.float64)
    want = og.round_to(want64, dt)
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-30))


def _tol(dt):
    return 1e-4 if dt == "float32" else 1e-2


def _weights(rng, lead, N, K, bits, gs, st):
    codes = rng.integers(0, 1 << bits, size=lead + (N, K))
    wqn = og.pack_codes(codes, bits)
    s, sv = _dev(rng.uniform(0.002, 0.02, size=lead + (N, K // gs)), st)
    b, bv = _dev(rng.uniform(-0.1, 0.1, size=lead + (N, K // gs)), st)
    return (dev_u32(wqn), s, b), (wqn, sv, bv)


@pytest.mark.parametrize("bits", [1, 2, 3, 5, 6])
@pytest.mark.parametrize("M", [1, 2, 3, 4])
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_code_widths_bfloat16(bits, M, gs):
    rng = np.random.default_rng(31000 + 10 * bits + M + gs)
    N, K = 77, gs * 9
    announce("gen_qmv", bits, M, gs, N, K)
    x, xv = _dev(rng.standard_normal((M, K)), "bfloat16")
    (wq, s, b), (wqn, sv, bv) = _weights(rng, (), N, K, bits, gs, "bfloat16")
    y = mq.quantized_matmul(x, wq, s, b, True, gs, bits)
    assert _rel(y, og.qmm(xv, wqn, sv, bv, True, gs, bits), "bfloat16") <= 1e-2


@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("xt,st,out", [("float32", "float32", "float32"), ("float16", "float16", "float16"),
                                       ("bfloat16", "float32", "float32"), ("float16", "bfloat16", "float32")])
def test_element_types(bits, xt, st, out):
    rng = np.random.default_rng(32000 + bits)
    N, K, gs = 300, 2048, 64
    M = 4 if bits % 2 else 1
    announce("gen_qmv_types", bits, xt, st, M, N, K)
    x, xv = _dev(rng.standard_normal((M, K)), xt)
    (wq, s, b), (wqn, sv, bv) = _weights(rng, (), N, K, bits, gs, st)
    y = mq.quantized_matmul(x, wq, s, b, True, gs, bits)
    assert _rel(y, og.qmm(xv, wqn, sv, bv, True, gs, bits), out) <= _tol(out)


@pytest.mark.parametrize("N,K", [(1, 32), (33, 96), (4096, 4096), (1000, 14336)])
@pytest.mark.parametrize("bits", [3, 6])
def test_shapes_against_the_tile_kernel(monkeypatch, N, K, bits):
    rng = np.random.default_rng(33000 + N + K + bits)
    gs = 32
    announce("gen_qmv_vs_tile", bits, N, K)
    x, xv = _dev(rng.standard_normal((2 if bits == 3 else 3, K)), "float16")
    (wq, s, b), (wqn, sv, bv) = _weights(rng, (), N, K, bits, gs, "float16")
    y = mq.quantized_matmul(x, wq, s, b, True, gs, bits)
    want = og.qmm(xv, wqn, sv, bv, True, gs, bits)
    assert _rel(y, want, "float16") <= 1e-2
    setknob(monkeypatch, "MLXQ_GEN_QMV", "0")
    y_tile = mq.quantized_matmul(x, wq, s, b, True, gs, bits)
    assert _rel(y_tile, want, "float16") <= 1e-2
    got, ref = y.float().cpu().numpy(), y_tile.float().cpu().numpy()
    assert float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30)) <= 1e-2


def test_batched_weights():
    rng = np.random.default_rng(34000)
    E, M, N, K, bits, gs = 3, 4, 130, 512, 5, 64
    announce("gen_qmv_batched", E, M, N, K, bits)
    x, xv = _dev(rng.standard_normal((E, M, K)), "bfloat16")
    (wq, s, b), (wqn, sv, bv) = _weights(rng, (E,), N, K, bits, gs, "bfloat16")
    y = mq.quantized_matmul(x, wq, s, b, True, gs, bits)
    want = np.stack([og.qmm(xv[e], wqn[e], sv[e], bv[e], True, gs, bits) for e in range(E)])
    assert _rel(y, want, "bfloat16") <= 1e-2


@pytest.mark.parametrize("M", [1, 2, 3])
def test_gather_segments(M):
    rng = np.random.default_rng(35000 + M)
    E, X, B, N, K, bits, gs = 6, 4, 11, 96, 384, 3, 64
    announce("gen_qmv_gather", M, E, X, B, N, K, bits)
    x, xv = _dev(rng.standard_normal((X, M, K)), "bfloat16")
    (wq, s, b), (wqn, sv, bv) = _weights(rng, (E,), N, K, bits, gs, "bfloat16")
    lhs, rhs = rng.integers(0, X, B), rng.integers(0, E, B)
    y = mq.gather_qmm(x, wq, s, b, torch.from_numpy(lhs.astype(np.int32)).cuda(),
                      torch.from_numpy(rhs.astype(np.int32)).cuda(), True, gs, bits)
    want = og.gather_qmm(xv, wqn, sv, bv, lhs, rhs, True, gs, bits, "affine")
    assert _rel(y, want, "bfloat16") <= 1e-2


# transpose=false: W is [K][N] with codes packed along N (qmv_gen_t_kernel);
# K needs no alignment, N is a multiple of the group size.
def _weights_t(rng, lead, K, N, bits, gs, st):
    codes = rng.integers(0, 1 << bits, size=lead + (K, N))
    wqn = og.pack_codes(codes, bits)
    s, sv = _dev(rng.uniform(0.002, 0.02, size=lead + (K, N // gs)), st)
    b, bv = _dev(rng.uniform(-0.1, 0.1, size=lead + (K, N // gs)), st)
    return (dev_u32(wqn), s, b), (wqn, sv, bv)


@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("M", [1, 2])
@pytest.mark.parametrize("xt", ["bfloat16", "float32"])
def test_no_transpose_widths(bits, M, xt):
    rng = np.random.default_rng(36000 + 10 * bits + M)
    K, N, gs = 333, 2112, 64  # a partial 2048-column block, K over several ranges
    announce("gen_qmv_t", bits, M, xt, K, N)
    x, xv = _dev(rng.standard_normal((M, K)), xt)
    (wq, s, b), (wqn, sv, bv) = _weights_t(rng, (), K, N, bits, gs, xt)
    y = mq.quantized_matmul(x, wq, s, b, False, gs, bits)
    assert _rel(y, og.qmm(xv, wqn, sv, bv, False, gs, bits), xt) <= _tol(xt)


@pytest.mark.parametrize("K,N,gs", [(1, 32, 32), (7, 64, 64), (100, 128, 128), (4096, 4096, 64), (4096, 14336, 64)])
def test_no_transpose_shapes_against_the_tile_kernel(monkeypatch, K, N, gs):
    rng = np.random.default_rng(37000 + K + N)
    bits = 4
    announce("gen_qmv_t_vs_tile", K, N, gs)
    x, xv = _dev(rng.standard_normal((1, K)), "bfloat16")
    (wq, s, b), (wqn, sv, bv) = _weights_t(rng, (), K, N, bits, gs, "bfloat16")
    y = mq.quantized_matmul(x, wq, s, b, False, gs, bits)
    want = og.qmm(xv, wqn, sv, bv, False, gs, bits)
    assert _rel(y, want, "bfloat16") <= 1e-2
    setknob(monkeypatch, "MLXQ_GEN_QMV", "0")
    y_tile = mq.quantized_matmul(x, wq, s, b, False, gs, bits)
    assert _rel(y_tile, want, "bfloat16") <= 1e-2


def test_no_transpose_gather():
    rng = np.random.default_rng(38000)
    E, X, B, K, N, bits, gs = 5, 3, 9, 200, 256, 6, 32
    announce("gen_qmv_t_gather", E, X, B, K, N, bits)
    x, xv = _dev(rng.standard_normal((X, 1, K)), "float16")
    (wq, s, b), (wqn, sv, bv) = _weights_t(rng, (E,), K, N, bits, gs, "float16")
    lhs, rhs = rng.integers(0, X, B), rng.integers(0, E, B)
    y = mq.gather_qmm(x, wq, s, b, torch.from_numpy(lhs.astype(np.int32)).cuda(),
                      torch.from_numpy(rhs.astype(np.int32)).cuda(), False, gs, bits)
    want = og.gather_qmm(xv, wqn, sv, bv, lhs, rhs, False, gs, bits, "affine")
    assert _rel(y, want, "float16") <= 1e-2
