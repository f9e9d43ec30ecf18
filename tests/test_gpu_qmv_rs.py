"""GPU parity of the three decode kernels behind quantized_matmul /
gather_qmm: the row-streaming kernel (1-2 rows per weight matrix, default
there; up to 4 when forced), the full-row kernel (1-2 rows) and the MFMA
kernel (default above 2 rows), each forced in turn with
MLXQ_QMV_KERNEL=fr|rs|mfma, against the oracle's
restatement of MLX's `_qmm_t` / `fp_qmm_t` (overlays/cpu/mlx/backend/cpu/
quantized.cpp:199-257, 550-597), max|y - y_ref| / max|y_ref| <= 1e-2.

Shapes are chosen to reach every launch variant: rows per wave (fr) or per
workgroup (rs) via MLXQ_QMV_R, rows of 1, 2, 3-4, 5-8 and 9-16 chunks of
1 KiB, rows that end inside a chunk, N not a multiple of the tile.
"""
import numpy as np
import pytest
import torch

import mlxcel_amd as mq
import oracle as orc
from helpers import TOL, affine_case, announce, dev_bf16, dev_u32, dev_u8, host_u16, max_rel, mxfp4_case, setknob

pytestmark = pytest.mark.gpu

KERNEL_R = [("fr", 0), ("fr", 1), ("fr", 2), ("fr", 4), ("fr", 8), ("rs", 4), ("rs", 8), ("rs", 16), ("mfma", 0)]


def affine(x, wq, s, b, gs, bits):
    y = mq.quantized_matmul(dev_bf16(x), dev_u32(wq), dev_bf16(s), dev_bf16(b), True, gs, bits)
    torch.cuda.synchronize()
    return host_u16(y)


def mxfp4(x, wq, sc):
    y = mq.quantized_matmul(dev_bf16(x), dev_u32(wq), dev_u8(sc), None, True, 32, 4, "mxfp4")
    torch.cuda.synchronize()
    return host_u16(y)


@pytest.mark.parametrize("kernel,R", KERNEL_R)
@pytest.mark.parametrize("bits,gs", [(4, 32), (4, 64), (4, 128), (8, 32), (8, 64), (8, 128)])
@pytest.mark.parametrize("M", [1, 2, 3, 4])
def test_affine_kernels(monkeypatch, kernel, R, bits, gs, M):
    setknob(monkeypatch, "MLXQ_QMV_KERNEL", kernel)
    setknob(monkeypatch, "MLXQ_QMV_R", str(R))
    N, K = 200, 2304  # 4-bit: 2 chunks per row, the second one ends mid-chunk
    announce("skinny_affine", kernel, R, bits, gs, M)
    x, wq, s, b = affine_case(M, N, K, gs, bits, 900 + M + bits + gs + R)
    assert max_rel(affine(x, wq, s, b, gs, bits), orc.qmm_t_affine(x, wq, s, b, gs, bits)) <= TOL


@pytest.mark.parametrize("kernel", ["fr", "rs"])
@pytest.mark.parametrize("M", [1, 2])
@pytest.mark.parametrize("bits,K", [(4, 1024), (4, 512), (4, 6144), (8, 6144), (4, 16384), (8, 2048)])
def test_affine_chunk_counts(monkeypatch, kernel, M, bits, K):
    # 1, 4, 8 and 16 chunks per row (compiled chunk bounds 1/4/8/16)
    setknob(monkeypatch, "MLXQ_QMV_KERNEL", kernel)
    announce("skinny_chunks", kernel, M, bits, K)
    x, wq, s, b = affine_case(M, 72, K, 64, bits, 970 + M + bits + K)
    assert max_rel(affine(x, wq, s, b, 64, bits), orc.qmm_t_affine(x, wq, s, b, 64, bits)) <= TOL


@pytest.mark.parametrize("kernel", ["fr", "rs", "mfma"])
@pytest.mark.parametrize("M", [1, 2, 4])
@pytest.mark.parametrize("bits,K", [(4, 28672), (8, 14336), (8, 9216)])
def test_affine_two_chunks_per_wave(monkeypatch, kernel, M, bits, K):
    # rows longer than 8 KiB: each wave streams two chunks of every row
    setknob(monkeypatch, "MLXQ_QMV_KERNEL", kernel)
    announce("rs_two_chunks", kernel, M, bits, K)
    x, wq, s, b = affine_case(M, 136, K, 64, bits, 950 + M + bits)
    assert max_rel(affine(x, wq, s, b, 64, bits), orc.qmm_t_affine(x, wq, s, b, 64, bits)) <= TOL


@pytest.mark.parametrize("kernel,R", KERNEL_R)
@pytest.mark.parametrize("M", [1, 2, 4])
def test_mxfp4_kernels(monkeypatch, kernel, R, M):
    setknob(monkeypatch, "MLXQ_QMV_KERNEL", kernel)
    setknob(monkeypatch, "MLXQ_QMV_R", str(R))
    announce("rs_mxfp4", kernel, R, M)
    x, wq, sc = mxfp4_case(M, 5760 + 8, 2880, 980 + M + R)
    assert max_rel(mxfp4(x, wq, sc), orc.fp_qmm_t_mxfp4(x, wq, sc)) <= TOL


@pytest.mark.parametrize("M", [1, 2, 3, 4])
def test_mxfp4_one_hot_is_exact_skinny(M):
    # one-hot activations pick single dequantized weights: LUT * 2^(s-127) is
    # exact, so every decode kernel must return the dequantize bits
    announce("skinny_mxfp4_one_hot", M)
    N, K = 40, 2880
    _, wq, sc = mxfp4_case(1, N, K, 23)
    ks = np.array([0, 31, 1439, 2879])[:M]
    x = np.zeros((M, K), np.uint16)
    x[np.arange(M), ks] = 0x3F80
    np.testing.assert_array_equal(mxfp4(x, wq, sc), orc.mxfp4_dequantize(wq, sc)[:, ks].T)


@pytest.mark.parametrize("M", [1, 2, 3])
def test_skinny_deterministic_and_matches_batched_layout(M):
    announce("skinny_determinism", M)
    N, K = 4096, 14336
    x, wq, s, b = affine_case(M, N, K, 64, 4, 991)
    W, S, Bi, xd = dev_u32(wq), dev_bf16(s), dev_bf16(b), dev_bf16(x)
    y1 = host_u16(mq.quantized_matmul(xd, W, S, Bi))
    y2 = host_u16(mq.quantized_matmul(xd, W, S, Bi))
    np.testing.assert_array_equal(y1, y2)
    # the same rows as a (1, M, K) batch give the same bits
    y3 = host_u16(mq.quantized_matmul(xd.reshape(1, M, K), W, S, Bi)).reshape(M, N)
    np.testing.assert_array_equal(y1, y3)
    assert max_rel(y1, orc.qmm_t_affine(x, wq, s, b, 64, 4)) <= TOL


def test_gather_segments_of_two_rows():
    # gather with 2 rows per gathered matrix (x.shape[-2] == 2), experts repeated
    announce("skinny_gather_m2")
    E, N, K, M = 6, 264, 2048, 2
    x = orc.normal_bf16((5, M, K), 1.0, 993)
    w = orc.normal_bf16((E, N, K), 0.02, 994)
    wq, s, b = orc.affine_quantize(w, 64, 4)
    lhs = np.array([4, 0, 2, 2, 1, 3, 0], np.uint32)
    rhs = np.array([5, 5, 0, 3, 1, 2, 4], np.uint32)
    got = host_u16(mq.gather_qmm(dev_bf16(x), dev_u32(wq), dev_bf16(s), dev_bf16(b),
                                 torch.from_numpy(lhs).cuda(), torch.from_numpy(rhs).cuda(), True, 64, 4))
    for i in range(len(lhs)):
        want = orc.qmm_t_affine(x[lhs[i]], wq[rhs[i]], s[rhs[i]], b[rhs[i]], 64, 4)
        assert max_rel(got[i], want) <= TOL
