"""GPU parity of the block-MFMA decode kernel (qmv_b4.hip, default for 3 to 16
activation rows per weight matrix; forced with MLXQ_QMV_KERNEL=b4 and shaped
with MLXQ_QMV_B4_RG / MLXQ_QMV_B4_CPW) against the oracle's restatement of
MLX's `_qmm_t` / `fp_qmm_t` (overlays/cpu/mlx/backend/cpu/quantized.cpp:
199-257, 550-597), max|y - y_ref| / max|y_ref| <= 1e-2.

Shapes reach every compiled variant: 1-4 / 5-8 / 9-16 activation rows
(1, 2 and 4 sets of four), every (row groups, chunks per wave) pair, rows
that end inside a 16-piece chunk, N not a multiple of the row tile, and the
mxfp4 path with its special e8m0 scales (2^-127 and NaN).
"""
import numpy as np
import pytest
import torch

import mlxcel_amd as mq
import oracle as orc
from helpers import TOL, affine_case, announce, dev_bf16, dev_u32, dev_u8, host_u16, max_rel, mxfp4_case, setknob

pytestmark = pytest.mark.gpu

SHAPES = [(1, 1), (2, 1), (4, 1), (8, 1), (1, 2), (2, 2), (4, 2), (1, 4), (2, 4), (1, 8)]  # (row groups, chunks/wave)


def affine(x, wq, s, b, gs, bits):
    y = mq.quantized_matmul(dev_bf16(x), dev_u32(wq), dev_bf16(s), dev_bf16(b), True, gs, bits)
    torch.cuda.synchronize()
    return host_u16(y)


def mxfp4(x, wq, sc):
    y = mq.quantized_matmul(dev_bf16(x), dev_u32(wq), dev_u8(sc), None, True, 32, 4, "mxfp4")
    torch.cuda.synchronize()
    return host_u16(y)


@pytest.fixture
def b4(monkeypatch):
    setknob(monkeypatch, "MLXQ_QMV_KERNEL", "b4")

    def shape(rg, cpw):
        setknob(monkeypatch, "MLXQ_QMV_B4_RG", str(rg))
        setknob(monkeypatch, "MLXQ_QMV_B4_CPW", str(cpw))
    return shape


@pytest.mark.parametrize("bits,gs", [(4, 32), (4, 64), (4, 128), (8, 32), (8, 64), (8, 128)])
@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8, 9, 16])
def test_b4_affine_default_shape(b4, bits, gs, M):
    # N = 202: the last row group is partial; K = 2304: the last chunk of a
    # row holds only some pieces
    N, K = 202, 2304
    announce("b4_affine", bits, gs, M)
    x, wq, s, b = affine_case(M, N, K, gs, bits, 1300 + M + bits + gs)
    assert max_rel(affine(x, wq, s, b, gs, bits), orc.qmm_t_affine(x, wq, s, b, gs, bits)) <= TOL


@pytest.mark.parametrize("rg,cpw", SHAPES)
@pytest.mark.parametrize("M", [1, 6, 13])
@pytest.mark.parametrize("bits", [4, 8])
def test_b4_affine_every_variant(b4, rg, cpw, M, bits):
    # 7.5 chunks of 16 pieces per row: every chunks-per-wave value fits in
    # the 8 waves of a workgroup, and the last chunk is partial
    b4(rg, cpw)
    N, K = 76, (3840 if bits == 4 else 1920)
    announce("b4_variant", rg, cpw, M, bits)
    x, wq, s, b = affine_case(M, N, K, 64, bits, 1400 + rg * 10 + cpw + M + bits)
    assert max_rel(affine(x, wq, s, b, 64, bits), orc.qmm_t_affine(x, wq, s, b, 64, bits)) <= TOL


@pytest.mark.parametrize("M", [1, 4, 8, 16])
@pytest.mark.parametrize("N,K", [(14336, 4096), (4096, 14336)])
def test_b4_llama_shapes(b4, M, N, K):
    announce("b4_llama", M, N, K)
    x, wq, s, b = affine_case(M, N, K, 64, 4, 1500 + M + N)
    assert max_rel(affine(x, wq, s, b, 64, 4), orc.qmm_t_affine(x, wq, s, b, 64, 4)) <= TOL


@pytest.mark.parametrize("M", [1, 3, 8, 16])
def test_b4_mxfp4(b4, M):
    # gpt-oss shapes: K = 2880 is 90 pieces, so the sixth chunk is partial
    announce("b4_mxfp4", M)
    x, wq, sc = mxfp4_case(M, 5760 + 12, 2880, 1600 + M)
    assert max_rel(mxfp4(x, wq, sc), orc.fp_qmm_t_mxfp4(x, wq, sc)) <= TOL


@pytest.mark.parametrize("M", [1, 5, 16])
def test_b4_mxfp4_one_hot_is_exact_with_special_scales(b4, M):
    # one-hot activations pick single dequantized weights: LUT * 2^(s-127)
    # is exact, so the kernel must return the dequantize bits, including the
    # 2^-127 (e8m0 0) groups; a NaN (e8m0 255) group makes its whole column
    # NaN, since 0 * NaN is NaN in the reference's sum as well
    announce("b4_mxfp4_one_hot", M)
    N, K = 40, 2880
    _, wq, sc = mxfp4_case(1, N, K, 31)
    sc = sc.copy()
    sc[3, 0] = 0      # column 3, k 0..31: 2^-127
    sc[5, 44] = 0     # column 5, k 1408..1439
    sc[7, 89] = 255   # column 7, k 2848..2879: NaN
    ks = np.array([0, 31, 1439, 2879, 5, 1408, 2848, 17, 100, 640, 1000, 1500, 2000, 2500, 2600, 2870])[:M]
    x = np.zeros((M, K), np.uint16)
    x[np.arange(M), ks] = 0x3F80
    got = mxfp4(x, wq, sc)
    want = orc.mxfp4_dequantize(wq, sc)[:, ks].T
    nan_cols = np.zeros((M, N), bool)
    nan_cols[:, 7] = True
    nan_ref = np.isnan(orc.bf16_to_f32(orc.fp_qmm_t_mxfp4(x, wq, sc)))
    np.testing.assert_array_equal(nan_ref, nan_cols)  # the oracle agrees
    np.testing.assert_array_equal(np.isnan(orc.bf16_to_f32(got)), nan_cols)
    np.testing.assert_array_equal(got[:, :7], want[:, :7])
    np.testing.assert_array_equal(got[:, 8:], want[:, 8:])


@pytest.mark.parametrize("M", [3, 8, 16])
def test_b4_deterministic_and_matches_batched_layout(b4, M):
    announce("b4_determinism", M)
    N, K = 4096, 14336
    x, wq, s, b = affine_case(M, N, K, 64, 4, 1700 + M)
    W, S, Bi, xd = dev_u32(wq), dev_bf16(s), dev_bf16(b), dev_bf16(x)
    y1 = host_u16(mq.quantized_matmul(xd, W, S, Bi))
    y2 = host_u16(mq.quantized_matmul(xd, W, S, Bi))
    np.testing.assert_array_equal(y1, y2)
    y3 = host_u16(mq.quantized_matmul(xd.reshape(1, M, K), W, S, Bi)).reshape(M, N)
    np.testing.assert_array_equal(y1, y3)


@pytest.mark.parametrize("M", [5, 16])
def test_b4_gather_segments(M):
    # default dispatch (b4 for 3-16 rows): gather with M rows per gathered
    # matrix, experts repeated, lhs reused
    announce("b4_gather", M)
    E, N, K = 6, 264, 2048
    x = orc.normal_bf16((5, M, K), 1.0, 1800 + M)
    w = orc.normal_bf16((E, N, K), 0.02, 1801 + M)
    wq, s, b = orc.affine_quantize(w, 64, 4)
    lhs = np.array([4, 0, 2, 2, 1, 3, 0], np.uint32)
    rhs = np.array([5, 5, 0, 3, 1, 2, 4], np.uint32)
    got = host_u16(mq.gather_qmm(dev_bf16(x), dev_u32(wq), dev_bf16(s), dev_bf16(b),
                                 torch.from_numpy(lhs).cuda(), torch.from_numpy(rhs).cuda(), True, 64, 4))
    for i in range(len(lhs)):
        want = orc.qmm_t_affine(x[lhs[i]], wq[rhs[i]], s[rhs[i]], b[rhs[i]], 64, 4)
        assert max_rel(got[i], want) <= TOL
