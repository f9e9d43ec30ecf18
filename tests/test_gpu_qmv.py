"""GPU parity: quantized_matmul (decode / skinny M) on gfx950 vs the CPU oracle.

Rule (north star): max|y - y_ref| / max|y_ref| <= 1e-2 against the oracle's
restatement of MLX's `_qmm_t` / `fp_qmm_t` (overlays/cpu/mlx/backend/cpu/
quantized.cpp:199-257, 550-597) on the same seeded inputs.  Run-to-run and
row-layout invariance are bitwise (tests/rocm_qmm_batched_rows.rs:26-31,
tests/rocm_gather_qmm_expert_batched.rs:46 in the reference).
"""
import numpy as np
import pytest
import torch

import mlxcel_amd as mq
import oracle as orc
from helpers import TOL, affine_case, announce, dev_bf16, dev_u32, dev_u8, host_u16, max_rel, mxfp4_case

pytestmark = pytest.mark.gpu


def run_affine(x, wq, s, b, gs, bits):
    y = mq.quantized_matmul(dev_bf16(x), dev_u32(wq), dev_bf16(s), dev_bf16(b), True, gs, bits)
    torch.cuda.synchronize()
    return host_u16(y)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("M", [1, 2, 3, 5, 8])
def test_affine_small_shapes(bits, gs, M):
    N, K = 200, 640  # ragged N (not a multiple of 16), K with a partial 128-step
    announce("affine_small", bits, gs, M)
    x, wq, s, b = affine_case(M, N, K, gs, bits, 100 + M + bits + gs)
    got = run_affine(x, wq, s, b, gs, bits)
    want = orc.qmm_t_affine(x, wq, s, b, gs, bits)
    assert got.shape == want.shape
    assert max_rel(got, want) <= TOL


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("N,K", [(4096, 4096), (14336, 4096), (4096, 14336)])
@pytest.mark.parametrize("M", [1, 2, 4, 8])
def test_affine_llama_shapes(bits, N, K, M):
    announce("affine_llama", bits, N, K, M)
    x, wq, s, b = affine_case(M, N, K, 64, bits, 7000 + N + K + M + bits)
    got = run_affine(x, wq, s, b, 64, bits)
    want = orc.qmm_t_affine(x, wq, s, b, 64, bits)
    assert max_rel(got, want) <= TOL


def test_affine_deterministic_and_row_layout_invariant():
    announce("determinism")
    B, N, K = 4, 4096, 14336  # split-K path
    x, wq, s, b = affine_case(B, N, K, 64, 4, 55)
    W, S, Bi = dev_u32(wq), dev_bf16(s), dev_bf16(b)
    xd = dev_bf16(x)
    y1 = host_u16(mq.quantized_matmul(xd, W, S, Bi))
    y2 = host_u16(mq.quantized_matmul(xd, W, S, Bi))
    np.testing.assert_array_equal(y1, y2)
    y3 = host_u16(mq.quantized_matmul(xd.reshape(B, 1, K), W, S, Bi)).reshape(B, N)
    y4 = host_u16(mq.quantized_matmul(xd.reshape(1, B, K), W, S, Bi)).reshape(B, N)
    np.testing.assert_array_equal(y1, y3)
    np.testing.assert_array_equal(y1, y4)
    assert max_rel(y1, orc.qmm_t_affine(x, wq, s, b, 64, 4)) <= TOL


def test_affine_batched_weights():
    announce("batched_w")
    E, M, N, K = 3, 2, 96, 512
    x = orc.normal_bf16((E, M, K), 1.0, 61)
    w = orc.normal_bf16((E, N, K), 0.02, 62)
    wq, s, b = orc.affine_quantize(w, 64, 4)
    got = host_u16(mq.quantized_matmul(dev_bf16(x), dev_u32(wq), dev_bf16(s), dev_bf16(b)))
    for e in range(E):
        assert max_rel(got[e], orc.qmm_t_affine(x[e], wq[e], s[e], b[e], 64, 4)) <= TOL


def test_affine_many_rows_fall_back_to_segments():
    # more rows than one skinny tile holds: computed as several row segments
    announce("rows_40")
    x, wq, s, b = affine_case(40, 128, 512, 64, 4, 77)
    got = run_affine(x, wq, s, b, 64, 4)
    assert max_rel(got, orc.qmm_t_affine(x, wq, s, b, 64, 4)) <= TOL


@pytest.mark.parametrize("M", [1, 3, 4, 8])
@pytest.mark.parametrize("N,K", [(96, 2880), (5760, 2880), (2880, 2880)])
def test_mxfp4(M, N, K):
    announce("mxfp4", M, N, K)
    x, wq, sc = mxfp4_case(M, N, K, 300 + M + N)
    got = host_u16(mq.quantized_matmul(dev_bf16(x), dev_u32(wq), dev_u8(sc), None, True, 32, 4, "mxfp4"))
    want = orc.fp_qmm_t_mxfp4(x, wq, sc)
    assert max_rel(got, want) <= TOL


def test_mxfp4_one_hot_is_exact():
    # x = e_k picks one dequantized weight per output: LUT * 2^(s-127) is
    # exact in bf16, so the GPU must reproduce the oracle's dequantize bits
    announce("mxfp4_one_hot")
    N, K = 48, 2880
    _, wq, sc = mxfp4_case(1, N, K, 17)
    ks = np.arange(16) * 173
    x = np.zeros((16, K), np.uint16)
    x[np.arange(16), ks] = 0x3F80
    got = host_u16(mq.quantized_matmul(dev_bf16(x), dev_u32(wq), dev_u8(sc), None, True, 32, 4, "mxfp4"))
    np.testing.assert_array_equal(got, orc.mxfp4_dequantize(wq, sc)[:, ks].T)


def test_unimplemented_raises():
    x, wq, s, b = affine_case(1, 64, 64, 64, 4, 3)
    with pytest.raises(NotImplementedError):
        mq.quantized_matmul(dev_bf16(x).double(), dev_u32(wq), dev_bf16(s).double(), dev_bf16(b).double())
    with pytest.raises(ValueError, match="Biases must be provided"):
        mq.quantized_matmul(dev_bf16(x), dev_u32(wq), dev_bf16(s), None)
