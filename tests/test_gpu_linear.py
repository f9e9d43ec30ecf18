"""GPU checks of mlxq_quantized_linear (the reference's quantized_linear_forward,
src/lib/mlxcel-core/cpp/mlx_cxx_bridge.cpp:1707-1746): bit for bit
quantized_matmul followed by MLX's bf16 `add` of the linear bias (torch's
bf16 add computes the same fp32 sum and rounds once), for a (N) bias, a
(1, N) bias and a full-shape bias, at decode and prefill row counts, affine
and mxfp4 (gpt-oss carries linear biases on every projection), plus the
oracle bound on the sum.
"""
import numpy as np
import pytest
import torch

import mlxcel_amd as mq
import oracle as orc
from helpers import TOL, announce, dev_bf16, dev_u32, dev_u8, host_u16, max_rel

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M", [1, 3, 20])
@pytest.mark.parametrize("bias_shape", ["n", "1n", "full"])
@pytest.mark.parametrize("N", [328, 333])  # 16-byte bias rows, and an odd width (element path)
def test_affine_linear_is_matmul_then_add(M, bias_shape, N):
    announce("linear_affine", M, bias_shape, N)
    K = 1024
    x, wq, s, b = orc.normal_bf16((M, K), 1.0, 1100 + M), *orc.affine_quantize(orc.normal_bf16((N, K), 0.02, 1101), 64, 4)
    shape = {"n": (N,), "1n": (1, N), "full": (M, N)}[bias_shape]
    lb = orc.normal_bf16(shape, 0.5, 1102)
    X, W, S, B, LB = dev_bf16(x), dev_u32(wq), dev_bf16(s), dev_bf16(b), dev_bf16(lb)
    got = host_u16(mq.quantized_linear(X, W, S, B, LB, 64, 4))
    want = host_u16(mq.quantized_matmul(X, W, S, B, True, 64, 4) + LB)
    np.testing.assert_array_equal(got, want)
    ref = orc.f32_to_bf16(orc.bf16_to_f32(orc.qmm_t_affine(x, wq, s, b, 64, 4)) + orc.bf16_to_f32(lb))
    assert max_rel(got, ref) <= TOL


def test_mxfp4_linear_and_no_bias():
    announce("linear_mxfp4")
    N, K = 512, 2880
    x = orc.normal_bf16((1, K), 1.0, 1110)
    wq, sc = orc.mxfp4_quantize(orc.normal_bf16((N, K), 0.02, 1111))
    lb = orc.normal_bf16((N,), 0.5, 1112)
    X, W, S, LB = dev_bf16(x), dev_u32(wq), dev_u8(sc), dev_bf16(lb)
    got = host_u16(mq.quantized_linear(X, W, S, None, LB, 32, 4, "mxfp4"))
    np.testing.assert_array_equal(got, host_u16(mq.quantized_matmul(X, W, S, None, True, 32, 4, "mxfp4") + LB))
    plain = host_u16(mq.quantized_linear(X, W, S, None, None, 32, 4, "mxfp4"))
    np.testing.assert_array_equal(plain, host_u16(mq.quantized_matmul(X, W, S, None, True, 32, 4, "mxfp4")))
    assert not mq.quantized_matmul_matches_dense_gemm(X, W, S, None, 32, 4)
