"""GPU parity of decode quantized_matmul at LM-head vocabulary widths, after the
reference's tests/cuda_qmv_reference_parity.rs (issue 2958: the last rows of
Gemma 4's N = 262144 head):

* N = 262144 (Gemma 4), 262147 (a ragged tail: not a multiple of any row
  tile) and 151936 (Qwen3), K = 512 (no partial chunk) and 576 (a partial
  1 KiB chunk), M = 1 as [1, K] and [1, 1, K] (byte-identical);
* the Qwen3-8B head itself (N = 151936, K = 4096);
* every decode kernel forced in turn at the ragged width;
* the full output within max|y - y_ref| / max|y_ref| <= 1e-2 of the oracle,
  the final 64 rows checked on their own (including row N - 1), all finite.
"""
import functools

import numpy as np
import pytest

import mlxcel_amd as mq
import oracle as orc
from helpers import TOL, announce, dev_bf16, dev_u32, host_u16, max_rel, setknob

pytestmark = pytest.mark.gpu

TAIL = 64


@functools.lru_cache(maxsize=4)
def head_case(N, K, bits=4, gs=64):
    """Random codes with scales ~ N(0, 0.002) and biases ~ N(0, 0.01) (what
    quantizing N(0, 0.02) weights gives, without quantizing 10^9 values)."""
    seed = 0x2958 ^ N ^ (K << 20)
    x = orc.normal_bf16((1, K), 1.0, seed)
    rng = np.random.Generator(np.random.Philox(seed + 1))
    wq = rng.integers(0, 1 << 32, size=(N, K * bits // 32), dtype=np.uint32)
    s = orc.normal_bf16((N, K // gs), 0.002, seed + 2)
    b = orc.normal_bf16((N, K // gs), 0.01, seed + 3)
    want = orc.qmm_t_affine(x, wq, s, b, gs, bits)
    return x, wq, s, b, want


def check(got, want, name):
    assert np.isfinite(orc.bf16_to_f32(got)).all(), f"{name}: non-finite output"
    err = max_rel(got, want)
    assert err <= TOL, f"{name}: all rows {err}"
    # the tail on its own, against the full output's scale
    scale = np.abs(orc.bf16_to_f32(want)).max()
    tail = np.abs(orc.bf16_to_f32(got[..., -TAIL:]).astype(np.float64) -
                  orc.bf16_to_f32(want[..., -TAIL:])).max() / scale
    assert tail <= TOL, f"{name}: tail rows {tail}"


@pytest.mark.parametrize("N", [262144, 262147, 151936])
@pytest.mark.parametrize("K", [512, 576])
def test_vocab_widths(N, K):
    announce("lm_head", N, K)
    x, wq, s, b, want = head_case(N, K)
    W, S, B = dev_u32(wq), dev_bf16(s), dev_bf16(b)
    xd = dev_bf16(x)
    got2 = host_u16(mq.quantized_matmul(xd, W, S, B, True, 64, 4))
    got3 = host_u16(mq.quantized_matmul(xd.view(1, 1, K), W, S, B, True, 64, 4))
    np.testing.assert_array_equal(got3.reshape(got2.shape), got2)
    check(got2, want, f"N={N} K={K}")


def test_qwen3_8b_head():
    announce("lm_head_qwen3_8b")
    x, wq, s, b, want = head_case(151936, 4096)
    got = host_u16(mq.quantized_matmul(dev_bf16(x), dev_u32(wq), dev_bf16(s), dev_bf16(b), True, 64, 4))
    check(got, want, "qwen3-8b head")


@pytest.mark.parametrize("kernel", ["rs", "fr", "b4", "mfma", "mid"])
def test_every_decode_kernel_at_a_ragged_width(monkeypatch, kernel):
    setknob(monkeypatch, "MLXQ_QMV_KERNEL", kernel)
    announce("lm_head_kernel", kernel)
    x, wq, s, b, want = head_case(262147, 576)
    got = host_u16(mq.quantized_matmul(dev_bf16(x), dev_u32(wq), dev_bf16(s), dev_bf16(b), True, 64, 4))
    check(got, want, f"{kernel} N=262147 K=576")
