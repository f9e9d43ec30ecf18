"""GPU parity of the mid-size decode kernel (qmv_mid.hip; 1-16 activation rows
against one affine 4/8-bit weight matrix, forced with MLXQ_QMV_KERNEL=mid)
against the oracle's restatement of MLX's `_qmm_t` (overlays/cpu/mlx/backend/
cpu/quantized.cpp:199-257), max|y - y_ref| / max|y_ref| <= 1e-2.

Shapes reach every compiled variant: group slots per window S in {1, 2, 4}
(4-bit g128/g64/g32, 8-bit g64/g32, and 8-bit g128, where one group spans two
windows and the scales stage two groups per load), 1 and 2 activation A
tiles (4-bit g32 above 8 rows would need 4 and runs another kernel), a
partial last row block (N not a multiple of 128), a single K range
(direct bf16 store) and several (fp32 partials added by the reduction
kernel), back-to-back calls and graph replays.
"""
import numpy as np
import pytest
import torch

import mlxcel_amd as mq
import oracle as orc
from helpers import TOL, affine_case, announce, dev_bf16, dev_u32, host_u16, max_rel, setknob

pytestmark = pytest.mark.gpu


@pytest.fixture
def mid(monkeypatch):
    setknob(monkeypatch, "MLXQ_QMV_KERNEL", "mid")


def run(x, wq, s, b, gs, bits):
    y = mq.quantized_matmul(dev_bf16(x), dev_u32(wq), dev_bf16(s), dev_bf16(b), True, gs, bits)
    torch.cuda.synchronize()
    return host_u16(y)


@pytest.mark.parametrize("bits,gs", [(4, 32), (4, 64), (4, 128), (8, 32), (8, 64), (8, 128)])
@pytest.mark.parametrize("M", [1, 3, 5, 8, 9, 12, 16])
def test_mid_affine_every_variant(mid, bits, gs, M):
    # N = 200: the second row block is partial; K = 2048: two K ranges of
    # 1024 (4-bit) or four of 512 (8-bit)
    N, K = 200, 2048
    announce("mid_affine", bits, gs, M)
    x, wq, s, b = affine_case(M, N, K, gs, bits, 2000 + M + bits + gs)
    assert max_rel(run(x, wq, s, b, gs, bits), orc.qmm_t_affine(x, wq, s, b, gs, bits)) <= TOL


@pytest.mark.parametrize("bits,K", [(4, 1024), (4, 3072), (8, 512), (8, 1536)])
@pytest.mark.parametrize("M", [6, 16])
def test_mid_k_ranges(mid, bits, K, M):
    # one K range (direct bf16 store) and three (reduction kernel)
    N = 264
    announce("mid_k_ranges", bits, K, M)
    x, wq, s, b = affine_case(M, N, K, 64, bits, 2100 + M + K + bits)
    assert max_rel(run(x, wq, s, b, 64, bits), orc.qmm_t_affine(x, wq, s, b, 64, bits)) <= TOL


@pytest.mark.parametrize("M", [5, 16])
def test_mid_8bit_g128_two_group_scale_loads(mid, M):
    # 8-bit g128: a 512-wide K range holds 4 groups, staged 2 per load
    announce("mid_8bit_g128", M)
    x, wq, s, b = affine_case(M, 136, 1536, 128, 8, 2250 + M)
    assert max_rel(run(x, wq, s, b, 128, 8), orc.qmm_t_affine(x, wq, s, b, 128, 8)) <= TOL


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M", [8, 16])
@pytest.mark.parametrize("N,K", [(14336, 4096), (4096, 14336)])
def test_mid_llama_shapes(mid, bits, M, N, K):
    announce("mid_llama", bits, M, N, K)
    x, wq, s, b = affine_case(M, N, K, 64, bits, 2300 + M + N + bits)
    assert max_rel(run(x, wq, s, b, 64, bits), orc.qmm_t_affine(x, wq, s, b, 64, bits)) <= TOL


def test_mid_back_to_back_calls_and_determinism(mid):
    # the split-K workspace is reused call after call
    announce("mid_back_to_back")
    M, N, K = 12, 520, 2048
    _, wq, s, b = affine_case(1, N, K, 64, 4, 2400)
    W, S, Bi = dev_u32(wq), dev_bf16(s), dev_bf16(b)
    first = None
    for i in range(4):
        x = orc.normal_bf16((M, K), 1.0, 2401 + i % 2)
        got = host_u16(mq.quantized_matmul(dev_bf16(x), W, S, Bi))
        assert max_rel(got, orc.qmm_t_affine(x, wq, s, b, 64, 4)) <= TOL
        if i == 0:
            first = got
        if i == 2:
            np.testing.assert_array_equal(got, first)


def test_mid_graph_replays(mid):
    announce("mid_graph_replays")
    M, N, K = 16, 392, 2048
    _, wq, s, b = affine_case(1, N, K, 64, 4, 2500)
    W, S, Bi = dev_u32(wq), dev_bf16(s), dev_bf16(b)
    xs = [orc.normal_bf16((M, K), 1.0, 2501 + i) for i in range(3)]
    xd = dev_bf16(xs[0])
    out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        mq.quantized_matmul(xd, W, S, Bi, out=out)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        mq.quantized_matmul(xd, W, S, Bi, out=out)
    torch.cuda.synchronize()
    for i in (0, 1, 2, 1):
        xd.copy_(dev_bf16(xs[i]))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        eager = host_u16(mq.quantized_matmul(xd, W, S, Bi))
        got = host_u16(out)
        np.testing.assert_array_equal(got, eager)
        assert max_rel(got, orc.qmm_t_affine(xs[i], wq, s, b, 64, 4)) <= TOL


def test_mid_unsupported_shapes_fall_back(mid):
    # K = 2880 is not a multiple of the 1024-wide K range: another kernel runs
    announce("mid_fallback")
    x, wq, s, b = affine_case(8, 96, 2880, 64, 4, 2600)
    assert max_rel(run(x, wq, s, b, 64, 4), orc.qmm_t_affine(x, wq, s, b, 64, 4)) <= TOL


@pytest.mark.parametrize("bits,gs", [(4, 32), (4, 64), (4, 128), (8, 64), (8, 128)])
@pytest.mark.parametrize("M", [5, 16])
def test_mid_half_k_range(mid, monkeypatch, bits, gs, M):
    # MLXQ_QMV_MID_WIN=4: K ranges of 4 windows (512 k for 4-bit, 256 for
    # 8-bit; 8-bit g128 then has one group per two ranges' worth of windows
    # staged two at a time), against the oracle, and a q/k/v launch bitwise
    # equal to its single calls at the same setting
    setknob(monkeypatch, "MLXQ_QMV_MID_WIN", "4")
    announce("mid_half_k", bits, gs, M)
    K = 2048
    x, wq, s, b = affine_case(M, 200, K, gs, bits, 2700 + M + bits + gs)
    assert max_rel(run(x, wq, s, b, gs, bits), orc.qmm_t_affine(x, wq, s, b, gs, bits)) <= TOL
    setknob(monkeypatch, "MLXQ_QMV_KERNEL", "")
    sets = [orc.affine_quantize(orc.normal_bf16((n, K), 0.02, 2710 + n), gs, bits) for n in (512, 128, 128)]
    xd = dev_bf16(x)
    dev = [(dev_u32(w), dev_bf16(sc), dev_bf16(bi)) for w, sc, bi in sets]
    multi = mq.quantized_matmul_multi(xd, [d[0] for d in dev], [d[1] for d in dev], [d[2] for d in dev], gs, bits)
    for m, d in zip(multi, dev):
        np.testing.assert_array_equal(host_u16(m), host_u16(mq.quantized_matmul(xd, *d, True, gs, bits)))
