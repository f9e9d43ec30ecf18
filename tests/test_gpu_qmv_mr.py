"""GPU parity of the whole-row mid-size decode kernel (qmv_mr.hip; 1-16
activation rows against one affine 4/8-bit weight matrix, forced with
MLXQ_QMV_KERNEL=mr, which also lifts its rows-per-CU condition) against the
oracle's restatement of MLX's `_qmm_t` (overlays/cpu/mlx/backend/cpu/
quantized.cpp:199-257), max|y - y_ref| / max|y_ref| <= 1e-2.

Shapes reach every compiled variant: group slots per window S in {1, 2, 4},
1 and 2 activation A tiles, 8 and 16 staged activation rows, one staged K
range and several (both LDS buffers, the last range's dead prefetch), a
partial last row block, graph replays, and fall-backs where a shape is not
covered.
"""
import numpy as np
import pytest
import torch

import mlxcel_amd as mq
import oracle as orc
from helpers import TOL, affine_case, announce, dev_bf16, dev_u32, host_u16, max_rel, setknob

pytestmark = pytest.mark.gpu


@pytest.fixture
def mr(monkeypatch):
    setknob(monkeypatch, "MLXQ_QMV_KERNEL", "mr")


def run(x, wq, s, b, gs, bits):
    y = mq.quantized_matmul(dev_bf16(x), dev_u32(wq), dev_bf16(s), dev_bf16(b), True, gs, bits)
    torch.cuda.synchronize()
    return host_u16(y)


@pytest.mark.parametrize("bits,gs", [(4, 32), (4, 64), (4, 128), (8, 32), (8, 64), (8, 128)])
@pytest.mark.parametrize("M", [1, 3, 5, 8, 9, 12, 16])
def test_mr_affine_every_variant(mr, bits, gs, M):
    # N = 200: the last row block is partial; K = 3072: three ranges of 1024
    # (4-bit: the last loop turn's second range multiplies zeros) or six of
    # 512 (8-bit)
    N, K = 200, 3072
    announce("mr_affine", bits, gs, M)
    x, wq, s, b = affine_case(M, N, K, gs, bits, 3300 + M + bits + gs)
    assert max_rel(run(x, wq, s, b, gs, bits), orc.qmm_t_affine(x, wq, s, b, gs, bits)) <= TOL


@pytest.mark.parametrize("ring", ["4", "16"])
@pytest.mark.parametrize("bits,gs", [(4, 32), (4, 64), (8, 64), (8, 128)])
@pytest.mark.parametrize("M", [2, 8, 12])
def test_mr_weight_ring_depths(mr, monkeypatch, ring, bits, gs, M):
    # the other ring depths (MLXQ_MR_RING; the default of 8 windows runs in
    # every other test): refills cross into the next staged range at 4
    # windows, and reach two ranges ahead at 16
    setknob(monkeypatch, "MLXQ_MR_RING", ring)
    N, K = 200, 3072
    announce("mr_ring", ring, bits, gs, M)
    x, wq, s, b = affine_case(M, N, K, gs, bits, 3900 + M + bits + gs)
    assert max_rel(run(x, wq, s, b, gs, bits), orc.qmm_t_affine(x, wq, s, b, gs, bits)) <= TOL


@pytest.mark.parametrize("bits,K", [(4, 1024), (4, 2048), (4, 5120), (8, 512), (8, 1024)])
@pytest.mark.parametrize("M", [6, 16])
def test_mr_range_counts(mr, bits, K, M):
    # one, two and five staged ranges
    N = 264
    announce("mr_ranges", bits, K, M)
    x, wq, s, b = affine_case(M, N, K, 64, bits, 3400 + M + K + bits)
    assert max_rel(run(x, wq, s, b, 64, bits), orc.qmm_t_affine(x, wq, s, b, 64, bits)) <= TOL


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M", [3, 4, 5, 8, 16])
def test_mr_llama_gate_shape(bits, M):
    # the Llama-3-8B gate/up shape (14336 rows: 224 workgroups) on the
    # default route, which takes this kernel at 3-8 rows (4-bit) and 5-16
    # rows (8-bit)
    N, K = 14336, 4096
    announce("mr_llama", bits, M)
    x, wq, s, b = affine_case(M, N, K, 64, bits, 3500 + M + bits)
    assert max_rel(run(x, wq, s, b, 64, bits), orc.qmm_t_affine(x, wq, s, b, 64, bits)) <= TOL


def test_mr_matches_split_k_kernel_and_repeats(monkeypatch):
    announce("mr_vs_mid")
    M, N, K = 8, 1000, 4096
    x, wq, s, b = affine_case(M, N, K, 64, 4, 3600)
    setknob(monkeypatch, "MLXQ_QMV_KERNEL", "mr")
    a1 = run(x, wq, s, b, 64, 4)
    a2 = run(x, wq, s, b, 64, 4)
    np.testing.assert_array_equal(a1, a2)
    setknob(monkeypatch, "MLXQ_QMV_KERNEL", "mid")
    assert max_rel(a1, run(x, wq, s, b, 64, 4)) <= TOL


def test_mr_graph_replays(mr):
    announce("mr_graph_replays")
    M, N, K = 12, 392, 4096
    _, wq, s, b = affine_case(1, N, K, 64, 4, 3700)
    W, S, Bi = dev_u32(wq), dev_bf16(s), dev_bf16(b)
    xs = [orc.normal_bf16((M, K), 1.0, 3701 + i) for i in range(3)]
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


@pytest.mark.parametrize("M,K,gs,bits", [(8, 2880, 64, 4), (12, 1536, 64, 4), (16, 4096, 32, 4)])
def test_mr_uncovered_shapes_fall_back(mr, M, K, gs, bits):
    # K not a multiple of the 1024-wide range; 16 rows x 4 group slots need
    # more than two A tiles: another kernel runs
    announce("mr_fallback", M, K, gs, bits)
    x, wq, s, b = affine_case(M, 96, K, gs, bits, 3800 + M)
    assert max_rel(run(x, wq, s, b, gs, bits), orc.qmm_t_affine(x, wq, s, b, gs, bits)) <= TOL
