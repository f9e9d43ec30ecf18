"""GPU parity of the K-split-over-waves decode kernel (qmv_kq_kernel in
qmv_mr.hip: 1-16 activation rows against one affine 4/8-bit weight matrix
of few rows; a workgroup owns 16-64 weight rows over the whole of K and
its eight waves split every staged range's windows) against the oracle's
restatement of MLX's `_qmm_t` (overlays/cpu/mlx/backend/cpu/quantized.cpp:
199-257), max|y - y_ref| / max|y_ref| <= 1e-2.

Forced with MLXQ_QMV_KERNEL=kq (MLXQ_QMV_KQ_T=1|2|3|4 sets the 16-row
tiles per workgroup); the default route takes it at 5-16 rows for matrices
whose blocks of up to 64 rows fit one round of the CUs (past 8 rows over
at most 12 staged ranges; 3-4 rows with 4-bit codes).  Shapes reach every
compiled variant:
group slots per window S in {1, 2, 4}, 1 and 2 A tiles, 8 and 16 staged
activation rows, 1 and 2 tiles per workgroup, one, two and an odd number of
staged K ranges (the last loop turn multiplies zeros), a partial last row
block, the multi-projection launch and graph replays.  Each output is the
same arithmetic whatever the tiles per workgroup, so results at 1 and 2
tiles and in one multi-projection launch are bitwise equal.
"""
import numpy as np
import pytest
import torch

import mlxcel_amd as mq
import oracle as orc
from helpers import TOL, affine_case, announce, dev_bf16, dev_u32, host_u16, max_rel, setknob

pytestmark = pytest.mark.gpu


@pytest.fixture
def kq(monkeypatch):
    setknob(monkeypatch, "MLXQ_QMV_KERNEL", "kq")


def run(x, wq, s, b, gs, bits):
    y = mq.quantized_matmul(dev_bf16(x), dev_u32(wq), dev_bf16(s), dev_bf16(b), True, gs, bits)
    torch.cuda.synchronize()
    return host_u16(y)


@pytest.mark.parametrize("bits,gs", [(4, 32), (4, 64), (4, 128), (8, 32), (8, 64), (8, 128)])
@pytest.mark.parametrize("M", [1, 3, 5, 8, 9, 12, 16])
def test_kq_affine_every_variant(kq, bits, gs, M):
    # N = 200: the last 16-row block is partial; K = 3072: three ranges of
    # 1024 (4-bit) or six of 512 (8-bit)
    N, K = 200, 3072
    announce("kq_affine", bits, gs, M)
    x, wq, s, b = affine_case(M, N, K, gs, bits, 5300 + M + bits + gs)
    assert max_rel(run(x, wq, s, b, gs, bits), orc.qmm_t_affine(x, wq, s, b, gs, bits)) <= TOL


@pytest.mark.parametrize("bits,K", [(4, 1024), (4, 2048), (4, 5120), (8, 512), (8, 1536)])
@pytest.mark.parametrize("M", [6, 16])
def test_kq_range_counts(kq, bits, K, M):
    # one, two, three and five staged ranges
    N = 264
    announce("kq_ranges", bits, K, M)
    x, wq, s, b = affine_case(M, N, K, 64, bits, 5400 + M + K + bits)
    assert max_rel(run(x, wq, s, b, 64, bits), orc.qmm_t_affine(x, wq, s, b, 64, bits)) <= TOL


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M", [5, 8, 16])
def test_kq_tiles_per_workgroup_bitwise(monkeypatch, bits, M):
    # 1, 2, 3 and 4 tiles per workgroup (partial last blocks): the same
    # sums in the same order
    N, K = 1000, 4096
    announce("kq_tiles", bits, M)
    x, wq, s, b = affine_case(M, N, K, 64, bits, 5500 + M + bits)
    setknob(monkeypatch, "MLXQ_QMV_KERNEL", "kq")
    ys = []
    for t in ("1", "2", "3", "4"):
        setknob(monkeypatch, "MLXQ_QMV_KQ_T", t)
        ys.append(run(x, wq, s, b, 64, bits))
    for y in ys[1:]:
        np.testing.assert_array_equal(ys[0], y)
    assert max_rel(ys[0], orc.qmm_t_affine(x, wq, s, b, 64, bits)) <= TOL


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M", [5, 8, 16])
@pytest.mark.parametrize("N,K", [(4096, 4096), (4096, 12288)])
def test_kq_qwen3_8b_shapes_default_route(monkeypatch, bits, M, N, K):
    # o (4096 x 4096) and down (4096 x 12288) of the Qwen3-8B shape on the
    # default route: this kernel past 8 rows only over at most 12 staged
    # ranges (8-bit down at 16 rows: 24, the split-K kernel); bitwise the
    # forced kernel's result, within tolerance of the oracle and of the other
    announce("kq_qwen3", bits, M, N, K)
    x, wq, s, b = affine_case(M, N, K, 64, bits, 5600 + M + bits + K)
    y = run(x, wq, s, b, 64, bits)
    routed, other = ("kq", "mid") if M <= 8 or K * bits <= 12288 * 4 else ("mid", "kq")
    setknob(monkeypatch, "MLXQ_QMV_KERNEL", routed)
    np.testing.assert_array_equal(y, run(x, wq, s, b, 64, bits))
    assert max_rel(y, orc.qmm_t_affine(x, wq, s, b, 64, bits)) <= TOL
    setknob(monkeypatch, "MLXQ_QMV_KERNEL", other)
    assert max_rel(y, run(x, wq, s, b, 64, bits)) <= TOL


def test_kq_repeats_bitwise(kq):
    announce("kq_repeats")
    M, N, K = 16, 520, 4096
    x, wq, s, b = affine_case(M, N, K, 64, 4, 5700)
    np.testing.assert_array_equal(run(x, wq, s, b, 64, 4), run(x, wq, s, b, 64, 4))


@pytest.mark.parametrize("M", [5, 8, 16])
def test_kq_qkv_one_launch(M):
    # q / k / v of the Qwen3-8B shape (4096 + 1024 + 1024 rows) in one launch
    # of 32-row workgroups: bitwise the single calls
    announce("kq_qkv_multi", M)
    K = 4096
    x = orc.normal_bf16((M, K), 1.0, 5800 + M)
    sets = [orc.affine_quantize(orc.normal_bf16((N, K), 0.02, 5810 + i), 64, 4) for i, N in enumerate([4096, 1024, 1024])]
    xd = dev_bf16(x)
    dev = [(dev_u32(w), dev_bf16(s), dev_bf16(b)) for w, s, b in sets]
    multi = mq.quantized_matmul_multi(xd, [d[0] for d in dev], [d[1] for d in dev], [d[2] for d in dev], 64, 4)
    single = [mq.quantized_matmul(xd, *d, True, 64, 4) for d in dev]
    torch.cuda.synchronize()
    for i in range(3):
        np.testing.assert_array_equal(host_u16(multi[i]), host_u16(single[i]), err_msg=f"projection {i}")
        assert max_rel(host_u16(multi[i]), orc.qmm_t_affine(x, *sets[i], 64, 4)) <= TOL


def test_kq_graph_replays(kq):
    announce("kq_graph_replays")
    M, N, K = 12, 392, 4096
    _, wq, s, b = affine_case(1, N, K, 64, 4, 5900)
    W, S, Bi = dev_u32(wq), dev_bf16(s), dev_bf16(b)
    xs = [orc.normal_bf16((M, K), 1.0, 5901 + i) for i in range(3)]
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


@pytest.mark.parametrize("M,K,gs,bits", [(8, 2880, 64, 4), (16, 4096, 32, 4)])
def test_kq_uncovered_shapes_fall_back(kq, M, K, gs, bits):
    # K not a multiple of the 1024-wide range; 16 rows x 4 group slots need
    # more than two A tiles: another kernel runs
    announce("kq_fallback", M, K, gs, bits)
    x, wq, s, b = affine_case(M, 96, K, gs, bits, 5950 + M)
    assert max_rel(run(x, wq, s, b, gs, bits), orc.qmm_t_affine(x, wq, s, b, gs, bits)) <= TOL


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
@pytest.mark.parametrize("M", [9, 12, 16])
@pytest.mark.parametrize("N,kernel", [(12288, "kq"), (14336, "mr")])
def test_single_tall_matrix_9_16_rows_route(monkeypatch, dtype, M, N, kernel):
    # a single 4-bit call at 9-16 rows: 12288 rows (768 tiles of 16, three
    # to a workgroup fill one round) take this kernel, 14336 rows (four to a
    # workgroup) the whole-row one; bitwise that forced kernel, within
    # tolerance of a float32 product of the dequantized weights
    announce("single_tall_route", dtype, M, N, kernel)
    K = 4096
    dt = torch.float16 if dtype == "float16" else torch.bfloat16
    g = torch.Generator(device="cuda").manual_seed(6000 + M + N)
    w = (torch.randn(N, K, device="cuda", generator=g) * 0.02).to(dt)
    x = torch.randn(M, K, device="cuda", generator=g).to(dt)
    wq, s, b = mq.quantize(w, 64, 4)
    y = host_u16(mq.quantized_matmul(x, wq, s, b, True, 64, 4))
    setknob(monkeypatch, "MLXQ_QMV_KERNEL", kernel)
    np.testing.assert_array_equal(y, host_u16(mq.quantized_matmul(x, wq, s, b, True, 64, 4)))
    ref = x.float() @ mq.dequantize(wq, s, b, 64, 4).float().t()
    got = torch.from_numpy(y.astype(np.int16)).view(dt).float().cuda()
    assert float((got - ref).abs().max() / ref.abs().max()) <= TOL


@pytest.mark.parametrize("M", [3, 4])
def test_lm_head_3_4_rows_takes_split_k(monkeypatch, M):
    # 4-bit, 151936 rows (2374 blocks of 64: past one round of the CUs) at
    # 3-4 rows: the split-K kernel, bitwise its forced result
    announce("lm_head_3_4_route", M)
    K, N = 4096, 151936
    g = torch.Generator(device="cuda").manual_seed(6100 + M)
    w = (torch.randn(N, K, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
    wq, s, b = mq.quantize(w, 64, 4)
    del w
    y = host_u16(mq.quantized_matmul(x, wq, s, b, True, 64, 4))
    setknob(monkeypatch, "MLXQ_QMV_KERNEL", "mid")
    np.testing.assert_array_equal(y, host_u16(mq.quantized_matmul(x, wq, s, b, True, 64, 4)))
    rows = slice(0, 4096)
    ref = x.float() @ mq.dequantize(wq[rows], s[rows], b[rows], 64, 4).float().t()
    got = torch.from_numpy(y[:, rows].astype(np.int16)).view(torch.bfloat16).float().cuda()
    assert float((got - ref).abs().max() / ref.abs().max()) <= TOL

