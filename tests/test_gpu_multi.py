"""GPU checks of mlxq_quantized_matmul_multi (several projections of one
activation: q/k/v, gate/up): every output is bit for bit the separate
mlxq_quantized_matmul call's, and within max|y - y_ref| / max|y_ref| <= 1e-2
of the oracle.  Decode rows (1-2, and 3-4 over long rows) take the single
row-streaming launch over all projections; 3-16 rows where every projection
takes the same mid-size kernel take one launch of it (and one reduction of
the split-K partials); other row counts, and forced kernels, run the calls
one after another and must give the same bytes.  Where the projections'
whole-row blocks together need more than one round of the CUs, the one
launch runs the mid-size kernel and matches single calls on that kernel.
"""
import numpy as np
import pytest
import torch

import mlxcel_amd as mq
import oracle as orc
from helpers import TOL, announce, dev_bf16, dev_u32, dev_u8, host_u16, max_rel, setknob

pytestmark = pytest.mark.gpu


def affine_sets(Ns, K, bits, gs, seed):
    sets = []
    for i, N in enumerate(Ns):
        wq, s, b = orc.affine_quantize(orc.normal_bf16((N, K), 0.02, seed + i), gs, bits)
        sets.append((wq, s, b))
    return sets


def run_both(x, sets, gs, bits, mode="affine"):
    xd = dev_bf16(x)
    if mode == "affine":
        dev = [(dev_u32(w), dev_bf16(s), dev_bf16(b)) for w, s, b in sets]
    else:
        dev = [(dev_u32(w), dev_u8(s), None) for w, s in sets]
    multi = mq.quantized_matmul_multi(xd, [d[0] for d in dev], [d[1] for d in dev],
                                      [d[2] for d in dev] if mode == "affine" else None, gs, bits, mode)
    single = [mq.quantized_matmul(xd, d[0], d[1], d[2], True, gs, bits, mode) for d in dev]
    torch.cuda.synchronize()
    return [host_u16(t) for t in multi], [host_u16(t) for t in single]


def check(x, sets, gs, bits, mode="affine"):
    multi, single = run_both(x, sets, gs, bits, mode)
    for i, (m, s) in enumerate(zip(multi, single)):
        np.testing.assert_array_equal(m, s, err_msg=f"projection {i}")
        if mode == "affine":
            want = orc.qmm_t_affine(x, *sets[i], gs, bits)
        else:
            want = orc.fp_qmm_t_mxfp4(x, *sets[i])
        assert max_rel(m, want) <= TOL, (i, max_rel(m, want))


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M", [1, 2, 4])
def test_qkv_llama3_8b(bits, M):
    announce("multi_qkv", bits, M)
    K = 4096
    x = orc.normal_bf16((M, K), 1.0, 900 + M)
    check(x, affine_sets([4096, 1024, 1024], K, bits, 64, 910 + bits), 64, bits)


@pytest.mark.parametrize("M", [1, 2])
def test_gate_up_qwen3_8b(M):
    announce("multi_gate_up", M)
    K = 4096
    x = orc.normal_bf16((1, M, K), 1.0, 920 + M)  # leading dims fold into rows
    check(x, affine_sets([12288, 12288], K, 4, 64, 930), 64, 4)


@pytest.mark.parametrize("n", [1, 2, 3, 4])
@pytest.mark.parametrize("gs", [32, 128])
def test_ragged_widths_and_counts(n, gs):
    # partial row tiles in every projection, one of them a single row
    announce("multi_ragged", n, gs)
    K = 1536
    Ns = [200, 77, 1, 333][:n]
    x = orc.normal_bf16((1, K), 1.0, 940 + n)
    check(x, affine_sets(Ns, K, 4, gs, 950 + n + gs), gs, 4)


def test_mxfp4_projections():
    announce("multi_mxfp4")
    K = 2880
    x = orc.normal_bf16((1, K), 1.0, 960)
    sets = [orc.mxfp4_quantize(orc.normal_bf16((N, K), 0.02, 961 + i)) for i, N in enumerate([4096, 512, 512])]
    check(x, sets, 32, 4, "mxfp4")


@pytest.mark.parametrize("M", [3, 8, 20])
def test_other_row_counts_run_separately(M):
    # 3 rows over short rows (block-MFMA), 8 (mid-size kernel), 20 (prefill GEMM)
    announce("multi_rows", M)
    K = 2048
    x = orc.normal_bf16((M, K), 1.0, 970 + M)
    check(x, affine_sets([512, 256], K, 4, 64, 975 + M), 64, 4)


@pytest.mark.parametrize("kernel", ["fr", "b4", "mfma"])
def test_forced_kernels(monkeypatch, kernel):
    setknob(monkeypatch, "MLXQ_QMV_KERNEL", kernel)
    announce("multi_forced", kernel)
    K = 4096
    x = orc.normal_bf16((1, K), 1.0, 980)
    check(x, affine_sets([1024, 512, 512], K, 4, 64, 981), 64, 4)


def test_graph_replays():
    announce("multi_graph")
    K = 4096
    sets = affine_sets([4096, 1024, 1024], K, 4, 64, 990)
    dev = [(dev_u32(w), dev_bf16(s), dev_bf16(b)) for w, s, b in sets]
    xs = [orc.normal_bf16((1, K), 1.0, 991 + i) for i in range(3)]
    xd = dev_bf16(xs[0])
    outs = [torch.empty(1, N, dtype=torch.bfloat16, device="cuda") for N in (4096, 1024, 1024)]
    args = ([d[0] for d in dev], [d[1] for d in dev], [d[2] for d in dev], 64, 4)
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        mq.quantized_matmul_multi(xd, *args, out=outs)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        mq.quantized_matmul_multi(xd, *args, out=outs)
    torch.cuda.synchronize()
    for i in (0, 1, 2, 1):
        xd.copy_(dev_bf16(xs[i]))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for o, (w, s, b) in zip(outs, dev):
            np.testing.assert_array_equal(host_u16(o), host_u16(mq.quantized_matmul(xd, w, s, b)))


def test_argument_errors():
    announce("multi_errors")
    K = 256
    sets = affine_sets([64, 64], K, 4, 64, 999)
    dev = [(dev_u32(w), dev_bf16(s), dev_bf16(b)) for w, s, b in sets]
    xd = dev_bf16(orc.normal_bf16((1, K), 1.0, 998))
    with pytest.raises(ValueError):  # K of the second weight disagrees with x
        bad = dev_u32(orc.affine_quantize(orc.normal_bf16((64, 512), 0.02, 997), 64, 4)[0])
        mq.quantized_matmul_multi(xd, [dev[0][0], bad], [d[1] for d in dev], [d[2] for d in dev], 64, 4)
    with pytest.raises(ValueError):  # more than four projections
        mq.quantized_matmul_multi(xd, [dev[0][0]] * 5, [dev[0][1]] * 5, [dev[0][2]] * 5, 64, 4)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M", [5, 8, 16])
def test_qkv_mid_one_launch(bits, M):
    # 5-16 rows: q/k/v of the Qwen3-8B shape each take the split-K mid-size
    # kernel alone, so the three run as one launch and one reduction
    announce("multi_qkv_mid", bits, M)
    K = 4096
    x = orc.normal_bf16((M, K), 1.0, 1900 + M)
    check(x, affine_sets([4096, 1024, 1024], K, bits, 64, 1910 + bits), 64, bits)


@pytest.mark.parametrize("M", [3, 4])
def test_gate_up_whole_row_one_launch(M):
    # 3-4 rows: gate/up (12288 rows each) each take the whole-row kernel
    # alone, so the two run as one launch of it
    announce("multi_gate_up_mr", M)
    K = 4096
    x = orc.normal_bf16((M, K), 1.0, 1920 + M)
    check(x, affine_sets([12288, 12288], K, 4, 64, 1930), 64, 4)


@pytest.mark.parametrize("M", [5, 8, 16])
def test_gate_up_past_one_round_takes_mid(monkeypatch, M):
    # 5-16 rows: gate and up alone each take the whole-row kernel (192
    # 64-row blocks, one round of the CUs), but together 384 blocks: the one
    # launch runs the split-K mid-size kernel instead, so each output is
    # bitwise a single call's on that kernel (MLXQ_QMV_MR=0 MLXQ_QMV_KQ=0) and within
    # tolerance of the oracle and of the whole-row single calls
    announce("multi_gate_up_mid", M)
    K = 4096
    x = orc.normal_bf16((M, K), 1.0, 1940 + M)
    sets = affine_sets([12288, 12288], K, 4, 64, 1950)
    multi, single_mr = run_both(x, sets, 64, 4)
    setknob(monkeypatch, "MLXQ_QMV_MR", "0")
    setknob(monkeypatch, "MLXQ_QMV_KQ", "0")  # single calls on the split-K kernel
    _, single_mid = run_both(x, sets, 64, 4)
    for i in range(2):
        np.testing.assert_array_equal(multi[i], single_mid[i], err_msg=f"projection {i}")
        assert max_rel(multi[i], single_mr[i]) <= TOL
        assert max_rel(multi[i], orc.qmm_t_affine(x, *sets[i], 64, 4)) <= TOL


@pytest.mark.parametrize("M", [5, 8, 16])
def test_gate_up_past_one_round_8bit_stays_whole_row(M):
    # 8-bit codes keep the whole-row kernel past one round of the CUs (it is
    # the faster there), alone and in one launch: bitwise the single calls
    announce("multi_gate_up_8bit_mr", M)
    K = 4096
    x = orc.normal_bf16((M, K), 1.0, 1960 + M)
    check(x, affine_sets([12288, 12288], K, 8, 64, 1970), 64, 8)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M", [5, 16])
def test_tall_matrix_route_by_code_width(monkeypatch, bits, M):
    # a 151936-row matrix (the LM head shape, 2374 blocks of 64 rows) at
    # 5-16 rows: 8-bit codes on the whole-row kernel, 4-bit on the split-K
    # kernel; bitwise the forced kernel of its width, within tolerance of the
    # oracle on a slice of rows
    announce("tall_route", bits, M)
    K, N = 4096, 151936
    g = torch.Generator(device="cuda").manual_seed(1980 + bits + M)
    w = (torch.randn(N, K, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
    wq, s, b = mq.quantize(w, 64, bits)
    del w
    y = host_u16(mq.quantized_matmul(x, wq, s, b, True, 64, bits))
    setknob(monkeypatch, "MLXQ_QMV_KERNEL", "mr" if bits == 8 else "mid")
    np.testing.assert_array_equal(y, host_u16(mq.quantized_matmul(x, wq, s, b, True, 64, bits)))
    rows = slice(0, 4096)
    ref = x.float() @ mq.dequantize(wq[rows], s[rows], b[rows], 64, bits).float().t()
    got = torch.from_numpy(y[:, rows].astype(np.int16)).view(torch.bfloat16).float().cuda()
    assert float((got - ref).abs().max() / ref.abs().max()) <= TOL


@pytest.mark.parametrize("gs", [32, 128])
def test_mid_one_launch_ragged(gs):
    # ragged widths (partial 128-row blocks, widths not a multiple of 4: the
    # reduction's scalar path), K with several splits
    announce("multi_mid_ragged", gs)
    K = 8192
    x = orc.normal_bf16((12, K), 1.0, 1940 + gs)
    check(x, affine_sets([1030, 77, 513], K, 4, gs, 1950 + gs), gs, 4)


def test_mid_one_launch_graph_replays():
    announce("multi_mid_graph")
    K, M = 4096, 8
    sets = affine_sets([4096, 1024, 1024], K, 4, 64, 1960)
    dev = [(dev_u32(w), dev_bf16(s), dev_bf16(b)) for w, s, b in sets]
    xs = [orc.normal_bf16((M, K), 1.0, 1961 + i) for i in range(3)]
    xd = dev_bf16(xs[0])
    outs = [torch.empty(M, N, dtype=torch.bfloat16, device="cuda") for N in (4096, 1024, 1024)]
    args = ([d[0] for d in dev], [d[1] for d in dev], [d[2] for d in dev], 64, 4)
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        mq.quantized_matmul_multi(xd, *args, out=outs)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        mq.quantized_matmul_multi(xd, *args, out=outs)
    torch.cuda.synchronize()
    for i in (0, 1, 2, 1):
        xd.copy_(dev_bf16(xs[i]))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for o, (w, s, b) in zip(outs, dev):
            np.testing.assert_array_equal(host_u16(o), host_u16(mq.quantized_matmul(xd, w, s, b)))
