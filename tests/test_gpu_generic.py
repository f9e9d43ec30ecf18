"""GPU parity of the general quantized matmul (qmm_gen.hip) against the numpy
restatement of MLX's CPU kernels (oracle/generic.py; overlays/cpu/mlx/backend/
cpu/quantized.cpp:107-257, 550-597):

- float16 / float32 activations and scales, and mixed ones (promoted to
  float32 as ops.cpp:4974-4992 does), for quantized_matmul, gather_qmm and
  quantized_linear;
- affine codes of 2, 3, 5 and 6 bits (and 4/8 through the general kernel
  when the types are not all bfloat16);
- transpose=false;
- more rows per gathered matrix than the decode kernels stage;
- batched weights that broadcast against x's batch;
- strided and misaligned operands (copied to row-contiguous first, as the
  reference's ensure_row_contiguous, rocm/quantized/qmm.hip:3557-3564): the
  result is bitwise that of the contiguous call.

Tolerance: max|y - y_ref| / max|y_ref| <= 1e-2 for 16-bit results (the
north-star bound; float16 also rounds the dequantized weights to float16 as
the reference's GPU route does) and <= 1e-4 for float32 results.
"""
import numpy as np
import pytest
import torch

import mlxcel_amd as mq
from oracle import generic as og
from helpers import announce, dev_u32, setknob

pytestmark = pytest.mark.gpu

TD = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}
PROMOTE = {("bfloat16", "bfloat16"): "bfloat16", ("float16", "float16"): "float16",
           ("float32", "float32"): "float32"}


def promote(a, b):
    return PROMOTE.get((a, b), "float32")


def tol(dtype):
    return 1e-4 if dtype == "float32" else 1e-2


def dev(vals, dtype):
    """device tensor of `dtype` holding vals rounded to it, and those exact values (float64)."""
    t = torch.from_numpy(np.asarray(vals, dtype=np.float32)).to(TD[dtype]).cuda()
    return t, t.float().cpu().numpy().astype(np.float64)


def case(M, N, K, bits, gs, xt, st, transpose, seed, batch=()):
    rng = np.random.default_rng(seed)
    x, xv = dev(rng.standard_normal(tuple(batch) + (M, K)), xt)
    rows, cols = (N, K) if transpose else (K, N)
    codes = rng.integers(0, 1 << bits, size=(rows, cols))
    wq = dev_u32(og.pack_codes(codes, bits))
    s, sv = dev(rng.uniform(0.002, 0.02, size=(rows, cols // gs)), st)
    b, bv = dev(rng.uniform(-0.1, 0.1, size=(rows, cols // gs)), st)
    return (x, wq, s, b), (xv, og.pack_codes(codes, bits), sv, bv)


def rel(got, want):
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-30))


def check(y, want64, dtype):
    assert y.dtype == TD[dtype]
    got = y.float().cpu().numpy().astype(np.float64)
    r = rel(got, og.round_to(want64, dtype))
    assert r <= tol(dtype), r


@pytest.mark.parametrize("transpose", [True, False])
@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("xt,st", [("float16", "float16"), ("float32", "float32"), ("bfloat16", "bfloat16"),
                                   ("bfloat16", "float16")])
def test_quantized_matmul_types_and_widths(transpose, bits, xt, st):
    gs = 64
    announce("gen_qmm", transpose, bits, xt, st)
    N = 200 if transpose else 192  # transpose=false quantizes along N: a multiple of group_size
    (x, wq, s, b), (xv, wqn, sv, bv) = case(7, N, 512, bits, gs, xt, st, transpose, 2000 + bits)
    y = mq.quantized_matmul(x, wq, s, b, transpose, gs, bits)
    check(y, og.qmm(xv, wqn, sv, bv, transpose, gs, bits), promote(xt, st))


@pytest.mark.parametrize("gs", [32, 128])
@pytest.mark.parametrize("M", [1, 16, 17, 100])
@pytest.mark.parametrize("dtype", ["float16", "float32"])
def test_rows_and_groups(gs, M, dtype):
    # 16- and 64-row tiles, partial tiles, the K split of small row counts
    announce("gen_rows", gs, M, dtype)
    (x, wq, s, b), (xv, wqn, sv, bv) = case(M, 136, 1024, 4, gs, dtype, dtype, True, 2100 + M + gs)
    y = mq.quantized_matmul(x, wq, s, b, True, gs, 4)
    check(y, og.qmm(xv, wqn, sv, bv, True, gs, 4), dtype)


@pytest.mark.parametrize("ks", [1, 3, 8])
def test_forced_k_split(monkeypatch, ks):
    setknob(monkeypatch, "MLXQ_GEN_KS", str(ks))
    announce("gen_ks", ks)
    (x, wq, s, b), (xv, wqn, sv, bv) = case(3, 100, 2048, 3, 64, "float16", "float16", True, 2200 + ks)
    y = mq.quantized_matmul(x, wq, s, b, True, 64, 3)
    check(y, og.qmm(xv, wqn, sv, bv, True, 64, 3), "float16")


@pytest.mark.parametrize("K", [40, 100, 264])
def test_no_transpose_ragged_k(K):
    # transpose=false reduces over the rows of w: K need not be a multiple of 32 or 8
    announce("gen_ragged_k", K)
    (x, wq, s, b), (xv, wqn, sv, bv) = case(5, 160, K, 4, 32, "float32", "float32", False, 2300 + K)
    y = mq.quantized_matmul(x, wq, s, b, False, 32, 4)
    check(y, og.qmm(xv, wqn, sv, bv, False, 32, 4), "float32")


@pytest.mark.parametrize("xt", ["float16", "float32"])
def test_mxfp4_float_activations(xt):
    announce("gen_mxfp4", xt)
    rng = np.random.default_rng(2400)
    x, xv = dev(rng.standard_normal((9, 256)), xt)
    codes = rng.integers(0, 16, size=(72, 256))
    wqn = og.pack_codes(codes, 4)
    sc = rng.integers(118, 127, size=(72, 8)).astype(np.uint8)
    wq = dev_u32(wqn)
    y = mq.quantized_matmul(x, wq, torch.from_numpy(sc).cuda(), None, True, 32, 4, "mxfp4")
    check(y, og.qmm(xv, wqn, sc, None, True, 32, 4, "mxfp4"), xt)


@pytest.mark.parametrize("xt,bits", [("float16", 3), ("float32", 6), ("bfloat16", 5)])
def test_gather_qmm_general(xt, bits):
    announce("gen_gather", xt, bits)
    E, N, K, gs = 5, 96, 256, 32
    rng = np.random.default_rng(2500 + bits)
    x, xv = dev(rng.standard_normal((3, 2, K)), xt)
    codes = rng.integers(0, 1 << bits, size=(E, N, K))
    wqn = og.pack_codes(codes, bits)
    wq = dev_u32(wqn)
    s, sv = dev(rng.uniform(0.002, 0.02, size=(E, N, K // gs)), xt)
    b, bv = dev(rng.uniform(-0.1, 0.1, size=(E, N, K // gs)), xt)
    lhs = np.array([[0, 2, 1, 1]], dtype=np.int32)
    rhs = np.array([[4, 0, 4, 2]], dtype=np.int64)
    y = mq.gather_qmm(x, wq, s, b, torch.from_numpy(lhs).cuda(), torch.from_numpy(rhs).cuda(), True, gs, bits)
    want = og.gather_qmm(xv, wqn, sv, bv, lhs, rhs, True, gs, bits).reshape(1, 4, 2, N)
    check(y, want, xt)


def test_gather_many_rows_per_matrix():
    # bfloat16 4-bit but 40 rows per gathered matrix: more than the decode
    # kernels stage, so the general kernel tiles them
    announce("gen_gather_rows")
    E, N, K, gs = 3, 64, 256, 64
    rng = np.random.default_rng(2550)
    x, xv = dev(rng.standard_normal((2, 40, K)), "bfloat16")
    codes = rng.integers(0, 16, size=(E, N, K))
    wqn = og.pack_codes(codes, 4)
    wq = dev_u32(wqn)
    s, sv = dev(rng.uniform(0.002, 0.02, size=(E, N, K // gs)), "bfloat16")
    b, bv = dev(rng.uniform(-0.1, 0.1, size=(E, N, K // gs)), "bfloat16")
    lhs = np.array([1, 0, 1], dtype=np.int32)
    rhs = np.array([2, 2, 0], dtype=np.int32)
    y = mq.gather_qmm(x, wq, s, b, torch.from_numpy(lhs).cuda(), torch.from_numpy(rhs).cuda(), True, gs, 4)
    check(y, og.gather_qmm(xv, wqn, sv, bv, lhs, rhs, True, gs, 4), "bfloat16")


def test_batched_weights_broadcast():
    # x [2, 1, M, K] against w [1, 3, N, Kp]: out [2, 3, M, N]
    announce("gen_batched")
    gs, bits, N, K, M = 32, 4, 64, 128, 3
    rng = np.random.default_rng(2600)
    x, xv = dev(rng.standard_normal((2, 1, M, K)), "float16")
    codes = rng.integers(0, 16, size=(1, 3, N, K))
    wqn = og.pack_codes(codes, bits)
    wq = dev_u32(wqn)
    s, sv = dev(rng.uniform(0.002, 0.02, size=(1, 3, N, K // gs)), "float16")
    b, bv = dev(rng.uniform(-0.1, 0.1, size=(1, 3, N, K // gs)), "float16")
    y = mq.quantized_matmul(x, wq, s, b, True, gs, bits)
    assert tuple(y.shape) == (2, 3, M, N)
    want = np.stack([np.stack([og.qmm(xv[i, 0], wqn[0, j], sv[0, j], bv[0, j], True, gs, bits)
                               for j in range(3)]) for i in range(2)])
    check(y, want, "float16")


def test_quantized_linear_float16_bias():
    announce("gen_linear")
    (x, wq, s, b), (xv, wqn, sv, bv) = case(4, 96, 256, 4, 64, "float16", "float16", True, 2700)
    rng = np.random.default_rng(2701)
    lb, lbv = dev(rng.standard_normal(96), "float16")
    y = mq.quantized_linear(x, wq, s, b, lb, 64, 4)
    # MLX adds the float16 bias to the float16 product: two roundings
    want = og.round_to(og.round_to(og.qmm(xv, wqn, sv, bv, True, 64, 4), "float16") + lbv, "float16")
    got = y.float().cpu().numpy().astype(np.float64)
    assert rel(got, want) <= 1e-2


@pytest.mark.parametrize("kind", ["x_transposed", "x_sliced", "out_strided", "w_strided"])
def test_strided_operands_bitwise(kind):
    # bfloat16 4-bit (the specialised kernels) and float16 3-bit (the general one)
    announce("gen_strided", kind)
    for bits, xt in ((4, "bfloat16"), (3, "float16")):
        (x, wq, s, b), _ = case(6, 128, 256, bits, 64, xt, xt, True, 2800 + bits)
        want = mq.quantized_matmul(x, wq, s, b, True, 64, bits)
        if kind == "x_transposed":
            xs = x.t().contiguous().t()  # same values, column-major
            assert not xs.is_contiguous()
            y = mq.quantized_matmul(xs, wq, s, b, True, 64, bits)
        elif kind == "x_sliced":
            big = torch.zeros(6, 256 + 3, dtype=x.dtype, device="cuda")
            big[:, 3:] = x
            xs = big[:, 3:]  # misaligned rows with a row stride of 259
            y = mq.quantized_matmul(xs, wq, s, b, True, 64, bits)
        elif kind == "w_strided":
            wbig = torch.zeros(2 * wq.shape[0], wq.shape[1], dtype=wq.dtype, device="cuda")
            wbig[::2] = wq
            y = mq.quantized_matmul(x, wbig[::2], s, b, True, 64, bits)
        else:
            obig = torch.full((128, 6), 7.0, dtype=want.dtype, device="cuda")
            y = obig.t()
            mq.quantized_matmul(x, wq, s, b, True, 64, bits, out=y)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(y.float().cpu().numpy(), want.float().cpu().numpy())


# ---- dequantize for every type and width -------------------------------------
# Bit for bit the reference's dequantize graph (ops.cpp:5494-5586 + astype at
# 5788-5793, oracle/generic.py dequantize_graph): To(T(T(q * s) + b)).

@pytest.mark.parametrize("ts", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("to", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("bits", [1, 3, 4, 5])
def test_dequantize_types_bitwise(ts, to, bits):
    announce("gen_dequant", ts, to, bits)
    rows, K, gs = 8, 256, 64
    rng = np.random.default_rng(2900 + bits)
    codes = rng.integers(0, 1 << bits, size=(rows, K))
    wqn = og.pack_codes(codes, bits)
    s, sv = dev(rng.uniform(-0.05, 0.05, size=(rows, K // gs)), ts)
    b, bv = dev(rng.uniform(-0.2, 0.2, size=(rows, K // gs)), ts)
    y = mq.dequantize(dev_u32(wqn), s, b, gs, bits, "affine", dtype=TD[to])
    assert y.dtype == TD[to]
    want = og.dequantize_graph(wqn, sv, bv, gs, bits, K, ts, to)
    np.testing.assert_array_equal(y.float().cpu().numpy().astype(np.float64), want)


@pytest.mark.parametrize("to", ["float16", "float32"])
def test_mxfp4_dequantize_every_code_and_scale(to):
    # row r has scale byte r (0..255) and codes 0..15 twice
    announce("gen_mxfp4_dequant", to)
    codes = np.tile(np.arange(32) % 16, (256, 1))
    wqn = og.pack_codes(codes, 4)
    sc = np.arange(256, dtype=np.uint8)[:, None]
    y = mq.dequantize(dev_u32(wqn), torch.from_numpy(sc).cuda(), None, 32, 4, "mxfp4", dtype=TD[to])
    want = og.mxfp4_dequantize_graph(wqn, sc, 32, to)
    np.testing.assert_array_equal(y.float().cpu().numpy().astype(np.float64), want)


def test_dequantize_strided_scales():
    # a transposed (non-contiguous) scales view is copied first: same bits
    announce("gen_dequant_strided")
    rng = np.random.default_rng(2950)
    codes = rng.integers(0, 16, size=(16, 128))
    wqn = og.pack_codes(codes, 4)
    s, _ = dev(rng.uniform(-0.05, 0.05, size=(16, 2)), "float16")
    b, _ = dev(rng.uniform(-0.2, 0.2, size=(16, 2)), "float16")
    want = mq.dequantize(dev_u32(wqn), s, b, 64, 4)
    st = s.t().contiguous().t()
    assert not st.is_contiguous()
    got = mq.dequantize(dev_u32(wqn), st, b, 64, 4)
    np.testing.assert_array_equal(got.float().cpu().numpy(), want.float().cpu().numpy())


# ---- float16 decode on the row-streaming kernel --------------------------------
# 1-4 rows of float16 x against 2-D weights with float16 scales/biases (affine
# 4/8-bit) or e8m0 scales (mxfp4) run the row-streaming kernel's float16
# instantiation (codes widened to float16 1024 + q pairs).

@pytest.mark.parametrize("bits,gs", [(4, 32), (4, 64), (4, 128), (8, 32), (8, 64), (8, 128)])
@pytest.mark.parametrize("M", [1, 2, 3, 4])
@pytest.mark.parametrize("N,K", [(1000, 2304), (4096, 4096), (512, 14336)])
def test_float16_decode_affine(bits, gs, M, N, K):
    announce("f16_decode", bits, gs, M, N, K)
    (x, wq, s, b), (xv, wqn, sv, bv) = case(M, N, K, bits, gs, "float16", "float16", True, 3000 + M + bits + gs)
    y = mq.quantized_matmul(x, wq, s, b, True, gs, bits)
    check(y, og.qmm(xv, wqn, sv, bv, True, gs, bits), "float16")


@pytest.mark.parametrize("bits,gs", [(4, 32), (4, 64), (4, 128), (8, 32), (8, 64), (8, 128)])
@pytest.mark.parametrize("M", [1, 3, 5, 8, 12, 16])
def test_float16_whole_row_decode(monkeypatch, bits, gs, M):
    # the whole-row mid-size kernel's float16 instantiation (MLXQ_QMV_KERNEL=mr
    # forces it at any row count; 1024 + q code pairs, float16 MFMAs)
    setknob(monkeypatch, "MLXQ_QMV_KERNEL", "mr")
    announce("f16_mr", bits, gs, M)
    (x, wq, s, b), (xv, wqn, sv, bv) = case(M, 200, 3072, bits, gs, "float16", "float16", True, 3300 + M + bits + gs)
    y = mq.quantized_matmul(x, wq, s, b, True, gs, bits)
    check(y, og.qmm(xv, wqn, sv, bv, True, gs, bits), "float16")


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M", [5, 16])
def test_float16_whole_row_decode_default_route(bits, M):
    # 5-16 float16 rows against a matrix with ~one 64-row block per CU take
    # the whole-row kernel by default (14336 rows: 224 blocks)
    announce("f16_mr_default", bits, M)
    (x, wq, s, b), (xv, wqn, sv, bv) = case(M, 14336, 4096, bits, 64, "float16", "float16", True, 3400 + M + bits)
    y = mq.quantized_matmul(x, wq, s, b, True, 64, bits)
    check(y, og.qmm(xv, wqn, sv, bv, True, 64, bits), "float16")


@pytest.mark.parametrize("bits,gs", [(4, 32), (4, 64), (4, 128), (8, 32), (8, 64), (8, 128)])
@pytest.mark.parametrize("M", [1, 5, 8, 12, 16])
def test_float16_split_k_mid_decode(monkeypatch, bits, gs, M):
    # the split-K mid-size kernel's float16 instantiation (MLXQ_QMV_KERNEL=mid
    # forces it), K = 3072: three or six K ranges whose fp32 partials the
    # reduction rounds to float16
    setknob(monkeypatch, "MLXQ_QMV_KERNEL", "mid")
    announce("f16_mid", bits, gs, M)
    (x, wq, s, b), (xv, wqn, sv, bv) = case(M, 200, 3072, bits, gs, "float16", "float16", True, 3500 + M + bits + gs)
    y = mq.quantized_matmul(x, wq, s, b, True, gs, bits)
    check(y, og.qmm(xv, wqn, sv, bv, True, gs, bits), "float16")


@pytest.mark.parametrize("bits,gs", [(4, 32), (4, 64), (4, 128), (8, 32), (8, 64), (8, 128)])
@pytest.mark.parametrize("M", [1, 3, 5, 8, 12, 16])
def test_float16_k_split_over_waves_decode(monkeypatch, bits, gs, M):
    # the K-split-over-waves kernel's float16 instantiation (MLXQ_QMV_KERNEL=kq
    # forces it), K = 3072: three or six staged ranges, a partial last block
    setknob(monkeypatch, "MLXQ_QMV_KERNEL", "kq")
    announce("f16_kq", bits, gs, M)
    (x, wq, s, b), (xv, wqn, sv, bv) = case(M, 200, 3072, bits, gs, "float16", "float16", True, 3550 + M + bits + gs)
    y = mq.quantized_matmul(x, wq, s, b, True, gs, bits)
    check(y, og.qmm(xv, wqn, sv, bv, True, gs, bits), "float16")


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M", [3, 5, 8, 16])
def test_float16_kq_default_route_bitwise(monkeypatch, bits, M):
    # 5-16 float16 rows (3-4 with 4-bit codes) against the Qwen3-8B o shape
    # (4096 x 4096: too few blocks for the whole-row kernel) take the
    # K-split-over-waves kernel by default: bitwise the forced kernel at 1-4
    # tiles per workgroup (8-bit at 3 rows: the row-streaming kernel)
    announce("f16_kq_default", bits, M)
    (x, wq, s, b), (xv, wqn, sv, bv) = case(M, 4096, 4096, bits, 64, "float16", "float16", True, 3580 + M + bits)
    y = mq.quantized_matmul(x, wq, s, b, True, 64, bits)
    check(y, og.qmm(xv, wqn, sv, bv, True, 64, bits), "float16")
    if bits == 8 and M < 5:
        return
    setknob(monkeypatch, "MLXQ_QMV_KERNEL", "kq")
    for t in ("1", "2", "3", "4"):
        setknob(monkeypatch, "MLXQ_QMV_KQ_T", t)
        assert torch.equal(y, mq.quantized_matmul(x, wq, s, b, True, 64, bits)), t


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M", [5, 16])
def test_float16_mid_decode_default_route(bits, M):
    # 5-16 float16 rows against the down shape (4096 rows: too few blocks for
    # the whole-row kernel) take the K-split-over-waves kernel at up to 8 rows
    # and the split-K mid kernel past 8 rows over rows longer than 12288
    announce("f16_mid_default", bits, M)
    (x, wq, s, b), (xv, wqn, sv, bv) = case(M, 4096, 14336, bits, 64, "float16", "float16", True, 3600 + M + bits)
    y = mq.quantized_matmul(x, wq, s, b, True, 64, bits)
    check(y, og.qmm(xv, wqn, sv, bv, True, 64, bits), "float16")


@pytest.mark.parametrize("tile", ["-1", "4", "5", "6", "7", "8"])
@pytest.mark.parametrize("bits,gs", [(4, 32), (4, 64), (8, 64), (8, 128)])
@pytest.mark.parametrize("M", [65, 300])
def test_float16_prefill_tile_kernel(monkeypatch, tile, bits, gs, M):
    # float16 prefill on the 32x32-MFMA tile kernel (every tile shape:
    # MLXQ_QMM_TILE; -1 = the planner's), weights dequantized to float16
    setknob(monkeypatch, "MLXQ_QMM_TILE", tile)
    announce("f16_prefill", tile, bits, gs, M)
    (x, wq, s, b), (xv, wqn, sv, bv) = case(M, 384, 1024, bits, gs, "float16", "float16", True, 3700 + M + bits + gs)
    y = mq.quantized_matmul(x, wq, s, b, True, gs, bits)
    check(y, og.qmm(xv, wqn, sv, bv, True, gs, bits), "float16")


@pytest.mark.parametrize("tile,ksplit", [("8", "3"), ("4", "2"), ("6", "5")])
def test_float16_prefill_split_k(monkeypatch, tile, ksplit):
    # K split across workgroups: fp32 partials summed and rounded to float16
    setknob(monkeypatch, "MLXQ_QMM_TILE", tile)
    setknob(monkeypatch, "MLXQ_QMM_KSPLIT", ksplit)
    announce("f16_prefill_splitk", tile, ksplit)
    (x, wq, s, b), (xv, wqn, sv, bv) = case(256, 256, 8192, 4, 64, "float16", "float16", True, 3800)
    y = mq.quantized_matmul(x, wq, s, b, True, 64, 4)
    check(y, og.qmm(xv, wqn, sv, bv, True, 64, 4), "float16")


@pytest.mark.parametrize("M", [1, 2, 4])
def test_float16_decode_mxfp4(M):
    announce("f16_decode_mxfp4", M)
    rng = np.random.default_rng(3100 + M)
    x, xv = dev(rng.standard_normal((M, 2880)), "float16")
    codes = rng.integers(0, 16, size=(2888, 2880))
    wqn = og.pack_codes(codes, 4)
    sc = rng.integers(118, 127, size=(2888, 90)).astype(np.uint8)
    y = mq.quantized_matmul(x, dev_u32(wqn), torch.from_numpy(sc).cuda(), None, True, 32, 4, "mxfp4")
    check(y, og.qmm(xv, wqn, sc, None, True, 32, 4, "mxfp4"), "float16")


def test_float16_decode_multi_matches_separate_calls():
    # quantized_matmul_multi with float16 operands runs the projections one by
    # one on the same kernel: bit for bit the separate calls
    announce("f16_multi")
    parts = [case(1, 512, 2048, 4, 64, "float16", "float16", True, 3200 + i)[0] for i in range(3)]
    x = parts[0][0]
    outs = mq.quantized_matmul_multi(x, [p[1] for p in parts], [p[2] for p in parts], [p[3] for p in parts], 64, 4)
    for p, o in zip(parts, outs):
        want = mq.quantized_matmul(x, p[1], p[2], p[3], True, 64, 4)
        np.testing.assert_array_equal(o.float().cpu().numpy(), want.float().cpu().numpy())
