"""GPU parity of the prefill GEMM (qmm.hip): quantized_matmul with more than
64 activation rows, against the oracle's restatement of MLX's `_qmm_t` /
`fp_qmm_t` (overlays/cpu/mlx/backend/cpu/quantized.cpp:199-257, 550-597) at
sizes the oracle finishes in seconds, and at the full Llama-3-8B prefill
shapes against a float32 torch product of the
bit-exact dequantized weights.  max|y - y_ref| / max|y_ref| <= 1e-2.
"""
import numpy as np
import pytest
import torch

import mlxcel_amd as mq
import oracle as orc
from helpers import TOL, affine_case, announce, dev_bf16, dev_u32, dev_u8, host_u16, max_rel, mxfp4_case, setknob

pytestmark = pytest.mark.gpu


def run(x, wq, s, b, gs, bits):
    y = mq.quantized_matmul(dev_bf16(x), dev_u32(wq), dev_bf16(s), dev_bf16(b), True, gs, bits)
    torch.cuda.synchronize()
    return host_u16(y)


@pytest.mark.parametrize("tile", [-1, 0, 1, 2, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("M,N,K", [(65, 200, 1024), (300, 136, 2048), (512, 384, 512)])
def test_affine_qmm_vs_oracle(monkeypatch, tile, bits, gs, M, N, K):
    # every output-tile shape (MLXQ_QMM_TILE: 16x16-MFMA kernel 0 = 256x128,
    # 1 = 256x256, 2 = 128x128; 32x32-MFMA tile kernel 4 = 256x256,
    # 5 = 256x128, 6 = 128x128, 7 = 256x256 on 4 waves, 8 = 256x128 on 8
    # waves with 8-byte 4-bit weight pieces; -1 = by shape)
    setknob(monkeypatch, "MLXQ_QMM_TILE", str(tile))
    announce("qmm_affine", tile, bits, gs, M, N, K)
    x, wq, s, b = affine_case(M, N, K, gs, bits, 2100 + M + N + bits + gs)
    assert max_rel(run(x, wq, s, b, gs, bits), orc.qmm_t_affine(x, wq, s, b, gs, bits)) <= TOL


@pytest.mark.parametrize("tile", [4, 5, 6, 7, 8])
@pytest.mark.parametrize("bits,gs", [(4, 32), (4, 64), (8, 32), (8, 64)])
def test_affine_qmm_unaligned_scale_rows(monkeypatch, tile, bits, gs):
    # K = 2880 (gpt-oss): K / gs groups per row = 90 or 45, so scale rows are
    # 180 or 90 bytes apart and the tile kernel's 16-byte scale chunks start
    # off their natural alignment
    setknob(monkeypatch, "MLXQ_QMM_TILE", str(tile))
    announce("qmm_unaligned_scales", tile, bits, gs)
    M, N, K = 130, 160, 2880
    x, wq, s, b = affine_case(M, N, K, gs, bits, 2150 + bits + gs)
    assert max_rel(run(x, wq, s, b, gs, bits), orc.qmm_t_affine(x, wq, s, b, gs, bits)) <= TOL


@pytest.mark.parametrize("tile,ksplit", [(-1, 0), (1, 3), (2, 5), (4, 3), (5, 5), (6, 2), (7, 3), (8, 3), (8, 5),
                                         (8, 1)])
def test_affine_qmm_split_k_and_batch_fold(monkeypatch, tile, ksplit):
    # few output tiles and a long K: the K range is split across workgroups
    # (uneven splits included); x given as [2, 128, K] folds into 256 rows
    setknob(monkeypatch, "MLXQ_QMM_TILE", str(tile))
    setknob(monkeypatch, "MLXQ_QMM_KSPLIT", str(ksplit))
    announce("qmm_splitk", tile, ksplit)
    M, N, K = 256, 256, 8192
    x, wq, s, b = affine_case(M, N, K, 64, 4, 2201)
    y = mq.quantized_matmul(dev_bf16(x).reshape(2, 128, K), dev_u32(wq), dev_bf16(s), dev_bf16(b))
    got = host_u16(y).reshape(M, N)
    assert max_rel(got, orc.qmm_t_affine(x, wq, s, b, 64, 4)) <= TOL
    again = host_u16(mq.quantized_matmul(dev_bf16(x).reshape(2, 128, K), dev_u32(wq), dev_bf16(s),
                                         dev_bf16(b))).reshape(M, N)
    np.testing.assert_array_equal(got, again)


@pytest.mark.parametrize("tile", [0, 1, 2, 4, 5, 6, 7, 8])
def test_mxfp4_qmm_vs_oracle(monkeypatch, tile):
    setknob(monkeypatch, "MLXQ_QMM_TILE", str(tile))
    announce("qmm_mxfp4", tile)
    M, N, K = 192, 576, 2880
    x, wq, sc = mxfp4_case(M, N, K, 2301)
    got = host_u16(mq.quantized_matmul(dev_bf16(x), dev_u32(wq), dev_u8(sc), None, True, 32, 4, "mxfp4"))
    assert max_rel(got, orc.fp_qmm_t_mxfp4(x, wq, sc)) <= TOL


def test_k_not_multiple_of_64_uses_row_segments():
    announce("qmm_fallback_k")
    M, N, K = 96, 128, 2592
    x, wq, s, b = affine_case(M, N, K, 32, 4, 2401)
    assert max_rel(run(x, wq, s, b, 32, 4), orc.qmm_t_affine(x, wq, s, b, 32, 4)) <= TOL


@pytest.mark.parametrize("tile", [-1])
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M", [512, 2048])
@pytest.mark.parametrize("N,K", [(14336, 4096), (4096, 14336)])
def test_llama_prefill_shapes_vs_dequant_fp32(monkeypatch, tile, bits, M, N, K):
    # full size: reference = float32 product of the bit-exact dequantized weights
    setknob(monkeypatch, "MLXQ_QMM_TILE", str(tile))
    announce("qmm_llama", tile, bits, M, N, K)
    g = torch.Generator(device="cuda").manual_seed(2500 + M + N + bits)
    w = (torch.randn(N, K, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
    wq, s, b = mq.quantize(w, 64, bits)
    wd = mq.dequantize(wq, s, b, 64, bits).float()
    y = mq.quantized_matmul(x, wq, s, b, True, 64, bits).float()
    ref = x.float() @ wd.t()
    err = float((y - ref).abs().max() / ref.abs().max())
    assert err <= TOL, err


@pytest.mark.parametrize("mode", ["affine4", "affine8", "mxfp4", "float16"])
@pytest.mark.parametrize("M,N", [(2048, 12288), (1536, 12288), (1280, 14336), (1999, 12200)])
def test_two_launch_tail_round_bitwise(monkeypatch, mode, M, N):
    # More 256 x 256 tiles than CUs (256 on MI355X) with a part-full last
    # round: whole tile columns in full rounds, the columns left as one round
    # of 256 x 128 tiles (1999 x 12200: ragged last row and column tiles).
    # Each output is the same MFMA sequence either way, so the result is
    # bitwise the single-launch plan's (MLXQ_QMM_MIX=0); the whole result is
    # checked against a float32 product of the bit-exact dequantized weights.
    K = 1024
    announce("qmm_mix", mode, M, N)
    setknob(monkeypatch, "MLXQ_QMM_STREAMK", "0")  # 1536 and 1280 rows would take stream-K
    g = torch.Generator(device="cuda").manual_seed(2600 + M)
    dt = torch.float16 if mode == "float16" else torch.bfloat16
    w = (torch.randn(N, K, device="cuda", generator=g) * 0.02).to(dt)
    x = torch.randn(M, K, device="cuda", generator=g).to(dt)
    if mode == "mxfp4":
        wq, s = mq.quantize(w, 32, 4, "mxfp4")
        args, gs, bits, md = (wq, s, None), 32, 4, "mxfp4"
    else:
        bits = 8 if mode == "affine8" else 4
        wq, s, b = mq.quantize(w, 64, bits)
        args, gs, md = (wq, s, b), 64, "affine"
    mixed = mq.quantized_matmul(x, *args, True, gs, bits, md)
    setknob(monkeypatch, "MLXQ_QMM_MIX", "0")
    single = mq.quantized_matmul(x, *args, True, gs, bits, md)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host_u16(mixed), host_u16(single))
    wd = mq.dequantize(*args, gs, bits, md).float()
    ref = x.float() @ wd.t()
    err = float((mixed.float() - ref).abs().max() / ref.abs().max())
    assert err <= TOL, err


@pytest.mark.parametrize("tile", [-1, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("mode,gs,N,K", [("affine4", 64, 579, 2880), ("affine8", 128, 631, 5504),
                                         ("affine4", 64, 243, 1344), ("mxfp4", 32, 695, 64),
                                         ("mxfp4", 32, 1215, 1344), ("float16", 64, 469, 2624)])
def test_scale_rows_ending_inside_a_dword(monkeypatch, tile, mode, gs, N, K):
    # N odd and K / gs odd (or 1-byte mxfp4 scales): the scale and bias
    # buffers end inside a dword, which a bounds-checked dword load would
    # read as 0 whole; the last weight row's last groups must still count
    # (every output column, the last one included, against the oracle)
    setknob(monkeypatch, "MLXQ_QMM_TILE", str(tile))
    announce("qmm_scale_tail", tile, mode, gs, N, K)
    M = 40
    if mode == "mxfp4":
        x, wq, sc = mxfp4_case(M, N, K, 3300 + N)
        y = host_u16(mq.quantized_matmul(dev_bf16(x), dev_u32(wq), dev_u8(sc), None, True, 32, 4, "mxfp4"))
        want = orc.fp_qmm_t_mxfp4(x, wq, sc)
    elif mode == "float16":
        g = torch.Generator().manual_seed(3400 + N)
        xv = torch.randn(M, K, generator=g).to(torch.float16)
        w = (torch.randn(N, K, generator=g) * 0.02).to(torch.float16).cuda()
        wq_, s_, b_ = mq.quantize(w, gs, 4)
        yt = mq.quantized_matmul(xv.cuda(), wq_, s_, b_, True, gs, 4).float()
        ref = xv.float().cuda() @ mq.dequantize(wq_, s_, b_, gs, 4).float().t()
        col = (yt[:, -1] - ref[:, -1]).abs().max() / ref.abs().max()
        assert float(col) <= TOL and float((yt - ref).abs().max() / ref.abs().max()) <= TOL
        return
    else:
        bits = 8 if mode == "affine8" else 4
        x, wq, s, b = affine_case(M, N, K, gs, bits, 3500 + N)
        y = host_u16(mq.quantized_matmul(dev_bf16(x), dev_u32(wq), dev_bf16(s), dev_bf16(b), True, gs, bits))
        want = orc.qmm_t_affine(x, wq, s, b, gs, bits)
    assert max_rel(y[:, -1:], want[:, -1:]) <= TOL
    assert max_rel(y, want) <= TOL
