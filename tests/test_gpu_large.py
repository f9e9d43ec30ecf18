"""GPU parity at sizes past the limits of one launch: operands of 2 GiB and
more, gathers with more index entries than a grid dimension holds, and
batched weights with more rows per batch than the decode kernels stage.

The reference takes all of these: it indexes activations in elements
(overlays/rocm/mlx/backend/rocm/quantized/qmv_tiled_kernel.hip:56-64), its
gather dispatch and CPU gather have no entry cap (rocm/quantized/qmm.hip:6590,
overlays/cpu/mlx/backend/cpu/quantized.cpp:764-813), and it folds any batch of
rows (qmm.hip:3606-3620).  Here the library splits such calls into launches
below the limits; each test checks the split call bitwise against calls that
need no split, and against the CPU oracle.
"""
import numpy as np
import pytest
import torch

import mlxcel_amd as mq
import oracle as orc
from helpers import TOL, announce, dev_bf16, dev_u32, dev_u8, host_u16, max_rel

pytestmark = pytest.mark.gpu


def test_quantized_matmul_activation_over_2gib():
    # x: 135,000 x 8192 bf16 = 2.21 GB (past the 2 GiB of one buffer
    # resource): the call runs as two row chunks below it.  The same rows as two
    # half-size calls (each 1.1 GB, no split) give the same bits.
    M, N, K = 135_000, 64, 8192
    announce("large_x", M, N, K)
    w = orc.normal_bf16((N, K), 0.02, 4100)
    wq, s, b = orc.affine_quantize(w, 64, 4)
    W, S, B = dev_u32(wq), dev_bf16(s), dev_bf16(b)
    g = torch.Generator(device="cuda").manual_seed(4101)
    X = torch.randn(M, K, device="cuda", generator=g, dtype=torch.float32).to(torch.bfloat16)
    assert X.numel() * 2 >= 1 << 31
    full = host_u16(mq.quantized_matmul(X, W, S, B, True, 64, 4))
    h = M // 2
    lo = host_u16(mq.quantized_matmul(X[:h], W, S, B, True, 64, 4))
    hi = host_u16(mq.quantized_matmul(X[h:], W, S, B, True, 64, 4))
    np.testing.assert_array_equal(full, np.concatenate([lo, hi]))
    # rows on both sides of the chunk boundary and at the ends, against the oracle
    rows = np.r_[0:4, 67_580:67_588, M - 4:M]  # chunks of 67,584 rows
    xs = host_u16(X[torch.from_numpy(rows).cuda()])
    assert max_rel(full[rows], orc.qmm_t_affine(xs, wq, s, b, 64, 4)) <= TOL


def sorted_ids(B, E, seed):
    return np.sort(np.random.default_rng(seed).integers(0, E, B)).astype(np.uint32)


@pytest.mark.parametrize("case", ["mxfp4_sorted", "affine_unsorted", "affine_explicit_lhs"])
def test_gather_more_entries_than_one_launch(case):
    # 70,000 index entries (one launch covers at most 65,528): the entries
    # run in chunks over flat copies of the indices
    B, E, N, K = 70_000, 8, 64, 256
    announce("large_gather", case, B)
    rng = np.random.default_rng(4200)
    if case == "mxfp4_sorted":
        w = orc.normal_bf16((E, N, K), 0.02, 4201)
        wq, sc = orc.mxfp4_quantize(w)
        args, s, b, gs, mode = (dev_u32(wq), dev_u8(sc), None), sc, None, 32, "mxfp4"
    else:
        w = orc.normal_bf16((E, N, K), 0.02, 4202)
        wq, s, b = orc.affine_quantize(w, 64, 4)
        args, gs, mode = (dev_u32(wq), dev_bf16(s), dev_bf16(b)), 64, "affine"
    if case == "affine_explicit_lhs":
        X_rows = 1000
        x = orc.normal_bf16((X_rows, 1, K), 1.0, 4203)
        lhs = rng.integers(0, X_rows, B).astype(np.int32)
        rhs = rng.integers(0, E, B).astype(np.int32)
        L, R = torch.from_numpy(lhs).cuda(), torch.from_numpy(rhs).cuda()
    else:
        x = orc.normal_bf16((B, 1, K), 1.0, 4204)
        lhs = np.arange(B, dtype=np.int32)
        rhs = sorted_ids(B, E, 4205) if case == "mxfp4_sorted" else rng.integers(0, E, B).astype(np.uint32)
        L, R = None, torch.from_numpy(rhs.astype(np.int32)).cuda()
    srt = case == "mxfp4_sorted"
    X = dev_bf16(x)
    got = host_u16(mq.gather_qmm(X, *args, L, R, True, gs, 4, mode, sorted_indices=srt))
    assert got.shape == (B, 1, N)
    want = orc.gather_qmm_t(x, wq, s, b, lhs.astype(np.uint32), rhs.astype(np.uint32), gs, 4, mode=mode)
    assert max_rel(got, want) <= TOL
    # the first 65,528 entries alone (one launch) give the same bits
    c = 65_528
    if L is None:
        part = host_u16(mq.gather_qmm(X[:c], *args, None, R[:c], True, gs, 4, mode, sorted_indices=srt))
    else:
        part = host_u16(mq.gather_qmm(X, *args, L[:c], R[:c], True, gs, 4, mode, sorted_indices=srt))
    np.testing.assert_array_equal(got[:c], part)


@pytest.mark.parametrize("xbatch", [(3,), (1,)], ids=["same_batch", "broadcast_x"])
def test_batched_weights_many_rows(xbatch):
    # w [3, N, K/8] with 64 activation rows per batch (more than the decode
    # kernels stage): the general kernel over the default gather indices
    E, M, N, K = 3, 64, 200, 512
    announce("batched_w_rows", xbatch, M)
    w = orc.normal_bf16((E, N, K), 0.02, 4300)
    wq, s, b = orc.affine_quantize(w, 64, 4)
    x = orc.normal_bf16(xbatch + (M, K), 1.0, 4301)
    got = host_u16(mq.quantized_matmul(dev_bf16(x), dev_u32(wq), dev_bf16(s), dev_bf16(b), True, 64, 4))
    assert got.shape == (E, M, N)
    for e in range(E):
        xe = x[e if xbatch[0] == E else 0]
        assert max_rel(got[e], orc.qmm_t_affine(xe, wq[e], s[e], b[e], 64, 4)) <= TOL


@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("M", [17, 40, 64])
def test_rows_per_matrix_over_the_skinny_lds(gs, M):
    # batched weights and gathered matrices with 17-64 activation rows each:
    # at 4-bit g128 the skinny kernel's activation tile of 64 rows does not
    # fit in LDS, so those calls run on the general kernel (or in smaller
    # row segments) instead of being refused; every group size against the
    # oracle
    E, N, K = 3, 200, 2048
    announce("rows_over_lds", gs, M)
    w = orc.normal_bf16((E, N, K), 0.02, 4400 + gs + M)
    wq, s, b = orc.affine_quantize(w, gs, 4)
    x = orc.normal_bf16((E, M, K), 1.0, 4401 + gs + M)
    W, S, B_ = dev_u32(wq), dev_bf16(s), dev_bf16(b)
    got = host_u16(mq.quantized_matmul(dev_bf16(x), W, S, B_, True, gs, 4))
    for e in range(E):
        assert max_rel(got[e], orc.qmm_t_affine(x[e], wq[e], s[e], b[e], gs, 4)) <= TOL
    rhs = np.array([2, 0, 1, 2, 0], dtype=np.int32)
    lhs = np.array([1, 1, 0, 2, 2], dtype=np.int32)
    g = host_u16(mq.gather_qmm(dev_bf16(x), W, S, B_, torch.from_numpy(lhs).cuda(), torch.from_numpy(rhs).cuda(),
                               True, gs, 4))
    want = orc.gather_qmm_t(x, wq, s, b, lhs.astype(np.uint32), rhs.astype(np.uint32), gs, 4)
    assert max_rel(g, want) <= TOL
