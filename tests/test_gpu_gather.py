"""GPU parity: gather_qmm (MoE experts) on gfx950 vs the CPU oracle's
restatement of `_bs_qmm_dispatch_typed` / `fp_bs_qmm_dispatch_mode`
(overlays/cpu/mlx/backend/cpu/quantized.cpp:764-813, 875-914).

Cases follow the reference's call sites and tests: gpt-oss decode (x
[T,1,1,K], rhs [T,4], unsorted), the sorted path (x [B,1,K], rhs sorted [B],
src/models/switch_layers.rs:2180-2203), broadcast index shapes
(tests/rocm_gather_qmm_expert_batched.rs:30-37), partial tiles (N=516), and
bitwise repeatability of sorted runs (same file :46).
"""
import numpy as np
import pytest
import torch

import mlxcel_amd as mq
import oracle as orc
from helpers import TOL, announce, dev_bf16, dev_u32, dev_u8, host_u16, max_rel, setknob

pytestmark = pytest.mark.gpu


def topk_ids(T, E, k, seed):
    rng = np.random.default_rng(seed)
    return np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.uint32)


def mx_experts(E, N, K, seed):
    w = orc.normal_bf16((E, N, K), 0.02, seed)
    return orc.mxfp4_quantize(w)


def affine_experts(E, N, K, seed, gs=64, bits=4):
    w = orc.normal_bf16((E, N, K), 0.02, seed)
    return orc.affine_quantize(w, gs, bits)


@pytest.mark.parametrize("T", [1, 4, 16])
def test_mxfp4_decode_unsorted(T):
    announce("gather_mxfp4_unsorted", T)
    E, N, K = 32, 576, 2880
    wq, sc = mx_experts(E, N, K, 900)
    x = orc.normal_bf16((T, 1, 1, K), 1.0, 901 + T)
    ids = topk_ids(T, E, 4, 902 + T)
    got = host_u16(mq.gather_qmm(dev_bf16(x), dev_u32(wq), dev_u8(sc), None, None,
                                 torch.from_numpy(ids.astype(np.int32)).cuda(), True, 32, 4, "mxfp4"))
    assert got.shape == (T, 4, 1, N)
    lhs = np.repeat(np.arange(T, dtype=np.uint32), 4)
    want = orc.gather_qmm_t(x.reshape(T, 1, K), wq, sc, None, lhs, ids.reshape(-1), mode="mxfp4")
    assert max_rel(got.reshape(T * 4, 1, N), want) <= TOL


@pytest.mark.parametrize("T", [16, 64])
def test_mxfp4_sorted(T):
    announce("gather_mxfp4_sorted", T)
    E, N, K = 32, 516, 2880  # N=516: partial column tile
    wq, sc = mx_experts(E, N, K, 910)
    ids = topk_ids(T, E, 4, 911 + T).reshape(-1)
    order = np.argsort(ids, kind="stable")
    x = orc.normal_bf16((T, 1, K), 1.0, 912 + T)
    xs = x[order // 4]  # gather_sort: rows in expert order
    rhs = ids[order]
    X, W, S, R = dev_bf16(xs), dev_u32(wq), dev_u8(sc), dev_u32(rhs)
    got = host_u16(mq.gather_qmm(X, W, S, None, None, R, True, 32, 4, "mxfp4", sorted_indices=True))
    again = host_u16(mq.gather_qmm(X, W, S, None, None, R, True, 32, 4, "mxfp4", sorted_indices=True))
    np.testing.assert_array_equal(got, again)
    want = orc.gather_qmm_t(xs, wq, sc, None, np.arange(T * 4, dtype=np.uint32), rhs, mode="mxfp4")
    assert max_rel(got, want) <= TOL
    # the unsorted call on the same pairs gives the same rows within tolerance
    # (tests/rocm_gather_qmm_expert_batched.rs:26-35 holds them to a tolerance
    # too; the sorted call runs equal experts together, which changes the
    # order of the fp32 sums)
    unsorted = host_u16(mq.gather_qmm(X, W, S, None, None, R, True, 32, 4, "mxfp4", sorted_indices=False))
    assert max_rel(unsorted, got) <= TOL


@pytest.mark.parametrize("bits", [4, 8])
def test_affine_gather_with_broadcast_indices(bits):
    announce("gather_affine_broadcast", bits)
    E, N, K, M = 6, 128, 512, 2
    wq, s, b = affine_experts(E, N, K, 920 + bits, 64, bits)
    x = orc.normal_bf16((3, M, K), 1.0, 921)
    lhs = np.array([[0], [2], [1]], np.int64)          # [3,1]
    rhs = np.array([5, 0, 3, 3], np.int32)              # [4] -> broadcast [3,4]
    got = host_u16(mq.gather_qmm(dev_bf16(x), dev_u32(wq), dev_bf16(s), dev_bf16(b),
                                 torch.from_numpy(lhs).cuda(), torch.from_numpy(rhs).cuda(), True, 64, bits))
    assert got.shape == (3, 4, M, N)
    L = np.broadcast_to(lhs, (3, 4)).reshape(-1).astype(np.uint32)
    Rr = np.broadcast_to(rhs, (3, 4)).reshape(-1).astype(np.uint32)
    want = orc.gather_qmm_t(x, wq, s, b, L, Rr, 64, bits)
    assert max_rel(got.reshape(12, M, N), want) <= TOL


def test_gather_default_lhs_is_arange():
    announce("gather_default_lhs")
    E, N, K = 4, 64, 256
    wq, s, b = affine_experts(E, N, K, 930)
    x = orc.normal_bf16((5, 1, K), 1.0, 931)
    rhs = np.array([3, 1, 1, 0, 2], np.uint32)
    got = host_u16(mq.gather_qmm(dev_bf16(x), dev_u32(wq), dev_bf16(s), dev_bf16(b), None, dev_u32(rhs)))
    want = orc.gather_qmm_t(x, wq, s, b, np.arange(5, dtype=np.uint32), rhs, 64, 4)
    assert max_rel(got, want) <= TOL


def test_gather_without_indices_is_quantized_matmul():
    announce("gather_no_indices")
    E, N, K = 1, 64, 256
    wq, s, b = affine_experts(E, N, K, 940)
    x = orc.normal_bf16((3, K), 1.0, 941)
    a = host_u16(mq.gather_qmm(dev_bf16(x), dev_u32(wq[0]), dev_bf16(s[0]), dev_bf16(b[0])))
    c = host_u16(mq.quantized_matmul(dev_bf16(x), dev_u32(wq[0]), dev_bf16(s[0]), dev_bf16(b[0])))
    np.testing.assert_array_equal(a, c)


@pytest.mark.parametrize("K", [1024, 1056])
@pytest.mark.parametrize("group", [0, 1])
@pytest.mark.parametrize("E,T,M,mode", [(32, 64, 1, "mxfp4"), (8, 40, 2, "affine"), (300, 50, 1, "affine"),
                                        (4, 16, 3, "mxfp4"), (2, 160, 1, "affine")])
def test_grouped_by_expert_matches_stack(monkeypatch, K, group, E, T, M, mode):
    # rows regrouped by expert on the device (MLXQ_GATHER_GROUP=1: the grouped
    # GEMM, or the MFMA skinny kernel when K is not a multiple of 64) and
    # per-entry segments (=0) both equal the stack of per-index matmuls
    # (CPUQ:792-812); E=2, T=160 gives segments of more than 64 rows
    if mode == "mxfp4" and K % 32:
        pytest.skip("mxfp4 needs K % 32 == 0")
    setknob(monkeypatch, "MLXQ_GATHER_GROUP", str(group))
    announce("gather_grouped", K, group, E, T, M, mode)
    N = 264
    rng = np.random.default_rng(1700 + E + T + M)
    x = orc.normal_bf16((T, M, K), 1.0, 1701 + T)
    rhs = rng.integers(0, E, size=(T, 2)).astype(np.int64)  # two experts per token, repeats likely
    lhs = np.repeat(np.arange(T)[:, None], 2, axis=1).astype(np.int32)
    if mode == "mxfp4":
        wq, sc = mx_experts(E, N, K, 1702 + E)
        got = host_u16(mq.gather_qmm(dev_bf16(x), dev_u32(wq), dev_u8(sc), None, torch.from_numpy(lhs).cuda(),
                                     torch.from_numpy(rhs).cuda(), True, 32, 4, "mxfp4"))
        want = orc.gather_qmm_t(x, wq, sc, None, lhs.reshape(-1).astype(np.uint32),
                                rhs.reshape(-1).astype(np.uint32), mode="mxfp4")
    else:
        gs = 64 if K % 64 == 0 else 32
        wq, s, b = affine_experts(E, N, K, 1703 + E, gs=gs)
        got = host_u16(mq.gather_qmm(dev_bf16(x), dev_u32(wq), dev_bf16(s), dev_bf16(b),
                                     torch.from_numpy(lhs).cuda(), torch.from_numpy(rhs).cuda(), True, gs, 4))
        want = orc.gather_qmm_t(x, wq, s, b, lhs.reshape(-1).astype(np.uint32), rhs.reshape(-1).astype(np.uint32),
                                group_size=gs)
    assert got.shape == (T, 2, M, N)
    assert max_rel(got.reshape(T * 2, M, N), want) <= TOL


def test_grouped_gather_is_deterministic_and_matches_per_entry(monkeypatch):
    announce("gather_grouped_det")
    E, N, K, T = 32, 576, 2880, 256
    wq, sc = mx_experts(E, N, K, 1800)
    ids = topk_ids(T, E, 4, 1801).reshape(-1)
    x = orc.normal_bf16((T, 1, K), 1.0, 1802)
    lhs = torch.from_numpy(np.repeat(np.arange(T), 4).astype(np.int32)).cuda()
    rhs = torch.from_numpy(ids.astype(np.int32)).cuda()
    args = (dev_bf16(x), dev_u32(wq), dev_u8(sc), None, lhs, rhs, True, 32, 4, "mxfp4")
    setknob(monkeypatch, "MLXQ_GATHER_GROUP", "1")
    g1 = host_u16(mq.gather_qmm(*args))
    g2 = host_u16(mq.gather_qmm(*args))
    np.testing.assert_array_equal(g1, g2)
    setknob(monkeypatch, "MLXQ_GATHER_GROUP", "0")
    per_entry = host_u16(mq.gather_qmm(*args))
    assert max_rel(g1, per_entry) <= TOL
    want = orc.gather_qmm_t(x, wq, sc, None, np.repeat(np.arange(T), 4).astype(np.uint32), ids.astype(np.uint32),
                            mode="mxfp4")
    assert max_rel(g1.reshape(T * 4, 1, N), want) <= TOL


@pytest.mark.parametrize("dtype", [torch.int32, torch.int64])
@pytest.mark.parametrize("case", ["topk_default_lhs", "explicit_lhs", "broadcast_rhs", "strided_rhs", "out_of_range"])
def test_direct_indices_match_index_prep(monkeypatch, dtype, case):
    # The decode kernels read contiguous 32/64-bit index arrays (and the
    # default lhs of the top-k pattern) in place; every other index layout
    # goes through index_prep.  Both routes must give the same bits.
    announce("gather_direct_indices", dtype, case)
    E, N, K, T = 8, 200, 1024, 5
    wq, s, b = affine_experts(E, N, K, 960)
    W, S, Bi = dev_u32(wq), dev_bf16(s), dev_bf16(b)
    ids = topk_ids(T, E, 3, 961)
    if case == "topk_default_lhs":
        x = dev_bf16(orc.normal_bf16((T, 1, 1, K), 1.0, 962))
        lhs, rhs = None, torch.from_numpy(ids.astype(np.int64)).to(dtype).cuda()
    elif case == "explicit_lhs":
        x = dev_bf16(orc.normal_bf16((T, 1, K), 1.0, 963))
        lhs = torch.from_numpy(np.repeat(np.arange(T), 3).reshape(T, 3)[:, ::-1].copy()).to(dtype).cuda()
        rhs = torch.from_numpy(ids.astype(np.int64)).to(dtype).cuda()
    elif case == "broadcast_rhs":
        x = dev_bf16(orc.normal_bf16((T, 3, 1, K), 1.0, 964))
        lhs, rhs = None, torch.from_numpy(ids[0].astype(np.int64)).to(dtype).cuda()  # [3] broadcast over T
    elif case == "strided_rhs":
        x = dev_bf16(orc.normal_bf16((T, 1, 1, K), 1.0, 965))
        full = torch.from_numpy(np.concatenate([ids, ids], 1).astype(np.int64)).to(dtype).cuda()
        lhs, rhs = None, full[:, ::2]  # non-contiguous view
    else:
        x = dev_bf16(orc.normal_bf16((T, 1, 1, K), 1.0, 966))
        bad = ids.astype(np.int64).copy()
        bad[0, 0], bad[2, 1] = 50, -1  # clamped to the last expert, like index_prep
        lhs, rhs = None, torch.from_numpy(bad).to(dtype).cuda()
    outs = []
    for direct in ("1", "0"):
        setknob(monkeypatch, "MLXQ_GATHER_DIRECT", direct)
        y = mq.gather_qmm(x, W, S, Bi, lhs, rhs, True, 64, 4)
        torch.cuda.synchronize()
        outs.append(host_u16(y))
    np.testing.assert_array_equal(outs[0], outs[1])
    if case == "topk_default_lhs":
        want = orc.gather_qmm_t(orc.normal_bf16((T, 1, K), 1.0, 962), wq, s, b,
                                np.repeat(np.arange(T, dtype=np.uint32), 3), ids.reshape(-1))
        assert max_rel(outs[0].reshape(T * 3, 1, N), want) <= TOL


@pytest.mark.parametrize("pattern", ["random_sorted", "one_expert", "pairs", "alternating", "unsorted"])
@pytest.mark.parametrize("dtype", [torch.int32, torch.int64])
def test_sorted_runs(monkeypatch, pattern, dtype):
    # the run path of sorted gathers (MLXQ_GATHER_RUNS=1): equal consecutive
    # experts form segments of up to 4 entries; every pattern must give the
    # per-entry result (oracle), with runs longer than 4, runs across
    # multiples of 4, a ragged tail (B = 37), and input that is not actually
    # sorted (the run path does not rely on the order)
    announce("gather_sorted_runs", pattern, dtype)
    E, N, K, B = 8, 264, 2048, 37
    rng = np.random.default_rng(970)
    # the run path; the expert-grouped path (the default for sorted mxfp4
    # gathers, test_sorted_grouped_mxfp4) relies on sorted_indices the way
    # the reference's sorted route does, and "pairs" (wrapping at E),
    # "alternating" and "unsorted" are not sorted
    setknob(monkeypatch, "MLXQ_GATHER_SORTED", "0")
    setknob(monkeypatch, "MLXQ_GATHER_RUNS", "1")
    if pattern == "random_sorted":
        rhs = np.sort(rng.integers(0, E, B))
    elif pattern == "one_expert":
        rhs = np.full(B, 5)
    elif pattern == "pairs":
        rhs = np.repeat(np.arange(B) // 2 % E, 1)
    elif pattern == "alternating":
        rhs = np.arange(B) % 2 * 3
    else:
        rhs = rng.integers(0, E, B)
    wq, sc = mx_experts(E, N, K, 971)
    x = orc.normal_bf16((B, 1, K), 1.0, 972)
    R = torch.from_numpy(rhs.astype(np.int64)).to(dtype).cuda()
    X, W, S = dev_bf16(x), dev_u32(wq), dev_u8(sc)
    got = host_u16(mq.gather_qmm(X, W, S, None, None, R, True, 32, 4, "mxfp4", sorted_indices=True))
    want = orc.gather_qmm_t(x, wq, sc, None, np.arange(B, dtype=np.uint32), rhs.astype(np.uint32), mode="mxfp4")
    assert max_rel(got, want) <= TOL
    again = host_u16(mq.gather_qmm(X, W, S, None, None, R, True, 32, 4, "mxfp4", sorted_indices=True))
    np.testing.assert_array_equal(got, again)
    setknob(monkeypatch, "MLXQ_GATHER_RUNS", "0")
    per_entry = host_u16(mq.gather_qmm(X, W, S, None, None, R, True, 32, 4, "mxfp4", sorted_indices=True))
    assert max_rel(per_entry, got) <= TOL


def test_sorted_runs_affine():
    announce("gather_sorted_runs_affine")
    E, N, K, B = 6, 200, 4096, 24
    rhs = np.sort(np.random.default_rng(973).integers(0, E, B)).astype(np.int32)
    wq, s, b = affine_experts(E, N, K, 974)
    x = orc.normal_bf16((B, 1, K), 1.0, 975)
    got = host_u16(mq.gather_qmm(dev_bf16(x), dev_u32(wq), dev_bf16(s), dev_bf16(b), None,
                                 torch.from_numpy(rhs).cuda(), True, 64, 4, sorted_indices=True))
    want = orc.gather_qmm_t(x, wq, s, b, np.arange(B, dtype=np.uint32), rhs.astype(np.uint32))
    assert max_rel(got, want) <= TOL


@pytest.mark.parametrize("fmt", ["mxfp4", "affine4", "affine8"])
@pytest.mark.parametrize("pattern", ["random_sorted", "one_expert", "skewed", "clamped_tail", "few_entries",
                                     "long"])
def test_sorted_expert_search(monkeypatch, fmt, pattern):
    # the expert-search form of the sorted run path (the default,
    # MLXQ_GATHER_RUNS=2, block-MFMA kernel): one workgroup row per expert
    # finds its entries by binary search and takes them 4 at a time.  Experts without entries, one expert holding all 37
    # entries (10 passes), a skewed spread, out-of-range ids at the end
    # (clamped to the last expert, which keeps the order), as many entries as
    # experts on a third of them, and 300 entries (searches of several
    # steps); bitwise the runs-of-4 result, within tolerance of the oracle
    announce("gather_sorted_expert_search", fmt, pattern)
    E, N, K, B = 8, 264, 2048, 37
    rng = np.random.default_rng(976)
    if pattern == "random_sorted":
        rhs = np.sort(rng.integers(0, E, B))
    elif pattern == "one_expert":
        rhs = np.full(B, 5)
    elif pattern == "skewed":
        rhs = np.sort(np.minimum(rng.geometric(0.3, B) - 1, E - 1))
    elif pattern == "clamped_tail":
        rhs = np.sort(rng.integers(0, E, B))
        rhs[-5:] = 1000
    elif pattern == "few_entries":
        E, B = 12, 12  # as many entries as experts (the search's limit), most on a few experts
        rhs = np.sort(rng.choice(4, B) * 3)
    else:
        B = 300
        rhs = np.sort(rng.integers(0, E, B))
    x = orc.normal_bf16((B, 1, K), 1.0, 977)
    R = torch.from_numpy(rhs.astype(np.int64)).cuda()
    if fmt == "mxfp4":
        wq, sc = mx_experts(E, N, K, 978)
        args, s, b, gs, bits, mode = (dev_u32(wq), dev_u8(sc), None), sc, None, 32, 4, "mxfp4"
    else:
        bits = 4 if fmt == "affine4" else 8
        wq, s, b = affine_experts(E, N, K, 979, bits=bits)
        args, sc, gs, mode = (dev_u32(wq), dev_bf16(s), dev_bf16(b)), s, 64, "affine"
    X = dev_bf16(x)
    setknob(monkeypatch, "MLXQ_GATHER_SORTED", "0")
    setknob(monkeypatch, "MLXQ_GATHER_GROUP", "0")
    setknob(monkeypatch, "MLXQ_GATHER_RUNS", "2")
    got = host_u16(mq.gather_qmm(X, *args, None, R, True, gs, bits, mode, sorted_indices=True))
    want = orc.gather_qmm_t(x, wq, sc, b, np.arange(B, dtype=np.uint32),
                            np.minimum(rhs, E - 1).astype(np.uint32), gs, bits, mode=mode)
    assert max_rel(got, want) <= TOL
    setknob(monkeypatch, "MLXQ_GATHER_RUNS", "1")
    runs = host_u16(mq.gather_qmm(X, *args, None, R, True, gs, bits, mode, sorted_indices=True))
    np.testing.assert_array_equal(got, runs)


@pytest.mark.parametrize("pattern", ["uniform", "one_expert", "skewed", "clamped_tail"])
@pytest.mark.parametrize("dtype", [torch.int32, torch.int64])
def test_sorted_grouped_mxfp4(pattern, dtype):
    # the expert-grouped kernel (qmm_group.hip): 1024 sorted entries; experts
    # with no rows, with more than 64 rows (chunks of 64), all rows on one
    # expert, and out-of-range indices at the end (clamped to the last expert,
    # which keeps the order); N = 516 ends inside a 128-row block and
    # K = 2880 inside a 128-k window
    announce("gather_sorted_grouped", pattern, dtype)
    E, N, K, B = 32, 516, 2880, 1024
    rng = np.random.default_rng(980)
    if pattern == "uniform":
        rhs = np.sort(rng.integers(0, E, B))
    elif pattern == "one_expert":
        rhs = np.full(B, 7)
    elif pattern == "skewed":
        rhs = np.sort(np.minimum(rng.geometric(0.15, B) - 1, E - 1))
    else:
        rhs = np.sort(rng.integers(0, E, B))
        rhs[-20:] = 1000
    wq, sc = mx_experts(E, N, K, 981)
    x = orc.normal_bf16((B, 1, K), 1.0, 982)
    R = torch.from_numpy(rhs.astype(np.int64)).to(dtype).cuda()
    X, W, S = dev_bf16(x), dev_u32(wq), dev_u8(sc)
    got = host_u16(mq.gather_qmm(X, W, S, None, None, R, True, 32, 4, "mxfp4", sorted_indices=True))
    assert got.shape == (B, 1, N)
    want = orc.gather_qmm_t(x, wq, sc, None, np.arange(B, dtype=np.uint32),
                            np.minimum(rhs, E - 1).astype(np.uint32), mode="mxfp4")
    assert max_rel(got, want) <= TOL
    again = host_u16(mq.gather_qmm(X, W, S, None, None, R, True, 32, 4, "mxfp4", sorted_indices=True))
    np.testing.assert_array_equal(got, again)


@pytest.mark.parametrize("K", [96, 128, 256, 4096])
def test_sorted_grouped_mxfp4_k(monkeypatch, K):
    # the expert-grouped kernel's ring at other reduction lengths: K below
    # 384 (fewer 128-k blocks than the ring's 3-ahead prologue: the blocks
    # past the last issue dead loads and skip their MFMAs), K = 96 (one
    # partial block), K = 128 / 256 / 4096 (multiples of 128: no tail window)
    announce("gather_sorted_grouped_k", K)
    E, N, B = 8, 256, 256
    rhs = np.sort(np.random.default_rng(990 + K).integers(0, E, B))
    wq, sc = mx_experts(E, N, K, 991 + K)
    x = orc.normal_bf16((B, 1, K), 1.0, 992 + K)
    X, W, S = dev_bf16(x), dev_u32(wq), dev_u8(sc)
    R = torch.from_numpy(rhs.astype(np.int32)).cuda()
    got = host_u16(mq.gather_qmm(X, W, S, None, None, R, True, 32, 4, "mxfp4", sorted_indices=True))
    want = orc.gather_qmm_t(x, wq, sc, None, np.arange(B, dtype=np.uint32), rhs.astype(np.uint32), mode="mxfp4")
    assert max_rel(got, want) <= TOL
    # the same entries on the routes that do not rely on the order agree
    # within tolerance (a different fp32 summation order)
    setknob(monkeypatch, "MLXQ_GATHER_SORTED", "0")
    setknob(monkeypatch, "MLXQ_GATHER_RUNS", "0")
    per_entry = host_u16(mq.gather_qmm(X, W, S, None, None, R, True, 32, 4, "mxfp4", sorted_indices=True))
    assert max_rel(per_entry, got) <= TOL


@pytest.mark.parametrize("N,K", [(256, 2880), (100, 2880), (516, 96), (130, 96), (256, 4160)])
def test_sorted_grouped_scale_table(monkeypatch, N, K):
    # the expert-grouped kernel's scale sources: an LDS table staged with
    # 16-byte direct loads (256 x 2880: every expert's 256 * 90 scale bytes a
    # multiple of 16), with 4-byte loads (100 x 2880: 9000 bytes; 516 x 96),
    # and per-block byte loads where the table does not apply (130 x 96: 390
    # bytes per expert, not 4-aligned; K = 4160: 130 bytes per row, past the
    # 128-byte table rows).  Each is bitwise the per-block loads' result
    # (MLXQ_GATHER_SCALE_TABLE=0) and within tolerance of the oracle; a
    # partial last 128-row block reads 0 for rows past N.
    announce("gather_sorted_grouped_scales", N, K)
    E, B = 8, 512
    rhs = np.sort(np.random.default_rng(1990 + N + K).integers(0, E, B))
    wq, sc = mx_experts(E, N, K, 1991 + N + K)
    x = orc.normal_bf16((B, 1, K), 1.0, 1992 + N + K)
    X, W, S = dev_bf16(x), dev_u32(wq), dev_u8(sc)
    R = torch.from_numpy(rhs.astype(np.int32)).cuda()
    got = host_u16(mq.gather_qmm(X, W, S, None, None, R, True, 32, 4, "mxfp4", sorted_indices=True))
    want = orc.gather_qmm_t(x, wq, sc, None, np.arange(B, dtype=np.uint32), rhs.astype(np.uint32), mode="mxfp4")
    assert max_rel(got, want) <= TOL
    setknob(monkeypatch, "MLXQ_GATHER_SCALE_TABLE", "0")
    per_block = host_u16(mq.gather_qmm(X, W, S, None, None, R, True, 32, 4, "mxfp4", sorted_indices=True))
    np.testing.assert_array_equal(got, per_block)


@pytest.mark.parametrize("N,K", [(2880, 2880), (200, 2880), (516, 96), (256, 4096), (130, 96), (256, 4160)])
def test_sorted_grouped_192_row_blocks(monkeypatch, N, K):
    # 192-row workgroups (3 weight tiles per wave, chunks of 48 activation
    # rows, scales from the LDS table) against 128-row ones
    # (MLXQ_GATHER_TILES=3 / 2): the same MFMA sequence per output, so the
    # same bits.  512 entries over 8 experts put ~64 rows on an expert, so
    # chunks of 48 repeat; partial last row blocks (200, 516, 130 rows); 130 x
    # 96 and K = 4160 have no scale table and keep 128-row workgroups.
    announce("gather_sorted_grouped_192", N, K)
    E, B = 8, 512
    rhs = np.sort(np.random.default_rng(2990 + N + K).integers(0, E, B))
    wq, sc = mx_experts(E, N, K, 2991 + N + K)
    x = orc.normal_bf16((B, 1, K), 1.0, 2992 + N + K)
    X, W, S = dev_bf16(x), dev_u32(wq), dev_u8(sc)
    R = torch.from_numpy(rhs.astype(np.int32)).cuda()
    outs = {}
    for tiles in ("2", "3"):
        setknob(monkeypatch, "MLXQ_GATHER_TILES", tiles)
        outs[tiles] = host_u16(mq.gather_qmm(X, W, S, None, None, R, True, 32, 4, "mxfp4", sorted_indices=True))
    np.testing.assert_array_equal(outs["3"], outs["2"])
    want = orc.gather_qmm_t(x, wq, sc, None, np.arange(B, dtype=np.uint32), rhs.astype(np.uint32), mode="mxfp4")
    assert max_rel(outs["3"], want) <= TOL
