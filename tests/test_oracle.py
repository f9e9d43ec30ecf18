"""Pins the CPU oracle (oracle/mlxq_oracle.c) before it is trusted as the checker.

Each test checks the oracle against something it did not compute itself:
closed-form known answers (tests/golden/kat.npz, tests/golden/make_golden.py),
torch's independent bf16 arithmetic, float64 references built from the
dequantized weights (the reference's own method,
src/lib/mlxcel-core/src/cpu_qmm_accum_tests.rs:237-287 with its
2x-store-rounding-floor rule, :103-108, :162-183), one-hot / all-ones
activations whose products are exact, and quantizer invariants.
"""
import os

import numpy as np
import pytest
import torch

GOLD = os.path.join(os.path.dirname(__file__), "golden", "kat.npz")


@pytest.fixture(scope="module")
def kat():
    return np.load(GOLD)


def bf16_from_torch(x):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16).view(torch.int16).numpy().astype(np.uint16)


def torch_from_bits(b):
    return torch.from_numpy(np.ascontiguousarray(b).astype(np.int16)).view(torch.bfloat16)


def codes_bytestream(wq, bits, K):
    """Code i of each row = bits [bits*i, bits*i+bits) of the row's little-endian
    byte stream (cpu_qmm_accum_tests.rs:73-84)."""
    by = np.ascontiguousarray(wq).view(np.uint8).reshape(wq.shape[0], -1)
    bitsarr = np.unpackbits(by, axis=1, bitorder="little")[:, : K * bits]
    bitsarr = bitsarr.reshape(wq.shape[0], K, bits).astype(np.uint32)
    return (bitsarr << np.arange(bits, dtype=np.uint32)).sum(-1)


# ---- bf16 conversion ---------------------------------------------------------

def test_bf16_rne_matches_torch(orc):
    rng = np.random.default_rng(1)
    x = np.concatenate([
        rng.standard_normal(100000).astype(np.float32) * 10 ** rng.uniform(-30, 30, 100000).astype(np.float32),
        # exact halfway points between bf16 neighbours
        (np.arange(1, 20000, dtype=np.uint32) << 16 | 0x8000).view(np.float32),
        np.array([0.0, -0.0, np.inf, -np.inf, 3.4e38, 1e-45], np.float32),
    ])
    np.testing.assert_array_equal(orc.f32_to_bf16(x), bf16_from_torch(x))
    assert orc.f32_to_bf16(np.array([np.nan], np.float32))[0] == 0x7FC0


# ---- affine quantize ---------------------------------------------------------

@pytest.mark.parametrize("bits", [2, 4, 6, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_affine_quantize_known_answers(orc, kat, bits, gs):
    wq, s, b = orc.affine_quantize(kat[f"ramp_w_b{bits}_g{gs}"], gs, bits)
    np.testing.assert_array_equal(wq, kat[f"ramp_wq_b{bits}_g{gs}"])
    np.testing.assert_array_equal(s, kat[f"ramp_s_b{bits}_g{gs}"])
    np.testing.assert_array_equal(b, kat[f"ramp_b_b{bits}_g{gs}"])


@pytest.mark.parametrize("bits", [4, 6, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_affine_quantize_invariants(orc, bits, gs):
    w = orc.normal_bf16((64, 512), 0.02, 7 + bits + gs)
    wq, s, b = orc.affine_quantize(w, gs, bits)
    wf = orc.bf16_to_f32(w).reshape(64, -1, gs)
    sf = orc.bf16_to_f32(s)[..., None]
    d2 = orc.bf16_to_f32(orc.affine_dequantize(wq, s, b, gs, bits, 2)).reshape(64, -1, gs)
    # the edge (w_min if |w_min| > |w_max| else w_max, quantized.cpp:1267-1277)
    # gets code 0 and dequantizes to itself
    wmin, wmax = wf.min(-1, keepdims=True), wf.max(-1, keepdims=True)
    edge = np.where(np.abs(wmin) > np.abs(wmax), wmin, wmax)
    at_edge = wf == edge
    np.testing.assert_array_equal(d2[at_edge], wf[at_edge])
    # Sanity bound: the edge snapping (scale = edge / rint(edge / scale0)) can
    # leave the far extreme clamped up to about one step away, on top of the
    # half-step rounding and the bf16 roundings of scale, q*s and the result.
    qmax = (1 << bits) - 1
    err = np.abs(d2 - wf)
    assert np.all(err <= np.abs(sf) * (1.5 + 2 * qmax * 2.0 ** -9) + np.abs(wf) * 2.0 ** -8 + 1e-12)


HAND = sorted({k[len("hand_w_"):] for k in np.load(GOLD).files if k.startswith("hand_w_")})


@pytest.mark.parametrize("case", HAND)
def test_affine_quantize_hand_cases(orc, kat, case):
    # worked by hand in float32 steps (tests/golden/make_golden.py HAND_CASES):
    # bf16-unrepresentable scales, rint ties of both parities in the codes and
    # in q0, the |w_min| == |w_max| branch, a clamped far extreme
    bits = int(case.rsplit("_b", 1)[1])
    wq, s, b = orc.affine_quantize(kat[f"hand_w_{case}"], 32, bits)
    np.testing.assert_array_equal(codes_bytestream(wq, bits, 32), codes_bytestream(kat[f"hand_wq_{case}"], bits, 32))
    np.testing.assert_array_equal(s, kat[f"hand_s_{case}"])
    np.testing.assert_array_equal(b, kat[f"hand_b_{case}"])


def numpy_affine_quantize(wf, gs, bits):
    """MLX's CPU affine quantizer (quantized.cpp:1251-1303) restated with
    vectorised numpy float32 arithmetic (IEEE division, np.rint = round half to
    even, like std::rint): codes, float32 scale and bias per group."""
    g = wf.reshape(-1, gs).astype(np.float32)
    T = np.float32((1 << bits) - 1)
    mn, mx = g.min(1), g.max(1)
    mask = np.abs(mn) > np.abs(mx)
    s0 = np.maximum((mx - mn) / T, np.float32(1e-7))
    s = np.where(mask, s0, -s0)
    edge = np.where(mask, mn, mx)
    q0 = np.rint(edge / s)
    nz = q0 != 0
    s = np.where(nz, edge / np.where(nz, q0, np.float32(1)), s).astype(np.float32)
    b = np.where(nz, edge, np.float32(0)).astype(np.float32)
    codes = np.clip(np.rint((g - b[:, None]) / s[:, None]), 0, T)
    return codes.astype(np.uint32).reshape(wf.shape), s, b


@pytest.mark.parametrize("bits", [2, 4, 6, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_affine_quantize_matches_numpy_restatement(orc, bits, gs):
    # random bf16 groups at scales from 1e-4 to 1e2, all-positive and
    # all-negative groups, constant and all-zero groups
    rng = np.random.default_rng(100 * bits + gs)
    rows, K = 48, 512
    x = rng.standard_normal((rows, K)).astype(np.float32)
    x *= (10.0 ** rng.uniform(-4, 2, (rows, 1))).astype(np.float32)
    x[8:12] = np.abs(x[8:12])
    x[12:16] = -np.abs(x[12:16])
    x[16, :gs] = 0.375
    x[17, :gs] = 0.0
    x[18, :gs] = -x[18, 0]
    w = bf16_from_torch(x)
    wf = torch_from_bits(w).float().numpy()
    codes, s, b = numpy_affine_quantize(wf, gs, bits)
    wq, so, bo = orc.affine_quantize(w, gs, bits)
    np.testing.assert_array_equal(codes_bytestream(wq, bits, K), codes)
    np.testing.assert_array_equal(so.reshape(-1), bf16_from_torch(s))
    np.testing.assert_array_equal(bo.reshape(-1), bf16_from_torch(b))


def test_affine_packing_is_little_endian_bitstream(orc):
    w = orc.normal_bf16((8, 256), 0.02, 11)
    for bits in (2, 4, 6, 8):
        wq, s, b = orc.affine_quantize(w, 64, bits)
        codes = codes_bytestream(wq, bits, 256).astype(np.float32)
        # D2 rebuilt from byte-stream codes with torch's bf16 ops
        st = torch_from_bits(s).repeat_interleave(64, dim=1)
        bt = torch_from_bits(b).repeat_interleave(64, dim=1)
        ref = (torch.from_numpy(codes).to(torch.bfloat16) * st) + bt
        np.testing.assert_array_equal(orc.affine_dequantize(wq, s, b, 64, bits, 2),
                                      ref.view(torch.int16).numpy().astype(np.uint16))


def test_six_bit_pack_layout_known_answer(orc):
    # the 3-byte pack of 4 codes as the reference's kernels read it
    # (mlx_cxx_kernels.cpp:3136-3151): v0 = b0 & 0x3f, v1 = (b0 >> 6) | ((b1 & 0xf) << 2),
    # v2 = (b1 >> 4) | ((b2 & 3) << 4), v3 = b2 >> 2.  Bytes ff 00 ff -> 63, 3, 48, 63.
    by = np.zeros(24, np.uint8)  # one group of 32 codes
    by[:3] = [0xFF, 0x00, 0xFF]
    by[3:6] = [0x41, 0x10, 0x04]  # codes 1, 1, 1, 1
    wq = by.view(np.uint32).reshape(1, 6)
    one, zero = np.array([[0x3F80]], np.uint16), np.zeros((1, 1), np.uint16)
    d = orc.affine_dequantize_f32(wq, one, zero, 32, 6)[0]
    np.testing.assert_array_equal(d[:8], [63, 3, 48, 63, 1, 1, 1, 1])
    assert (d[8:] == 0).all()


# ---- dequantize --------------------------------------------------------------

def test_dequant_d2_halfway_cases(orc, kat):
    q = kat["d2_q"].reshape(-1, 1) * np.array([1, 0, 0, 0, 0, 0, 0, 0], np.uint32)
    d2 = orc.affine_dequantize(q.astype(np.uint32), kat["d2_s"].reshape(-1, 1), kat["d2_b"].reshape(-1, 1), 32, 8, 2)
    np.testing.assert_array_equal(d2[:, 0], kat["d2_out"])


def test_dequant_d1_matches_float_then_round(orc):
    w = orc.normal_bf16((32, 512), 0.02, 5)
    wq, s, b = orc.affine_quantize(w, 64, 4)
    codes = codes_bytestream(wq, 4, 512).astype(np.float32)
    sf = torch.from_numpy(orc.bf16_to_f32(s)).repeat_interleave(64, 1)
    bf = torch.from_numpy(orc.bf16_to_f32(b)).repeat_interleave(64, 1)
    ref = (sf * torch.from_numpy(codes) + bf).to(torch.bfloat16)
    np.testing.assert_array_equal(orc.affine_dequantize(wq, s, b, 64, 4, 1),
                                  ref.view(torch.int16).numpy().astype(np.uint16))


def test_mxfp4_dequant_exhaustive_table(orc, kat):
    table = kat["mxfp4_table"]
    codes = np.zeros((256, 32), np.uint32)
    codes[:, :16] = np.arange(16)
    wq = np.zeros((256, 4), np.uint32)
    for j in range(32):
        wq[:, j // 8] |= codes[:, j] << (4 * (j % 8))
    d = orc.mxfp4_dequantize(wq, np.arange(256, dtype=np.uint8).reshape(256, 1))
    np.testing.assert_array_equal(d[:, :16].T, table)
    for s in range(256):
        assert orc.e8m0_to_bf16(s) == (0x40 if s == 0 else (0x7FC0 if s == 255 else s << 7))


# ---- mxfp4 quantize ----------------------------------------------------------

def test_mxfp4_exponent_is_ceil_log2_for_every_bf16_scale(orc):
    # one group per positive finite bf16 magnitude: amax = that value.  Scales
    # below 2^-127 have no e8m0 code (the reference casts a negative exponent
    # to uint8, which is undefined), so the sweep starts at amax = 6 * 2^-127.
    mags = np.arange(0x0080, 0x7F80, dtype=np.uint32)  # normal bf16
    vals = orc.bf16_to_f32(mags.astype(np.uint16)).astype(np.float64)
    mags = mags[vals >= 6.0 * 2.0 ** -127]
    g = np.zeros((mags.size, 32), np.uint16)
    g[:, 0] = mags
    _, sc = orc.mxfp4_quantize(g)
    amax = orc.bf16_to_f32(mags.astype(np.uint16)).astype(np.float64)
    s = orc.bf16_to_f32(orc.f32_to_bf16((amax / 6.0).astype(np.float32))).astype(np.float64)
    e = np.ceil(np.log2(s))
    e = np.where(2.0 ** e < s, e + 1, e)
    e = np.where(2.0 ** (e - 1) >= s, e - 1, e)
    np.testing.assert_array_equal(sc[:, 0].astype(np.int64), (e + 127).astype(np.int64))


def test_mxfp4_quantize_nearest_code_and_roundtrip(orc):
    w = orc.normal_bf16((64, 2880), 0.02, 9)
    wq, sc = orc.mxfp4_quantize(w)
    wf = orc.bf16_to_f32(w).astype(np.float64).reshape(64, -1, 32)
    scale = np.ldexp(1.0, sc.astype(np.int64) - 127)[..., None]
    v = wf / scale
    codes = codes_bytestream(wq, 4, 2880).reshape(64, -1, 32)
    lut = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0., -.5, -1, -1.5, -2, -3, -4, -6])
    # v = w / 2^e is exact, and so is every |v - lut| in float64: the code is
    # the first index of the exact minimum distance (argmin order)
    dist = np.abs(v[..., None] - lut)
    np.testing.assert_array_equal(codes, dist.argmin(-1))
    assert np.all(np.abs(v).max(-1) <= 6.0)  # round-up keeps the block maximum representable
    d = orc.bf16_to_f32(orc.mxfp4_dequantize(wq, sc)).reshape(64, -1, 32)
    np.testing.assert_array_equal(d, (lut[codes.astype(np.int64)] * scale).astype(np.float32))


def test_mxfp4_quantize_hand_cases(orc, kat):
    # tests/golden/make_golden.py MXFP4_HAND: exponents ceil(log2(max|w|/6)),
    # ties to the first LUT index (+0 before -0)
    wq, sc = orc.mxfp4_quantize(kat["mxfp4_hand_w"])
    np.testing.assert_array_equal(codes_bytestream(wq, 4, 96), codes_bytestream(kat["mxfp4_hand_wq"], 4, 96))
    np.testing.assert_array_equal(sc, kat["mxfp4_hand_scales"])


def test_mxfp4_quantize_zero_group(orc):
    wq, sc = orc.mxfp4_quantize(np.zeros((2, 32), np.uint16))
    assert (wq == 0).all() and (sc == 127).all()


# ---- quantized matmul --------------------------------------------------------

def rel_l2(got, want):
    return np.sqrt(((got - want) ** 2).sum() / max((want ** 2).sum(), 1e-30))


def store_floor(want, orc):
    return rel_l2(orc.bf16_to_f32(orc.f32_to_bf16(want.astype(np.float32))).astype(np.float64), want)


@pytest.mark.parametrize("bits,gs", [(4, 64), (4, 32), (4, 128), (8, 64), (2, 64)])
def test_qmm_t_vs_f64_reference(orc, bits, gs):
    M, N, K = 3, 96, 2048
    x = orc.normal_bf16((M, K), 1.0, 0x2248 + bits)
    w = orc.normal_bf16((N, K), 0.02, 0x2249 + bits)
    wq, s, b = orc.affine_quantize(w, gs, bits)
    y = orc.bf16_to_f32(orc.qmm_t_affine(x, wq, s, b, gs, bits)).astype(np.float64)
    codes = codes_bytestream(wq, bits, K).astype(np.float64)
    sf = np.repeat(orc.bf16_to_f32(s).astype(np.float64), gs, 1)
    bf = np.repeat(orc.bf16_to_f32(b).astype(np.float64), gs, 1)
    want = orc.bf16_to_f32(x).astype(np.float64) @ (sf * codes + bf).T
    assert rel_l2(y, want) <= 2 * store_floor(want, orc)


def test_qmm_t_one_hot_picks_single_weights(orc):
    N, K, gs = 40, 256, 64
    w = orc.normal_bf16((N, K), 0.02, 3)
    wq, s, b = orc.affine_quantize(w, gs, 4)
    x = np.zeros((K, K), np.uint16)
    x[np.arange(K), np.arange(K)] = 0x3F80  # one-hot rows (1.0)
    y = orc.qmm_t_affine(x, wq, s, b, gs, 4)  # y[k, n] = bf16(s*q[n,k] + b)
    np.testing.assert_array_equal(y, orc.affine_dequantize(wq, s, b, gs, 4, 1).T)


def test_qmm_t_all_ones_sums_codes_exactly(orc):
    N, K = 16, 64
    rng = np.random.default_rng(4)
    codes = rng.integers(0, 2, (N, K)).astype(np.uint32)
    wq = np.zeros((N, K // 8), np.uint32)
    for k in range(K):
        wq[:, k // 8] |= codes[:, k] << (4 * (k % 8))
    s = np.full((N, 1), 0x3F80, np.uint16)
    b = np.zeros((N, 1), np.uint16)
    x = np.full((1, K), 0x3F80, np.uint16)
    y = orc.bf16_to_f32(orc.qmm_t_affine(x, wq, s, b, 64, 4))
    np.testing.assert_array_equal(y[0], codes.sum(1).astype(np.float32))


def test_qmm_non_transposed_vs_f64(orc):
    M, N, K, gs = 2, 128, 96, 64
    x = orc.normal_bf16((M, K), 1.0, 21)
    w = orc.normal_bf16((K, N), 0.02, 22)  # [K, N] quantized along N
    wq, s, b = orc.affine_quantize(w, gs, 4)
    y = orc.bf16_to_f32(orc.qmm_affine(x, wq, s, b, gs, 4)).astype(np.float64)
    deq = orc.bf16_to_f32(orc.affine_dequantize(wq, s, b, gs, 4, 1)).astype(np.float64)
    want = orc.bf16_to_f32(x).astype(np.float64) @ deq
    assert rel_l2(y, want) <= 2 * store_floor(want, orc) + 1e-3


def test_fp_qmm_t_mxfp4_vs_f64_and_one_hot(orc):
    M, N, K = 2, 64, 2880
    x = orc.normal_bf16((M, K), 1.0, 0x22480001)
    w = orc.normal_bf16((N, K), 0.02, 0x22480002)
    wq, sc = orc.mxfp4_quantize(w)
    y = orc.bf16_to_f32(orc.fp_qmm_t_mxfp4(x, wq, sc)).astype(np.float64)
    deq = orc.bf16_to_f32(orc.mxfp4_dequantize(wq, sc)).astype(np.float64)
    want = orc.bf16_to_f32(x).astype(np.float64) @ deq.T
    assert rel_l2(y, want) <= 2 * store_floor(want, orc)
    xo = np.zeros((64, K), np.uint16)
    xo[np.arange(64), np.arange(64) * 7] = 0x3F80
    yo = orc.fp_qmm_t_mxfp4(xo, wq, sc)
    np.testing.assert_array_equal(yo, orc.mxfp4_dequantize(wq, sc)[:, np.arange(64) * 7].T)


def test_gather_is_stack_of_matmuls(orc):
    E, N, K, M = 5, 48, 256, 2
    w = orc.normal_bf16((E, N, K), 0.02, 31)
    wq, s, b = orc.affine_quantize(w, 64, 4)
    x = orc.normal_bf16((3, M, K), 1.0, 32)
    lhs = np.array([0, 2, 1, 2, 0, 1], np.uint32)
    rhs = np.array([4, 0, 0, 3, 1, 4], np.uint32)
    out = orc.gather_qmm_t(x, wq, s, b, lhs, rhs, 64, 4)
    for i in range(lhs.size):
        np.testing.assert_array_equal(out[i], orc.qmm_t_affine(x[lhs[i]], wq[rhs[i]], s[rhs[i]], b[rhs[i]], 64, 4))
    wm, sm = orc.mxfp4_quantize(w)
    outm = orc.gather_qmm_t(x, wm, sm, None, lhs, rhs, mode="mxfp4")
    for i in range(lhs.size):
        np.testing.assert_array_equal(outm[i], orc.fp_qmm_t_mxfp4(x[lhs[i]], wm[rhs[i]], sm[rhs[i]]))


# ---- fused single-token decode MoE --------------------------------------------

def moe_case(orc, din, dff, E, k, gu_bits, d_bits, gs, seed):
    """Random experts quantized by the oracle, distinct expert ids, softmax-like
    positive scores (fused_moe_parity_tests.rs:131-205)."""
    x = orc.normal_bf16((din,), 1.0, seed)
    gate = orc.affine_quantize(orc.normal_bf16((E, dff, din), 0.02, seed + 1), gs, gu_bits)
    up = orc.affine_quantize(orc.normal_bf16((E, dff, din), 0.02, seed + 2), gs, gu_bits)
    down = orc.affine_quantize(orc.normal_bf16((E, din, dff), 0.02, seed + 3), gs, d_bits)
    rng = np.random.default_rng(seed)
    idx = rng.permutation(E)[:k].astype(np.uint32)
    sc = rng.random(k).astype(np.float32)
    return x, idx, sc / sc.sum(), gate, up, down


def norm_dev(a, b):
    """(nrms, nmax) of a - b normalized by b's rms (fused_moe_parity_tests.rs:350-367)."""
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    rms = max(np.sqrt((b ** 2).mean()), 1e-20)
    return np.sqrt(((a - b) ** 2).mean()) / rms, np.abs(a - b).max() / rms


@pytest.mark.parametrize("act", ["swiglu", "geglu"])
@pytest.mark.parametrize("bits", [4, 8])
def test_fused_moe_matches_the_gather_qmm_chain(orc, act, bits):
    # The reference's graph fallback built from the oracle's (separately
    # pinned) gather_qmm: gate/up per slot, activation, down per slot,
    # score-weighted sum.  It rounds through bf16 between the products, so it
    # agrees only to bf16 jitter (the reference's ceilings for it are nrms <
    # 5e-2, nmax < 2e-1, fused_moe_parity_tests.rs:395-409; tighter bounds
    # here); any mix-up of experts, rows, activation or scores is far outside.
    din, dff, E, k, gs = 256, 128, 6, 4, 64
    x, idx, sc, gate, up, down = moe_case(orc, din, dff, E, k, bits, bits, gs, 77 + bits)
    fused = orc.fused_moe(x, idx, sc, gate, up, down, gs, bits, bits, act)
    zero = np.zeros(k, np.uint32)
    g = orc.bf16_to_f32(orc.gather_qmm_t(x.reshape(1, 1, din), *gate, zero, idx, gs, bits)).astype(np.float64)
    u = orc.bf16_to_f32(orc.gather_qmm_t(x.reshape(1, 1, din), *up, zero, idx, gs, bits)).astype(np.float64)
    if act == "geglu":
        a = 0.5 * g * (1 + np.tanh(0.7978845608028654 * (g + 0.044715 * g ** 3))) * u
    else:
        a = g / (1 + np.exp(-g)) * u
    a16 = orc.f32_to_bf16(a.astype(np.float32)).reshape(k, 1, dff)
    d = orc.bf16_to_f32(orc.gather_qmm_t(a16, *down, np.arange(k, dtype=np.uint32), idx, gs, bits))
    chain = (d.reshape(k, din).astype(np.float64) * sc[:, None]).sum(0)
    nrms, nmax = norm_dev(chain, fused)
    # measured here: nrms ~3e-3, nmax ~1e-2 (bf16 roundings of the chain)
    assert nrms < 1e-2 and nmax < 4e-2, (nrms, nmax)
    # pairing the scores with the wrong experts lands far outside the ceiling
    bad = orc.fused_moe(x, idx[::-1].copy(), sc, gate, up, down, gs, bits, bits, act)
    assert norm_dev(chain, bad)[0] > 0.1


def pack_bitstream(codes, bits):
    """Codes -> uint32 words of their little-endian bit stream (per row)."""
    b = (codes.astype(np.uint8)[..., None] >> np.arange(bits, dtype=np.uint8)) & 1
    by = np.packbits(b.reshape(codes.shape[0], -1).astype(np.uint8), axis=1, bitorder="little")
    return np.ascontiguousarray(by).view(np.uint32)


@pytest.mark.parametrize("d_bits", [4, 6, 8])
@pytest.mark.parametrize("act", ["swiglu", "geglu"])
def test_fused_moe_closed_form_identity_experts(orc, act, d_bits):
    # Hand-packed experts with scale 1, bias -8 (4-bit gate/up) so weights are
    # code - 8; x is one-hot at position 0.  Gate row f has weight
    # (f % 16) - 8 there and up rows weight 1, so g_f = (f % 16) - 8, u_f = 1;
    # down is the identity (weight 1 on h == f, 0 elsewhere).  Hence
    # out[h] = score * A((h % 16) - 8), checked against the activations'
    # published values.
    din = dff = gs = 32
    one = 0x3F80
    x = np.zeros(din, np.uint16)
    x[0] = one
    gcodes = np.full((dff, din), 8, np.uint8)
    gcodes[:, 0] = np.arange(dff) % 16
    ucodes = np.full((dff, din), 8, np.uint8)
    ucodes[:, 0] = 9
    dbias = 8
    dcodes = np.full((din, dff), dbias, np.uint8) + np.eye(din, dtype=np.uint8)
    s1 = np.full((1, 32, 1), one, np.uint16)
    m8 = np.full((1, 32, 1), 0xC100, np.uint16)  # -8.0
    gate = (pack_bitstream(gcodes, 4)[None], s1, m8)
    up = (pack_bitstream(ucodes, 4)[None], s1, m8)
    down = (pack_bitstream(dcodes, d_bits)[None], s1, m8)
    out = orc.fused_moe(x, np.array([0], np.uint32), np.array([0.5], np.float32), gate, up, down, gs, 4, d_bits,
                        act)
    g = (np.arange(din) % 16 - 8).astype(np.float64)
    if act == "geglu":
        want = 0.5 * 0.5 * g * (1 + np.tanh(np.sqrt(2 / np.pi) * (g + 0.044715 * g ** 3)))
        anchors = {1: 0.8411919906082768, -1: -0.15880800939172324}
    else:
        want = 0.5 * g / (1 + np.exp(-g))
        anchors = {1: 0.7310585786300049, -1: -0.2689414213699951}
    np.testing.assert_allclose(out, want, rtol=1e-6, atol=1e-7)
    for gv, av in anchors.items():
        h = int(gv + 8)  # rows with g = gv
        assert abs(out[h] - 0.5 * av) < 1e-6
    assert out[8] == 0.0  # A(0) = 0


def test_fused_moe_invariants(orc):
    # linear in the scores, independent of slot order, and a repeated expert
    # equals one slot carrying the summed score
    din, dff, E, gs = 128, 64, 5, 32
    x, _, _, gate, up, down = moe_case(orc, din, dff, E, 3, 4, 4, gs, 91)
    idx = np.array([3, 1, 4], np.uint32)
    s1 = np.array([0.2, 0.5, 0.3], np.float32)
    s2 = np.array([0.1, -0.25, 0.75], np.float32)
    f = lambda i, s: orc.fused_moe(x, i, s, gate, up, down, gs, 4, 4).astype(np.float64)
    np.testing.assert_allclose(f(idx, s1 + s2), f(idx, s1) + f(idx, s2), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(f(idx[[2, 0, 1]], s1[[2, 0, 1]]), f(idx, s1), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(f(np.array([2, 2], np.uint32), np.array([0.25, 0.5], np.float32)),
                               f(np.array([2], np.uint32), np.array([0.75], np.float32)), rtol=1e-5, atol=1e-6)
    # out-of-range expert ids are clamped to the last expert
    np.testing.assert_array_equal(f(np.array([9], np.uint32), s1[:1]), f(np.array([E - 1], np.uint32), s1[:1]))


# ---- fp8 e4m3, mxfp8, nvfp4 ----------------------------------------------------

def e4m3_value(c):
    """e4m3fn code -> value from the format definition (bias 7, no infinities,
    0x7F / 0xFF NaN, subnormals m * 2^-9), in float64."""
    c = np.asarray(c, np.int64)
    s = np.where(c & 0x80, -1.0, 1.0)
    e, m = (c >> 3) & 15, c & 7
    v = np.where(e == 0, np.ldexp(m.astype(np.float64), -9), np.ldexp((8 + m).astype(np.float64), e - 10))
    v = s * v
    return np.where((e == 15) & (m == 7), np.nan, v)


def test_e4m3_decode_exhaustive(orc):
    codes = np.arange(256, dtype=np.uint8)
    np.testing.assert_array_equal(orc.e4m3_decode(codes), e4m3_value(codes).astype(np.float32))


def test_e4m3_encode_round_trips_every_finite_code(orc):
    codes = np.array([c for c in range(256) if c not in (0x7F, 0xFF)], np.uint8)
    np.testing.assert_array_equal(orc.e4m3_encode(e4m3_value(codes).astype(np.float32)), codes)


def test_e4m3_encode_hand_cases(orc, kat):
    # tests/golden/make_golden.py E4M3_HAND: half-up ties, saturation and the
    # [464, 496) NaN code, underflow, truncated subnormals, the carry quirk
    np.testing.assert_array_equal(orc.e4m3_encode(kat["e4m3_hand_in"]), kat["e4m3_hand_code"])


def test_e4m3_encode_normal_range_is_nearest_ties_up(orc):
    # in the normal range [2^-6, 448] the encoder returns the nearest e4m3
    # value, ties to the larger magnitude (brute force over the codes)
    pos = np.arange(0x08, 0x7F)
    vals = e4m3_value(pos)
    rng = np.random.default_rng(7)
    x = np.concatenate([np.exp(rng.uniform(np.log(2.0 ** -6), np.log(448.0), 20000)),
                        (vals[:-1] + vals[1:]) / 2])  # every midpoint
    x = x.astype(np.float32).astype(np.float64)
    x = x[(x >= 2.0 ** -6) & (x <= 448.0)]
    d = np.abs(x[:, None] - vals[None, :])
    best = d.min(1, keepdims=True)
    want = np.where(d == best, pos[None, :], -1).max(1)  # ties: the larger code
    for sgn in (1, -1):
        got = orc.e4m3_encode((sgn * x).astype(np.float32)).astype(np.int64)
        np.testing.assert_array_equal(got, want | (0x80 if sgn < 0 else 0))


def test_mxfp8_and_nvfp4_quantize_hand_cases(orc, kat):
    wq, sc = orc.mxfp8_quantize(kat["mxfp8_hand_w"])
    np.testing.assert_array_equal(wq, kat["mxfp8_hand_wq"])
    np.testing.assert_array_equal(sc, kat["mxfp8_hand_scales"])
    wq, sc = orc.nvfp4_quantize(kat["nvfp4_hand_w"])
    np.testing.assert_array_equal(wq, kat["nvfp4_hand_wq"])
    np.testing.assert_array_equal(sc, kat["nvfp4_hand_scales"])


def assert_bf16_equal_nan_any_sign(got, want):
    # MLX's NaN sign through from_fp8 and the bf16 conversion is not pinned:
    # NaN positions must match, other bits exactly
    isnan = lambda b: (b & 0x7FFF) > 0x7F80
    np.testing.assert_array_equal(isnan(got), isnan(want))
    np.testing.assert_array_equal(got[~isnan(want)], want[~isnan(want)])


def test_mxfp8_dequantize_table(orc):
    # every code under scales 0, 1, 100, 127, 254, 255: from_fp8(code) *
    # 2^(s-127), one bf16 rounding (float64 ldexp is exact), NaN for s == 255
    codes = np.arange(256, dtype=np.uint8)
    for s in (0, 1, 100, 127, 254, 255):
        wq = np.tile(codes, 1).reshape(8, 32).copy().view(np.uint32)
        sc = np.full((8, 1), s, np.uint8)
        got = orc.mxfp8_dequantize(wq, sc).reshape(-1)
        want = e4m3_value(codes) * (np.nan if s == 255 else 2.0 ** (s - 127))
        assert_bf16_equal_nan_any_sign(got, bf16_from_torch(want.astype(np.float32)).reshape(-1))


def test_nvfp4_dequantize_table(orc):
    # 16 codes x every e4m3 scale: LUT[code] * e4m3(scale), exact in bf16
    lut = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0., -.5, -1, -1.5, -2, -3, -4, -6])
    codes = np.arange(16, dtype=np.uint32)
    wq = np.zeros((256, 2), np.uint32)
    for j in range(16):
        wq[:, j // 8] |= codes[j] << (4 * (j % 8))
    sc = np.arange(256, dtype=np.uint8).reshape(256, 1)
    got = orc.nvfp4_dequantize(wq, sc)
    want = lut[None, :] * e4m3_value(np.arange(256))[:, None]
    assert_bf16_equal_nan_any_sign(got, bf16_from_torch(want.astype(np.float32)))
