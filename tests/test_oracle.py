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

@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_affine_quantize_known_answers(orc, kat, bits, gs):
    wq, s, b = orc.affine_quantize(kat[f"ramp_w_b{bits}_g{gs}"], gs, bits)
    np.testing.assert_array_equal(wq, kat[f"ramp_wq_b{bits}_g{gs}"])
    np.testing.assert_array_equal(s, kat[f"ramp_s_b{bits}_g{gs}"])
    np.testing.assert_array_equal(b, kat[f"ramp_b_b{bits}_g{gs}"])


@pytest.mark.parametrize("bits", [4, 8])
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


def test_affine_packing_is_little_endian_bitstream(orc):
    w = orc.normal_bf16((8, 256), 0.02, 11)
    for bits in (2, 4, 8):
        wq, s, b = orc.affine_quantize(w, 64, bits)
        codes = codes_bytestream(wq, bits, 256).astype(np.float32)
        # D2 rebuilt from byte-stream codes with torch's bf16 ops
        st = torch_from_bits(s).repeat_interleave(64, dim=1)
        bt = torch_from_bits(b).repeat_interleave(64, dim=1)
        ref = (torch.from_numpy(codes).to(torch.bfloat16) * st) + bt
        np.testing.assert_array_equal(orc.affine_dequantize(wq, s, b, 64, bits, 2),
                                      ref.view(torch.int16).numpy().astype(np.uint16))


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
    dist = np.abs(v[..., None] - lut)
    chosen = np.take_along_axis(dist, codes[..., None].astype(np.int64), -1)[..., 0]
    assert np.all(chosen <= dist.min(-1) * (1 + 2 ** -7) + 1e-30)
    assert np.all(np.abs(v).max(-1) <= 6.0 * (1 + 2 ** -7))  # round-up keeps the block maximum representable
    d = orc.bf16_to_f32(orc.mxfp4_dequantize(wq, sc)).reshape(64, -1, 32)
    np.testing.assert_array_equal(d, (lut[codes.astype(np.int64)] * scale).astype(np.float32))


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
