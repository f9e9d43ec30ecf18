"""Pins of oracle/generic.py, the numpy restatement that checks the general
kernel (any float type, affine 2-8-bit codes, both transposes).

- Code order: hand-worked byte patterns for every width, written from the
  reference's explicit masks (overlays/cpu/mlx/backend/cpu/quantized.cpp:
  107-137 for 3/5/6 bits, the `wi & bitmask; wi >>= bits` loop of 161-178 /
  222-236 for 2/4/8 bits), not from the oracle's bit-stream formula.
- The matmul structure (which index is the reduction, scale/bias placement):
  agreement with the C oracle (oracle/mlxq_oracle.c, pinned against the
  reference's golden vectors) for 4/8-bit affine at both transposes and for
  mxfp4.
"""
import numpy as np
import pytest

import oracle as orc
from oracle import generic as og


def row_from_bytes(bs):
    b = np.array(bs + [0] * (-len(bs) % 4), dtype=np.uint8)
    return b.view(np.uint32)[None, :]


def test_three_bit_codes_hand_worked():
    # bytes 0xC5 0x9A 0x3E:  v0 = b0&7 = 5; v1 = (b0&0x38)>>3 = 0;
    # v2 = ((b0&0xC0)>>6) + ((b1&1)<<2) = 3; v3 = (b1&0xE)>>1 = 5;
    # v4 = (b1&0x70)>>4 = 1; v5 = ((b1&0x80)>>7) + ((b2&3)<<1) = 5;
    # v6 = (b2&0x1C)>>2 = 7; v7 = (b2&0xE0)>>5 = 1
    got = og.unpack_codes(row_from_bytes([0xC5, 0x9A, 0x3E]), 3, 8)[0]
    assert got.tolist() == [5, 0, 3, 5, 1, 5, 7, 1]


def test_five_bit_codes_hand_worked():
    # bytes 0x3A 0xC7 0x5E 0x91 0xB6:
    # v0 = b0&0x1F = 26; v1 = ((b0&0xE0)>>5) + ((b1&3)<<3) = 1 + 24 = 25;
    # v2 = (b1&0x7C)>>2 = 17; v3 = ((b1&0x80)>>7) + ((b2&0xF)<<1) = 1 + 28 = 29;
    # v4 = ((b2&0xF0)>>4) + ((b3&1)<<4) = 5 + 16 = 21; v5 = (b3&0x3E)>>1 = 8;
    # v6 = ((b3&0xC0)>>6) + ((b4&7)<<2) = 2 + 24 = 26; v7 = (b4&0xF8)>>3 = 22
    got = og.unpack_codes(row_from_bytes([0x3A, 0xC7, 0x5E, 0x91, 0xB6]), 5, 8)[0]
    assert got.tolist() == [26, 25, 17, 29, 21, 8, 26, 22]


def test_six_bit_codes_hand_worked():
    # bytes 0x9D 0x4B 0xE2: v0 = b0&0x3F = 29; v1 = ((b0>>6)&3) + ((b1&0xF)<<2) = 2 + 44 = 46;
    # v2 = ((b1>>4)&0xF) + ((b2&3)<<4) = 4 + 32 = 36; v3 = (b2>>2)&0x3F = 56
    got = og.unpack_codes(row_from_bytes([0x9D, 0x4B, 0xE2]), 6, 4)[0]
    assert got.tolist() == [29, 46, 36, 56]


@pytest.mark.parametrize("bits,byte,want", [
    (1, 0xB4, [0, 0, 1, 0, 1, 1, 0, 1]),  # 1011 0100, low bit first
    (2, 0xB4, [0, 1, 3, 2]),        # 10 11 01 00, low pair first
    (4, 0xB4, [4, 11]),             # low nibble first
    (8, 0xB4, [180]),
])
def test_power_of_two_codes_hand_worked(bits, byte, want):
    got = og.unpack_codes(row_from_bytes([byte]), bits, 8 // bits)[0]
    assert got.tolist() == want


@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 6, 8])
def test_pack_unpack_round_trip(bits):
    rng = np.random.default_rng(bits)
    codes = rng.integers(0, 1 << bits, size=(3, 96))
    wq = og.pack_codes(codes, bits)
    assert wq.shape == (3, 96 * bits // 32)
    np.testing.assert_array_equal(og.unpack_codes(wq, bits, 96), codes)


def rel(a, b):
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64])
def test_qmm_transpose_matches_c_oracle(bits, gs):
    x = orc.normal_bf16((5, 256), 1.0, 40 + bits)
    w = orc.normal_bf16((24, 256), 0.02, 41 + bits)
    wq, s, b = orc.affine_quantize(w, gs, bits)
    want = orc.bf16_to_f32(orc.qmm_t_affine(x, wq, s, b, gs, bits)).astype(np.float64)
    got = og.round_to(og.qmm(orc.bf16_to_f32(x), wq, orc.bf16_to_f32(s), orc.bf16_to_f32(b), True, gs, bits),
                      "bfloat16")
    assert rel(got, want) <= 8e-3


@pytest.mark.parametrize("bits", [4, 8])
def test_qmm_no_transpose_matches_c_oracle(bits):
    gs = 32
    x = orc.normal_bf16((3, 64), 1.0, 50 + bits)
    w = orc.normal_bf16((64, 96), 0.02, 51 + bits)  # [K, N], quantized along N
    wq, s, b = orc.affine_quantize(w, gs, bits)
    want = orc.bf16_to_f32(orc.qmm_affine(x, wq, s, b, gs, bits)).astype(np.float64)
    got = og.round_to(og.qmm(orc.bf16_to_f32(x), wq, orc.bf16_to_f32(s), orc.bf16_to_f32(b), False, gs, bits),
                      "bfloat16")
    assert rel(got, want) <= 8e-3


def test_mxfp4_matches_c_oracle():
    x = orc.normal_bf16((4, 128), 1.0, 60)
    w = orc.normal_bf16((40, 128), 0.02, 61)
    wq, sc = orc.mxfp4_quantize(w)
    want = orc.bf16_to_f32(orc.fp_qmm_t_mxfp4(x, wq, sc)).astype(np.float64)
    got = og.round_to(og.qmm(orc.bf16_to_f32(x), wq, sc, None, True, 32, 4, "mxfp4"), "bfloat16")
    assert rel(got, want) <= 8e-3


@pytest.mark.parametrize("bits", [2, 4, 6, 8])
def test_dequantize_matches_c_oracle(bits):
    w = orc.normal_bf16((6, 128), 0.02, 70 + bits)
    wq, s, b = orc.affine_quantize(w, 64, bits)
    want = orc.affine_dequantize_f32(wq, s, b, 64, bits).astype(np.float64)
    got = og.dequantize(wq, orc.bf16_to_f32(s), orc.bf16_to_f32(b), 64, bits, 128)
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-9)


def test_round_to_bfloat16_ties_to_even():
    # 1 + 2^-8 is halfway between 1 and 1 + 2^-7: ties to the even 1.0;
    # 1 + 3 * 2^-8 is halfway between 1 + 2^-7 and 1 + 2^-6: ties up
    y = np.array([1 + 2.0 ** -8, 1 + 3 * 2.0 ** -8, -(1 + 2.0 ** -8)])
    np.testing.assert_array_equal(og.round_to(y, "bfloat16"), [1.0, 1 + 2.0 ** -6, -1.0])


@pytest.mark.parametrize("bits", [2, 4, 6, 8])
def test_dequantize_graph_bfloat16_is_the_pinned_c_oracle(bits):
    # bfloat16 scales and result: bit for bit the C oracle's dequantize
    # (pinned against the reference's fixtures)
    w = orc.normal_bf16((6, 256), 0.05, 80 + bits)
    wq, s, b = orc.affine_quantize(w, 64, bits)
    want = orc.bf16_to_f32(orc.affine_dequantize(wq, s, b, 64, bits)).astype(np.float64)
    got = og.dequantize_graph(wq, orc.bf16_to_f32(s), orc.bf16_to_f32(b), 64, bits, 256, "bfloat16", "bfloat16")
    np.testing.assert_array_equal(got, want)


def test_dequantize_graph_float16_rounds_each_op():
    # q = 3, s = f16(0.1) = 0.0999755859375, b = f16(-0.2) = -0.199951171875:
    # q*s = 0.2999267578125 lies halfway between the float16 neighbours
    # 1228 * 2^-12 and 1229 * 2^-12, so it rounds to the even 0.2998046875;
    # + b = 0.099853515625 (= 1636 * 2^-14, exact).  A fused q*s + b would
    # give 0.0999755859375 instead.
    codes = np.zeros((1, 32), np.int64)
    codes[0, 0] = 3
    wq = og.pack_codes(codes, 4)
    got = og.dequantize_graph(wq, np.array([[np.float16(0.1)]], np.float64),
                              np.array([[np.float16(-0.2)]], np.float64), 32, 4, 32, "float16", "float16")
    assert got[0, 0] == 0.099853515625
    assert got[0, 1] == float(np.float16(-0.2))


def test_mxfp4_dequantize_graph_float16_scale_range():
    # scale 2^(s-127) formed in float16: 2^-25 rounds to 0 (tie to even),
    # 2^-24 is the smallest subnormal, 2^16 overflows to inf; NaN for 255
    codes = np.full((4, 32), 2, np.int64)  # LUT[2] = 1.0
    wq = og.pack_codes(codes, 4)
    sc = np.array([[102], [103], [143], [255]], np.uint8)
    got = og.mxfp4_dequantize_graph(wq, sc, 32, "float16")[:, 0]
    assert got[0] == 0.0 and got[1] == 2.0 ** -24 and np.isinf(got[2]) and np.isnan(got[3])
    got32 = og.mxfp4_dequantize_graph(wq, sc, 32, "float32")[:, 0]
    assert got32[0] == 2.0 ** -25 and got32[2] == 2.0 ** 16
