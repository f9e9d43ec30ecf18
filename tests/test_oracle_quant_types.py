"""Pins of the oracle's typed affine quantizer (oracle_affine_quantize_t:
float16 / bfloat16 / float32 weights, bits 1-6 and 8) and of its float16
conversions.

- float16 <-> float32: every one of the 65,536 float16 patterns against
  numpy's decoding, and float32 -> float16 rounding against numpy's
  astype(float16) (IEEE round-to-nearest-even) on random values over the whole
  range, the halfway points around each binade edge, subnormals and the
  overflow threshold.
- The quantizer: against an independent numpy float32 restatement of MLX's
  CPU quantizer (quantized.cpp:1251-1303, the 1-bit branch at 1261-1264
  included), on random data at scales 1e-4..1e2, one-signed, constant and
  zero groups, for every dtype and width; 1-bit and 3-bit groups worked by
  hand; the packing as one little-endian bit stream of `bits` bits per code.
"""
import numpy as np
import pytest

import oracle as orc
from test_oracle import bf16_from_torch, codes_bytestream, torch_from_bits


def test_f16_to_f32_every_pattern():
    h = np.arange(65536, dtype=np.uint32)
    want = h.astype(np.uint16).view(np.float16).astype(np.float32)
    got = np.array([orc.f16_bits_to_f32(int(v)) for v in h], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    np.testing.assert_array_equal(got[~nan], want[~nan])


def test_f32_to_f16_round_to_nearest_even():
    rng = np.random.default_rng(3)
    x = rng.standard_normal(20000).astype(np.float32) * (10.0 ** rng.uniform(-9, 5, 20000)).astype(np.float32)
    edges = []
    for e in range(-24, 16):
        for m in (0.0, 0.5, 1.0, 1.5, 1023.5):  # halfway points between neighbours, both parities
            v = np.float32(2.0 ** e * (1 + m / 1024.0))
            edges += [v, -v, np.nextafter(v, np.float32(0)), np.nextafter(v, np.float32(np.inf))]
    edges += [65504.0, 65519.996, 65520.0, 65536.0, 2.0 ** -25, 2.0 ** -25 * 1.0001, 2.0 ** -26, 3 * 2.0 ** -25,
              0.0, -0.0, np.inf, -np.inf]
    x = np.concatenate([x, np.array(edges, np.float32)])
    want = x.astype(np.float16).view(np.uint16)
    got = np.array([orc.f32_to_f16_bits(float(v)) for v in x], np.uint16)
    np.testing.assert_array_equal(got, want)


def numpy_quantize_typed(wf, gs, bits):
    """quantized.cpp:1251-1303 in numpy float32: codes, float32 scale, bias."""
    g = wf.reshape(-1, gs).astype(np.float32)
    T = np.float32((1 << bits) - 1)
    mn, mx = g.min(1), g.max(1)
    if bits == 1:
        s = np.maximum(mx - mn, np.float32(1e-7)).astype(np.float32)
        b = mn.astype(np.float32)
    else:
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


def weights(dtype, rows, K, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, K)).astype(np.float32)
    x *= (10.0 ** rng.uniform(-4, 2, (rows, 1))).astype(np.float32)
    x[4:6] = np.abs(x[4:6])
    x[6:8] = -np.abs(x[6:8])
    x[8] = 0.375
    x[9] = 0.0
    if dtype == "bfloat16":
        w = bf16_from_torch(x)
        return w, torch_from_bits(w).float().numpy()
    if dtype == "float16":
        w = x.astype(np.float16)
        return w, w.astype(np.float32)
    return x, x


def stored(v32, dtype):
    if dtype == "bfloat16":
        return bf16_from_torch(v32)
    if dtype == "float16":
        return v32.astype(np.float16)
    return v32.astype(np.float32)


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_typed_quantize_matches_numpy_restatement(dtype, bits, gs):
    rows, K = 24, 256
    w, wf = weights(dtype, rows, K, 10 * bits + gs)
    codes, s, b = numpy_quantize_typed(wf, gs, bits)
    wq, so, bo = orc.affine_quantize_t(w, dtype, gs, bits)
    assert wq.shape == (rows, K * bits // 32)
    np.testing.assert_array_equal(codes_bytestream(wq, bits, K), codes)
    np.testing.assert_array_equal(np.asarray(so).reshape(-1).view(np.uint8),
                                  np.asarray(stored(s, dtype)).view(np.uint8))
    np.testing.assert_array_equal(np.asarray(bo).reshape(-1).view(np.uint8),
                                  np.asarray(stored(b, dtype)).view(np.uint8))


def test_bfloat16_typed_entry_is_the_bfloat16_quantizer():
    w = orc.normal_bf16((8, 256), 0.05, 5)
    for bits in (2, 4, 6, 8):
        a = orc.affine_quantize(w, 64, bits)
        b = orc.affine_quantize_t(w, "bfloat16", 64, bits)
        for x, y in zip(a, b):
            np.testing.assert_array_equal(x, y)


def test_one_bit_group_worked_by_hand():
    # w_min = -0.25, w_max = 0.5: scale = 0.75, bias = -0.25 (no edge snapping
    # at 1 bit); codes rint((w + 0.25) / 0.75): 0.5 -> 1, -0.25 -> 0,
    # 0.125 -> rint(0.5) = 0 (tie to even), 0.2 -> rint(0.6) = 1
    w = np.zeros((1, 32), np.float32)
    w[0, :4] = [0.5, -0.25, 0.125, 0.2]
    wq, s, b = orc.affine_quantize_t(w, "float32", 32, 1)
    assert s[0, 0] == np.float32(0.75) and b[0, 0] == np.float32(-0.25)
    # the rest are 0.0 -> rint(0.25 / 0.75) = 0; code i is bit i of the word
    assert int(wq[0, 0]) == 0b1001


def test_three_bit_group_worked_by_hand():
    # w = [0, 0.5, ..., 3.5] repeated: w_min = 0, w_max = 3.5, n_bins = 7 ->
    # scale -0.5 (|w_min| < |w_max|), edge 3.5, q0 = rint(3.5 / -0.5) = -7,
    # scale = 3.5 / -7 = -0.5, bias = 3.5: code = rint((w - 3.5) / -0.5) = 7 - 2w
    w = np.tile(np.arange(8, dtype=np.float32) * 0.5, 4)[None, :]
    wq, s, b = orc.affine_quantize_t(w.astype(np.float16), "float16", 32, 3)
    assert s[0, 0] == np.float16(-0.5) and b[0, 0] == np.float16(3.5)
    want = np.tile(7 - np.arange(8), 4)
    np.testing.assert_array_equal(codes_bytestream(wq, 3, 32)[0], want)
    # 3 bytes per 8 codes: codes 7,6,5,4,3,2,1,0 -> bits 111 011 101 001 110 010 100 000 (low first)
    assert wq.view(np.uint8)[0, :3].tolist() == [0x77, 0x39, 0x05]
