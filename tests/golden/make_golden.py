"""Write tests/golden/kat.npz: known-answer vectors derived from closed forms.

Nothing here calls the oracle or the product library.  Every expected value
comes from hand-derived formulas of the reference algorithms, evaluated with
numpy/torch arithmetic:

* mxfp4_table[c, s]  bf16 bits of FP4_LUT[c] * 2^(s-127) (s == 255 -> NaN),
  the definition in overlays/rocm/mlx/ops.cpp:5646-5695 and the CPU scale
  decode overlays/cpu/mlx/backend/cpu/quantized.cpp:91-105.  float64 ldexp is
  exact for these values; bf16 conversion by torch.
* affine ramp groups (quantized.cpp:1233-1305 worked by hand; 6-bit codes
  packed 4 per 3 bytes, the little-endian bit stream):
    c_k = k % 2^bits (last c = 2^bits - 1), T = 2^bits - 1:
    w_k = c_k * d  -> w_max edge, scale = -d, bias = T d, code = T - c_k
    w_k = -c_k * d -> w_min edge, scale = +d, bias = -T d, code = T - c_k
    all-zero group      -> scale = bf16(-1e-7), bias = 0, code = 0
  with d a power of two, so every quantity is exact.
* affine hand cases (quantized.cpp:1251-1303 worked by hand in float32 steps,
  see HAND_CASES): groups whose float32 scale is not a bf16 value (so codes
  computed from bf16(scale) differ), exact rint ties of either parity in the
  codes and in q0 = rint(edge / scale), the |w_min| == |w_max| branch and a
  clamped far extreme, at bits 2/4/6/8.
* mxfp4 hand cases (ops.cpp:5364-5431 worked by hand): the e8m0 exponent is
  ceil(log2(bf16(max|w| / 6))), the codes the first index of the minimum
  distance in FP4_LUT order (ties between neighbours, +0 before -0).
* e4m3 hand cases (MLX to_fp8 on the ROCm backend, convert_fp8.hip:18-66,
  worked by hand): half-up ties, saturation to 448 and the NaN code for
  [464, 496), underflow below 2^-9, truncated subnormals and the subnormal
  carry quirk.
* mxfp8 / nvfp4 quantizer hand groups (ops.cpp:5364-5431 with those encoders).
* dequant_d2: bf16(bf16(q * s) + b) evaluated with torch's bfloat16 ops (an
  independent implementation of MLX's bf16 arithmetic), on halfway cases.

Run:  python tests/golden/make_golden.py
"""
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LUT = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0], dtype=np.float64)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().astype(np.uint16)


def mxfp4_table() -> np.ndarray:
    c = np.arange(16)[:, None]
    s = np.arange(256)[None, :]
    with np.errstate(over="ignore"):
        v = np.ldexp(LUT[c], (s - 127).astype(np.int64))
        v32 = v.astype(np.float32)  # exact or +-inf
    out = bf16_bits(v32)
    out[:, 255] = 0x7FC0
    return out


def pack(codes: np.ndarray, bits: int) -> np.ndarray:
    if bits == 6:
        # 4 codes per 3 bytes, i.e. the little-endian bit stream of the codes
        # (quantized.cpp:1238-1240, 1283-1297)
        b = (codes.astype(np.uint8)[..., None] >> np.arange(6, dtype=np.uint8)) & 1
        by = np.packbits(b.reshape(codes.shape[0], -1).astype(np.uint8), axis=1, bitorder="little")
        return np.ascontiguousarray(by).view(np.uint32)
    per = 32 // bits
    codes = codes.reshape(codes.shape[0], -1, per).astype(np.uint64)
    shifts = (np.arange(per, dtype=np.uint64) * bits)[None, None, :]
    return (codes << shifts).sum(-1).astype(np.uint32)


def affine_ramps(bits: int, gs: int):
    d = np.float32(2.0 ** -6)
    k = np.arange(gs)
    mod = 1 << bits
    c = k % mod
    c[-1] = mod - 1  # the group spans the full code range [0, 2^bits - 1]
    ramp = c.astype(np.float32)
    rows = np.stack([ramp * d, -ramp * d, np.zeros(gs, np.float32)])
    w = bf16_bits(rows)
    codes = np.stack([(mod - 1) - c, (mod - 1) - c, np.zeros(gs, np.int64)])
    top = np.float32(mod - 1) * d
    scales = bf16_bits(np.array([[-d], [d], [np.float32(-1e-7)]], np.float32))
    biases = bf16_bits(np.array([[top], [-top], [0.0]], np.float32))
    return w, pack(codes, bits), scales, biases


# Hand-worked groups of MLX's CPU affine quantizer (quantized.cpp:1251-1303).
# T = 2^bits - 1; scale0 = max((w_max - w_min) / T, 1e-7), negated unless
# |w_min| > |w_max|; edge = w_min if |w_min| > |w_max| else w_max;
# q0 = rint(edge / scale0); if q0 != 0: scale = edge / q0, bias = edge;
# code = clamp(rint((w - bias) / scale), 0, T); scale and bias are stored as
# bf16 only after the codes are computed.  Each group is 32 values: the listed
# head, whose first value is the edge, then the edge repeated (code 0).  Values: (bits, head, codes of the
# head, bf16 bits of the stored scale, bf16 bits of the stored bias).
HAND_CASES = {
    # T=3, edge w_min=-0.75: scale0 = 0.75/3 = 0.25 exactly, q0 = rint(-3) = -3,
    # scale = 0.25, bias = -0.75; (w+0.75)/0.25 = 0.5, 1.5, 2.5 at -0.625,
    # -0.375, -0.125: rint ties to 0, 2, 2 (round-half-away would give 1, 2, 3).
    "tie2": (2, [-0.75, 0.0, -0.625, -0.375, -0.125, -0.5, -0.25],
             [0, 3, 0, 2, 2, 1, 2], 0x3E80, 0xBF40),
    # T=15, |w_min| = 0 < w_max = 0.9375: edge = w_max, scale0 = -0.0625,
    # q0 = rint(0.9375 / -0.0625) = -15, scale = -0.0625, bias = 0.9375;
    # (0.9375 - w) * 16 = 0.5, 1.5, 2.5, 7.5, 14.5 -> 0, 2, 2, 8, 14.
    "tie4": (4, [0.9375, 0.0, 0.90625, 0.84375, 0.78125, 0.46875, 0.03125],
             [0, 15, 0, 2, 2, 8, 14], 0xBD80, 0x3F70),
    # T=3, w_min=-1, w_max=0: scale0 = fl(1/3) = 0x3EAAAAAB, q0 = -3,
    # scale = fl(-1/-3) = 0x3EAAAAAB, bias = -1.  w = -0.166015625:
    # 0.833984375 / 0.33333334 = 2.50195 -> 3 (bf16(scale) = 0.333984375 would
    # give 2.4970 -> 2).
    "scale2": (2, [-1.0, 0.0, -0.166015625], [0, 3, 3], 0x3EAB, 0xBF80),
    # T=15: scale = fl(1/15) = 0x3D888889 (q0 = rint(-14.999999) = -15).
    # w = -0.03125: 0.96875 / 0.06666667 = 14.53125 -> 15 (bf16 scale
    # 0.06689453125: 14.4817 -> 14).
    "scale4": (4, [-1.0, 0.0, -0.03125], [0, 15, 15], 0x3D89, 0xBF80),
    # T=63: scale = fl(1/63) = 0x3C820821 (q0 = rint(-62.999996) = -63), whose
    # bf16 0x3C82 = 0.015869140625 is smaller.  w = -0.008056640625:
    # 0.991943359375 / 0.015873017 = 62.4924 -> 62 (bf16 scale: 62.5080 -> 63).
    "scale6": (6, [-1.0, 0.0, -0.008056640625], [0, 63, 62], 0x3C82, 0xBF80),
    # T=255: scale = fl(1/255) = 0x3B808081.  w = 0: 1 / 0.003921569 = 254.99999
    # -> 255 (bf16 scale 0.003936767578125: 254.0186 -> 254).
    "scale8": (8, [-1.0, 0.0], [0, 255], 0x3B81, 0xBF80),
    # |w_min| == |w_max| = 1 takes the w_max branch: scale0 = -fl(2/15) =
    # -0.13333334, 1 / -0.13333334 = -7.4999995 -> q0 = -7, scale = fl(1/-7) =
    # 0xBE124925, bias = 1; codes (1-w)/0.14285715: 1 -> 0, -1 -> 14, 0 -> 7.
    "equal4": (4, [1.0, -1.0, 0.0], [0, 14, 7], 0xBE12, 0x3F80),
    # rint tie in q0: w_min = -0.53125, w_max = 0.40625: scale0 = 0.9375/15 =
    # 0.0625, edge/scale0 = -8.5 exactly -> q0 = -8 (not -9), scale = 0.06640625,
    # bias = -0.53125; w_max: 0.9375 / 0.06640625 = 14.1176 -> 14 (q0 = -9 would
    # give scale 0.0590278 and 15.88 -> 15).
    "q0tie4": (4, [-0.53125, 0.40625], [0, 14], 0x3D88, 0xBF08),
    # q0 tie of the other parity and a clamped far extreme: w_min = -0.59375,
    # w_max = 0.34375: scale0 = 0.0625, edge/scale0 = -9.5 -> q0 = -10,
    # scale = fl(0.059375) = 0x3D733333, bias = -0.59375; w_max:
    # 0.9375 / 0.059375 = 15.79 -> 16, clamped to 15.
    "clamp4": (4, [-0.59375, 0.34375], [0, 15], 0x3D73, 0xBF18),
}


def affine_hand_cases():
    out = {}
    for name, (bits, head, codes, s_bits, b_bits) in HAND_CASES.items():
        w = np.full(32, head[0], np.float32)
        w[: len(head)] = head
        c = np.zeros(32, np.int64)
        c[: len(codes)] = codes
        wb = bf16_bits(w[None])
        # every listed value is a bf16 value (the quantizer's input)
        assert np.array_equal(torch.from_numpy(wb.astype(np.int16)).view(torch.bfloat16).float().numpy()[0], w)
        out[f"hand_w_{name}_b{bits}"] = wb
        out[f"hand_wq_{name}_b{bits}"] = pack(c[None], bits)
        out[f"hand_s_{name}_b{bits}"] = np.array([[s_bits]], np.uint16)
        out[f"hand_b_{name}_b{bits}"] = np.array([[b_bits]], np.uint16)
    return out


# mxfp4 graph quantizer (ops.cpp:5364-5431) by hand.  Group 0: max|w| = 6,
# scale bf16(6/6) = 1, exponent 0 (byte 127), v = w.  Ties go to the first
# index of FP4_LUT = [0, .5, 1, 1.5, 2, 3, 4, 6, -0, -.5, -1, -1.5, -2, -3, -4, -6]:
# 5 -> 4 (index 6), 0.75 -> 0.5 (1), -0.25 -> +0 (0), -0 -> +0 (0), ...
# Group 1: max|w| = 3, scale 0.5, exponent -1 (byte 126), v = 2w.
# Group 2: max|w| = 7, scale bf16(7/6) = 1.1640625, exponent ceil(log2) = 1
# (byte 128), v = w/2: 7 -> 3.5 -> 3 (index 5).
MXFP4_HAND = [
    ([6, -6, 5, -5, 0.25, -0.25, 0.75, -0.75, 2.5, -2.5, 3.5, -3.5, 1.25, -1.25, 1.75, -1.75,
      0.10009765625, -0.10009765625, 0.0, -0.0, 4.5, -4.5, 5.5, -5.5, 0.5, -0.5, 1, -1, 3, -3, 6, 6],
     [7, 15, 6, 14, 0, 0, 1, 9, 4, 12, 5, 13, 2, 10, 3, 11,
      0, 0, 0, 0, 6, 14, 7, 15, 1, 9, 2, 10, 5, 13, 7, 7], 127),
    ([3, -3, 2.5, -2.5, 0.125, -0.125, 0.375, -0.375, 1.25, -1.25, 1.75, -1.75] + [0.0] * 20,
     [7, 15, 6, 14, 0, 0, 1, 9, 4, 12, 5, 13] + [0] * 20, 126),
    ([7, -7, 5, -5, 1, -1, 0.5, -0.5] + [0.0] * 24,
     [5, 13, 4, 12, 1, 9, 0, 0] + [0] * 24, 128),
]


def mxfp4_hand_cases():
    w = np.array([g[0] for g in MXFP4_HAND], np.float32).reshape(1, -1)
    codes = np.array([g[1] for g in MXFP4_HAND], np.int64).reshape(1, -1)
    wb = bf16_bits(w)
    assert np.array_equal(torch.from_numpy(wb.astype(np.int16)).view(torch.bfloat16).float().numpy(), w)
    return {"mxfp4_hand_w": wb, "mxfp4_hand_wq": pack(codes, 4),
            "mxfp4_hand_scales": np.array([[g[2] for g in MXFP4_HAND]], np.uint8)}


# MLX to_fp8 on the ROCm backend (convert_fp8.hip:18-66) by hand: value ->
# code.  The float's exponent e and 23-bit fraction f: e < -9 -> signed zero;
# e > 8 -> 0x7E; else exponent field e + 7 and mantissa (f + 2^19) >> 20
# (half-up), a mantissa of 8 carrying into the exponent (past 15 -> 0x7E);
# an exponent field <= 0 instead takes (2^23 + f) >> (21 - field).
E4M3_HAND = [
    (1.0, 0x38),                  # field 7, mantissa 0
    (1.0625, 0x39),               # 1 + 0.5/8: tie, half-up -> 1 (to-even would be 0)
    (1.1875, 0x3A),               # 1 + 1.5/8 -> 2
    (1.3125, 0x3B),               # 1 + 2.5/8: tie -> 3 (to-even would be 2)
    (-3.0, 0xC4),                 # 1.5 * 2^1: field 8, mantissa 4, sign
    (448.0, 0x7E),                # 1.75 * 2^8, the largest finite
    (449.0, 0x7E),                # rounds to 1.75 * 2^8
    (464.0, 0x7F),                # 1.8125 * 2^8 -> mantissa 7 in field 15: the NaN code
    (495.0, 0x7F),
    (496.0, 0x7E),                # mantissa 8 carries to field 16 -> 0x7E
    (1.0e6, 0x7E), (float("inf"), 0x7E), (float("-inf"), 0xFE), (float("nan"), 0x7F),
    (0.0, 0x00), (-0.0, 0x80),
    (2.0 ** -6, 0x08),            # smallest normal
    (2.0 ** -9, 0x01),            # smallest subnormal: field -2 -> (2^23) >> 23 = 1
    (2.0 ** -10, 0x00),           # e = -10 < -9: zero
    (1.5 * 2.0 ** -10, 0x00),     # also zero (nearest would be 2^-9)
    (1.75 * 2.0 ** -9, 0x01),     # field -2: (1.75 * 2^23) >> 23 = 1, truncated
    (1.5 * 2.0 ** -8, 0x03),      # field -1: (1.5 * 2^23) >> 22 = 3
    (1.96875 * 2.0 ** -8, 0x07),  # mantissa carries to field 0, then (1.96875 * 2^23) >> 21 = 7
    (1.96875 * 2.0 ** -9, 0x03),  # carries to field -1: >> 22 = 3
    (1.96875 * 2.0 ** -7, 0x08),  # carries to field 1: the smallest normal
]

# mxfp8 groups (32 values): G1 max 448 -> scale bf16(448/448) = 1, exponent 0
# (byte 127), codes = to_fp8(w); G2 max 1 -> bf16(1/448) = 1.140625 * 2^-9,
# log2 = -8.81 -> bf16 -8.8125 -> round -9, 2^-9 < scale -> exponent -8 (byte
# 119), codes = to_fp8(w * 256): 1 -> 256 = 0x78, -0.5 -> -128 = 0xF0,
# 0.25 -> 64 = 0x68, 2^-16 -> 2^-8 = 2 * 2^-9 = 0x02; G3 zeros -> byte 127, codes 0.
MXFP8_HAND = [
    ([448.0, -448.0, 1.0, 1.0625, 1.3125, -3.0, 2.0 ** -9, 1.75 * 2.0 ** -9, 1.5 * 2.0 ** -8,
      1.96875 * 2.0 ** -8, 2.0 ** -6, 0.0, -0.0] + [0.0] * 19,
     [0x7E, 0xFE, 0x38, 0x39, 0x3B, 0xC4, 0x01, 0x01, 0x03, 0x07, 0x08, 0x00, 0x80] + [0x00] * 19, 127),
    ([1.0, -0.5, 0.25, 2.0 ** -16] + [0.0] * 28, [0x78, 0xF0, 0x68, 0x02] + [0x00] * 28, 119),
    ([0.0] * 32, [0x00] * 32, 127),
]

# nvfp4 groups (16 values, no global scale): N1 max 6 -> bf16(6/6) = 1 ->
# to_fp8 0x38, divisor 1, codes = first nearest FP4_LUT index; N2 max 7 ->
# bf16(7/6) = 1.1640625 -> to_fp8 0x39 (1.125): 7/1.125 -> bf16 6.21875 -> 6
# (7), 1/1.125 -> 0.88671875 -> 1 (2), -2.8125/1.125 = -2.5: tie -> -2 (12),
# 0.5625/1.125 = 0.5 (1); N3 zeros -> scale 0, 0/0 -> NaN -> code 0; N4 max
# 6 * 2^-12 -> 2^-12 -> to_fp8 0 -> w/0 = +-inf -> code 0.
NVFP4_HAND = [
    ([6.0, -6.0, 5.0, 0.25, -0.25, 0.75, -0.75, 2.5, 3.5, 1.25, 1.75, -5.0, 0.0, -0.0, 1.0, -1.0],
     [7, 15, 6, 0, 0, 1, 9, 4, 5, 2, 3, 14, 0, 0, 2, 10], 0x38),
    ([7.0, 1.0, -2.8125, 0.5625] + [0.0] * 12, [7, 2, 12, 1] + [0] * 12, 0x39),
    ([0.0] * 16, [0] * 16, 0x00),
    ([6.0 * 2.0 ** -12, -2.0 ** -12] + [0.0] * 14, [0] * 16, 0x00),
]


def fp_hand_cases():
    enc = np.array([v for v, _ in E4M3_HAND], np.float32)
    out = {"e4m3_hand_in": enc, "e4m3_hand_code": np.array([c for _, c in E4M3_HAND], np.uint8)}
    w = np.array([g[0] for g in MXFP8_HAND], np.float32)
    wb = bf16_bits(w)
    assert np.array_equal(torch.from_numpy(wb.astype(np.int16)).view(torch.bfloat16).float().numpy(), w)
    out["mxfp8_hand_w"] = wb
    out["mxfp8_hand_wq"] = np.ascontiguousarray(np.array([g[1] for g in MXFP8_HAND], np.uint8)).view(np.uint32)
    out["mxfp8_hand_scales"] = np.array([[g[2]] for g in MXFP8_HAND], np.uint8)
    w = np.array([g[0] for g in NVFP4_HAND], np.float32)
    wb = bf16_bits(w)
    assert np.array_equal(torch.from_numpy(wb.astype(np.int16)).view(torch.bfloat16).float().numpy(), w)
    out["nvfp4_hand_w"] = wb
    out["nvfp4_hand_wq"] = pack(np.array([g[1] for g in NVFP4_HAND], np.int64), 4)
    out["nvfp4_hand_scales"] = np.array([[g[2]] for g in NVFP4_HAND], np.uint8)
    return out


def dequant_d2_cases():
    rng = np.random.default_rng(2248)
    n = 4096
    q = rng.integers(0, 256, n).astype(np.float32)
    # scales/biases with mantissa bits that put q*s and q*s+b on bf16 halfway points
    s = bf16_bits(rng.standard_normal(n).astype(np.float32) * np.float32(0.01))
    b = bf16_bits(rng.standard_normal(n).astype(np.float32) * np.float32(0.05))
    st = torch.from_numpy(s.astype(np.int16)).view(torch.bfloat16)
    bt = torch.from_numpy(b.astype(np.int16)).view(torch.bfloat16)
    qt = torch.from_numpy(q).to(torch.bfloat16)
    d2 = (qt * st) + bt
    return q.astype(np.uint32), s, b, d2.view(torch.int16).numpy().astype(np.uint16)


def main():
    out = {"mxfp4_table": mxfp4_table()}
    for bits in (2, 4, 6, 8):
        for gs in (32, 64, 128):
            w, wq, s, b = affine_ramps(bits, gs)
            out[f"ramp_w_b{bits}_g{gs}"] = w
            out[f"ramp_wq_b{bits}_g{gs}"] = wq
            out[f"ramp_s_b{bits}_g{gs}"] = s
            out[f"ramp_b_b{bits}_g{gs}"] = b
    out.update(affine_hand_cases())
    out.update(mxfp4_hand_cases())
    out.update(fp_hand_cases())
    q, s, b, d2 = dequant_d2_cases()
    out.update(d2_q=q, d2_s=s, d2_b=b, d2_out=d2)
    np.savez_compressed(os.path.join(HERE, "kat.npz"), **out)
    print("wrote", os.path.join(HERE, "kat.npz"), {k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    main()
