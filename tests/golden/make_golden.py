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
    q, s, b, d2 = dequant_d2_cases()
    out.update(d2_q=q, d2_s=s, d2_b=b, d2_out=d2)
    np.savez_compressed(os.path.join(HERE, "kat.npz"), **out)
    print("wrote", os.path.join(HERE, "kat.npz"), {k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    main()
