"""numpy restatement of MLX's CPU quantized matmul for every element type and
code width (float16 / bfloat16 / float32 activations and scales; affine
codes of 2, 3, 4, 5, 6 and 8 bits; mxfp4; both transposes).

TEST INFRASTRUCTURE ONLY (the checker of the general kernel,
mlxcel_amd/csrc/qmm_gen.hip); the product package never imports it.

Reference: overlays/cpu/mlx/backend/cpu/quantized.cpp
  - extract_bits (107-137): codes of 3, 5 and 6 bits are a little-endian bit
    stream over bytes (3 bytes hold 8 codes of 3 bits, 5 bytes 8 of 5, 3
    bytes 4 of 6); the power-of-two widths (the `wi & bitmask; wi >>= bits`
    loops of 139-257) read the same stream.  So code i of a packed row sits
    at bits [i*bits, (i+1)*bits) of the row's bytes, low bit first.
  - _qmm (139-197, transpose=false) and _qmm_t (199-257, transpose=true):
    float accumulator, `x * (scale * q + bias)` with x, scale, bias converted
    from T to float (exact for bfloat16 / float16 / float32), result cast to T.
  - fp_qmm_t (550-597) with the e2m1 table and e8m0 scales (73-105) for mxfp4.
The promotion of x / scales / biases to one type T (overlays/rocm/mlx/
ops.cpp:4974-4992) is exact for these types, so the inputs here are float32
arrays of the values; the sum is taken in float64 and the caller rounds to T.
"""
from __future__ import annotations

import numpy as np

E2M1 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                 -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0], dtype=np.float64)


def unpack_codes(wq: np.ndarray, bits: int, n: int) -> np.ndarray:
    """Codes of each packed row: [..., words] uint32 -> [..., n] int64."""
    wq = np.ascontiguousarray(wq, dtype=np.uint32)
    by = wq.view(np.uint8).reshape(wq.shape[:-1] + (wq.shape[-1] * 4,))
    bitarr = np.unpackbits(by, axis=-1, bitorder="little")  # bit j of the row stream
    bitarr = bitarr[..., : n * bits].reshape(wq.shape[:-1] + (n, bits)).astype(np.int64)
    return (bitarr << np.arange(bits, dtype=np.int64)).sum(axis=-1)


def pack_codes(codes: np.ndarray, bits: int) -> np.ndarray:
    """Inverse of unpack_codes: [..., n] codes (n * bits a multiple of 32) -> [..., n*bits/32] uint32."""
    codes = np.asarray(codes, dtype=np.int64)
    n = codes.shape[-1]
    assert (n * bits) % 32 == 0
    bitarr = ((codes[..., None] >> np.arange(bits, dtype=np.int64)) & 1).astype(np.uint8)
    bitarr = bitarr.reshape(codes.shape[:-1] + (n * bits,))
    by = np.packbits(bitarr, axis=-1, bitorder="little")
    return np.ascontiguousarray(by).view(np.uint32).reshape(codes.shape[:-1] + (n * bits // 32,))


def e8m0_to_f64(s: np.ndarray) -> np.ndarray:
    """2^(s-127); s == 255 -> NaN (quantized.cpp:97-101 builds the bf16 of it)."""
    s = np.asarray(s, dtype=np.int64)
    v = np.ldexp(1.0, s - 127)
    return np.where(s == 255, np.nan, v)


def dequantize(wq, scales, biases, group_size: int, bits: int, n: int, mode: str = "affine") -> np.ndarray:
    """Dequantized rows in float64: [..., n] from codes grouped along the last axis."""
    q = unpack_codes(wq, bits, n).astype(np.float64)
    g = np.repeat(np.asarray(scales, dtype=np.float64), group_size, axis=-1)
    if mode == "mxfp4":
        return E2M1[q.astype(np.int64)] * np.repeat(e8m0_to_f64(scales), group_size, axis=-1)
    b = np.repeat(np.asarray(biases, dtype=np.float64), group_size, axis=-1)
    return g * q + b


def dequantize_graph(wq, scales, biases, group_size: int, bits: int, n: int, ts: str, to: str) -> np.ndarray:
    """mlx::core::dequantize, affine (overlays/rocm/mlx/ops.cpp:5494-5586, then
    astype(out_type) at 5788-5793): the codes times the scales in the scales'
    type T, plus the biases in T, each op computed in float32 and rounded to T,
    then cast to the output type:  To(T(f32(T(f32(q * s)) + b))).
    scales / biases hold values of type ts; returns float64 values of type to."""
    q = unpack_codes(wq, bits, n).astype(np.float64)
    sc = np.repeat(np.asarray(scales, dtype=np.float64), group_size, axis=-1)
    bi = np.repeat(np.asarray(biases, dtype=np.float64), group_size, axis=-1)
    prod = round_to(round_to(q * sc, "float32"), ts)
    tot = round_to(round_to(prod + bi, "float32"), ts)
    return round_to(tot, to)


def mxfp4_dequantize_graph(wq, scales, n: int, to: str) -> np.ndarray:
    """mxfp4 dequantize to float16 / float32 (ops.cpp:5646-5695 with out_type):
    the scale 2^(s-127) is formed in the output type (rounded to it), s == 255
    gives NaN, and LUT[q] * scale is rounded once."""
    q = unpack_codes(wq, 4, n)
    s = np.asarray(scales, dtype=np.int64)
    scale = np.where(s == 255, np.nan, np.ldexp(1.0, s - 127))
    scale = round_to(scale, to)
    return round_to(E2M1[q] * np.repeat(scale, 32, axis=-1), to)


def qmm(x, wq, scales, biases, transpose: bool, group_size: int, bits: int, mode: str = "affine") -> np.ndarray:
    """y = x @ W^T (transpose) or x @ W for 2-D W, float64.

    x: [..., M, K] float values; transpose: wq [N, K*bits/32], scales/biases
    [N, K/gs]; otherwise wq [K, N*bits/32], scales/biases [K, N/gs]."""
    x = np.asarray(x, dtype=np.float64)
    if transpose:
        K = x.shape[-1]
        w = dequantize(wq, scales, biases, group_size, bits, K, mode)  # [N, K]
        return x @ w.T
    N = wq.shape[-1] * 32 // bits
    w = dequantize(wq, scales, biases, group_size, bits, N, mode)  # [K, N]
    return x @ w


def gather_qmm(x, wq, scales, biases, lhs, rhs, transpose: bool, group_size: int, bits: int,
               mode: str = "affine") -> np.ndarray:
    """x: [X, M, K]; wq/scales/biases: [E, ...]; lhs/rhs: [B] -> [B, M, N] float64."""
    out = []
    for l, r in zip(np.asarray(lhs).reshape(-1), np.asarray(rhs).reshape(-1)):
        out.append(qmm(x[int(l)], wq[int(r)], scales[int(r)], None if biases is None else biases[int(r)],
                       transpose, group_size, bits, mode))
    return np.stack(out)


def round_to(y: np.ndarray, dtype: str) -> np.ndarray:
    """float64 -> the result type T, round to nearest even, returned as float64 values."""
    if dtype == "float32":
        return y.astype(np.float32).astype(np.float64)
    if dtype == "float16":
        return y.astype(np.float16).astype(np.float64)
    # bfloat16: round the float32 value to the upper 16 bits, ties to even
    f = y.astype(np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return (u.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
