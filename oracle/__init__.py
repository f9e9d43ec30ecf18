"""ctypes view of the CPU oracle (``liboracle.so`` built from ``mlxq_oracle.c``).

TEST INFRASTRUCTURE ONLY.  Imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` as the checker; the product
package ``mlxcel_amd`` never imports it.

Arrays are numpy; bf16 tensors travel as ``uint16`` bit patterns.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None


def build() -> None:
    """Compile liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE, "-B", "liboracle.so"], check=True)


def build_info() -> dict:
    """Compiler and flags liboracle.so is built with (the Makefile's CC and
    CFLAGS), for reports that time the oracle."""
    cflags = ""
    for line in open(os.path.join(_HERE, "Makefile")):
        if line.startswith("CFLAGS"):
            cflags = line.split("=", 1)[1].strip()
    cc = os.environ.get("CC", "gcc")
    try:
        ver = subprocess.run([cc, "--version"], capture_output=True, text=True).stdout.splitlines()[0]
    except Exception:
        ver = cc
    return {"compiler": ver, "cflags": cflags}


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int


def _declare(l: ctypes.CDLL) -> None:
    sig = {
        "oracle_f32_to_bf16_n": [_P, _P, _I64],
        "oracle_bf16_to_f32_n": [_P, _P, _I64],
        "oracle_affine_quantize": [_P, _I64, _I64, _I, _I, _P, _P, _P],
        "oracle_affine_quantize_t": [_P, _I, _I64, _I64, _I, _I, _P, _P, _P],
        "oracle_affine_dequantize": [_P, _P, _P, _I64, _I64, _I, _I, _I, _P],
        "oracle_mxfp4_quantize": [_P, _I64, _I64, _P, _P],
        "oracle_mxfp4_dequantize": [_P, _P, _I64, _I64, _P],
        "oracle_qmm_t_affine": [_P, _P, _P, _P, _I64, _I64, _I64, _I, _I, _P],
        "oracle_qmm_affine": [_P, _P, _P, _P, _I64, _I64, _I64, _I, _I, _P],
        "oracle_fp_qmm_t_mxfp4": [_P, _P, _P, _I64, _I64, _I64, _P],
        "oracle_gather_qmm_t": [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I, _I, _I, _P],
        "oracle_affine_dequantize_f32": [_P, _P, _P, _I64, _I64, _I, _I, _P],
        "oracle_fused_moe": [_P] * 12 + [_I64] * 4 + [_I] * 4 + [_P],
        "oracle_e4m3_encode_n": [_P, _P, _I64],
        "oracle_e4m3_decode_n": [_P, _P, _I64],
        "oracle_mxfp8_quantize": [_P, _I64, _I64, _P, _P],
        "oracle_mxfp8_dequantize": [_P, _P, _I64, _I64, _P],
        "oracle_nvfp4_quantize": [_P, _I64, _I64, _P, _P],
        "oracle_nvfp4_dequantize": [_P, _P, _I64, _I64, _P],
    }
    for name, args in sig.items():
        fn = getattr(l, name)
        fn.argtypes = args
        fn.restype = None if name.endswith("_n") else _I
    l.oracle_f32_to_f16.argtypes = [ctypes.c_float]
    l.oracle_f32_to_f16.restype = ctypes.c_uint16
    l.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
    l.oracle_f16_to_f32.restype = ctypes.c_float
    l.oracle_e8m0_to_bf16.argtypes = [ctypes.c_uint8]
    l.oracle_e8m0_to_bf16.restype = ctypes.c_uint16


def _ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise ValueError(f"oracle {what}: unsupported arguments")


# ---- bf16 helpers -----------------------------------------------------------

def f32_to_bf16(a) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    lib().oracle_f32_to_bf16_n(_ptr(a), _ptr(out), a.size)
    return out


def bf16_to_f32(a) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.uint16)
    out = np.empty(a.shape, dtype=np.float32)
    lib().oracle_bf16_to_f32_n(_ptr(a), _ptr(out), a.size)
    return out


# ---- quantize / dequantize --------------------------------------------------

def affine_quantize(w_bf16: np.ndarray, group_size: int = 64, bits: int = 4):
    w = np.ascontiguousarray(w_bf16, dtype=np.uint16)
    K = w.shape[-1]
    rows = w.size // K
    wq = np.empty(w.shape[:-1] + (K * bits // 32,), dtype=np.uint32)
    s = np.empty(w.shape[:-1] + (K // group_size,), dtype=np.uint16)
    b = np.empty_like(s)
    _check(lib().oracle_affine_quantize(_ptr(w), rows, K, group_size, bits, _ptr(wq), _ptr(s), _ptr(b)),
           "affine_quantize")
    return wq, s, b


_QDT = {"bfloat16": (0, np.uint16), "float16": (1, np.float16), "float32": (2, np.float32)}


def affine_quantize_t(w: np.ndarray, dtype: str, group_size: int = 64, bits: int = 4):
    """Typed affine quantize: w holds bfloat16 bits (uint16), float16 or
    float32 values per `dtype`; scales / biases come back in the same form."""
    code, npdt = _QDT[dtype]
    w = np.ascontiguousarray(w, dtype=npdt)
    K = w.shape[-1]
    rows = w.size // K
    wq = np.empty(w.shape[:-1] + (K * bits // 32,), dtype=np.uint32)
    s = np.empty(w.shape[:-1] + (K // group_size,), dtype=npdt)
    b = np.empty_like(s)
    _check(lib().oracle_affine_quantize_t(_ptr(w), code, rows, K, group_size, bits, _ptr(wq), _ptr(s), _ptr(b)),
           "affine_quantize_t")
    return wq, s, b


def f32_to_f16_bits(v: float) -> int:
    return int(lib().oracle_f32_to_f16(float(v)))


def f16_bits_to_f32(h: int) -> float:
    return float(lib().oracle_f16_to_f32(int(h)))


def affine_dequantize(wq, scales, biases, group_size: int = 64, bits: int = 4, rounding: int = 2):
    wq = np.ascontiguousarray(wq, dtype=np.uint32)
    scales = np.ascontiguousarray(scales, dtype=np.uint16)
    biases = np.ascontiguousarray(biases, dtype=np.uint16)
    K = wq.shape[-1] * 32 // bits
    rows = wq.size // wq.shape[-1]
    out = np.empty(wq.shape[:-1] + (K,), dtype=np.uint16)
    _check(lib().oracle_affine_dequantize(_ptr(wq), _ptr(scales), _ptr(biases), rows, K,
                                          group_size, bits, rounding, _ptr(out)),
           "affine_dequantize")
    return out


def affine_dequantize_f32(wq, scales, biases, group_size: int = 64, bits: int = 4):
    """s * q + b in float32 (no bf16 rounding)."""
    wq = np.ascontiguousarray(wq, dtype=np.uint32)
    scales = np.ascontiguousarray(scales, dtype=np.uint16)
    biases = np.ascontiguousarray(biases, dtype=np.uint16)
    K = wq.shape[-1] * 32 // bits
    rows = wq.size // wq.shape[-1]
    out = np.empty(wq.shape[:-1] + (K,), dtype=np.float32)
    _check(lib().oracle_affine_dequantize_f32(_ptr(wq), _ptr(scales), _ptr(biases), rows, K, group_size, bits,
                                              _ptr(out)), "affine_dequantize_f32")
    return out


def e8m0_to_bf16(s: int) -> int:
    return int(lib().oracle_e8m0_to_bf16(s))


def mxfp4_quantize(w_bf16: np.ndarray):
    w = np.ascontiguousarray(w_bf16, dtype=np.uint16)
    K = w.shape[-1]
    rows = w.size // K
    wq = np.empty(w.shape[:-1] + (K // 8,), dtype=np.uint32)
    s = np.empty(w.shape[:-1] + (K // 32,), dtype=np.uint8)
    _check(lib().oracle_mxfp4_quantize(_ptr(w), rows, K, _ptr(wq), _ptr(s)), "mxfp4_quantize")
    return wq, s


def mxfp4_dequantize(wq, scales):
    wq = np.ascontiguousarray(wq, dtype=np.uint32)
    scales = np.ascontiguousarray(scales, dtype=np.uint8)
    K = wq.shape[-1] * 8
    rows = wq.size // wq.shape[-1]
    out = np.empty(wq.shape[:-1] + (K,), dtype=np.uint16)
    _check(lib().oracle_mxfp4_dequantize(_ptr(wq), _ptr(scales), rows, K, _ptr(out)), "mxfp4_dequantize")
    return out


# ---- matmuls ----------------------------------------------------------------

def qmm_t_affine(x_bf16, wq, scales, biases, group_size: int = 64, bits: int = 4):
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    wq = np.ascontiguousarray(wq, dtype=np.uint32)
    scales = np.ascontiguousarray(scales, dtype=np.uint16)
    biases = np.ascontiguousarray(biases, dtype=np.uint16)
    K = x.shape[-1]
    M = x.size // K
    N = wq.shape[0]
    out = np.empty(x.shape[:-1] + (N,), dtype=np.uint16)
    _check(lib().oracle_qmm_t_affine(_ptr(x), _ptr(wq), _ptr(scales), _ptr(biases), M, N, K,
                                     group_size, bits, _ptr(out)), "qmm_t_affine")
    return out


def qmm_affine(x_bf16, wq, scales, biases, group_size: int = 64, bits: int = 4):
    """transpose=False: w is [K, N*bits/32]."""
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    wq = np.ascontiguousarray(wq, dtype=np.uint32)
    scales = np.ascontiguousarray(scales, dtype=np.uint16)
    biases = np.ascontiguousarray(biases, dtype=np.uint16)
    K = x.shape[-1]
    M = x.size // K
    N = wq.shape[1] * 32 // bits
    out = np.empty(x.shape[:-1] + (N,), dtype=np.uint16)
    _check(lib().oracle_qmm_affine(_ptr(x), _ptr(wq), _ptr(scales), _ptr(biases), M, N, K,
                                   group_size, bits, _ptr(out)), "qmm_affine")
    return out


def fp_qmm_t_mxfp4(x_bf16, wq, scales):
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    wq = np.ascontiguousarray(wq, dtype=np.uint32)
    scales = np.ascontiguousarray(scales, dtype=np.uint8)
    K = x.shape[-1]
    M = x.size // K
    N = wq.shape[0]
    out = np.empty(x.shape[:-1] + (N,), dtype=np.uint16)
    _check(lib().oracle_fp_qmm_t_mxfp4(_ptr(x), _ptr(wq), _ptr(scales), M, N, K, _ptr(out)),
           "fp_qmm_t_mxfp4")
    return out


def gather_qmm_t(x_bf16, wq, scales, biases, lhs, rhs, group_size=64, bits=4, mode="affine"):
    """x: [X, M, K]; w: [E, N, Kp]; lhs/rhs: [B] -> out [B, M, N]."""
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    wq = np.ascontiguousarray(wq, dtype=np.uint32)
    lhs = np.ascontiguousarray(lhs, dtype=np.uint32).reshape(-1)
    rhs = np.ascontiguousarray(rhs, dtype=np.uint32).reshape(-1)
    assert lhs.size == rhs.size
    M, K = x.shape[-2], x.shape[-1]
    N = wq.shape[-2]
    if mode == "affine":
        scales = np.ascontiguousarray(scales, dtype=np.uint16)
        biases = np.ascontiguousarray(biases, dtype=np.uint16)
        bptr, m = _ptr(biases), 0
    else:
        scales = np.ascontiguousarray(scales, dtype=np.uint8)
        bptr, m = None, 1
        group_size = 32
    out = np.empty((lhs.size, M, N), dtype=np.uint16)
    _check(lib().oracle_gather_qmm_t(_ptr(x), _ptr(wq), _ptr(scales), bptr, _ptr(lhs), _ptr(rhs),
                                     lhs.size, M, N, K, group_size, bits, m, _ptr(out)),
           "gather_qmm_t")
    return out


def fused_moe(x_bf16, indices, scores, gate, up, down, group_size: int = 64, gu_bits: int = 4,
              d_bits: int = 4, act: str = "swiglu") -> np.ndarray:
    """Dense fp64 restatement of the reference's fused single-token decode MoE
    (``fused_moe_expert_kernel`` / ``fused_moe_geglu_kernel``): gate, up and
    down are ``(wq, scales, biases)`` stacks over experts; returns float32
    ``(din,)``, not rounded."""
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16).reshape(-1)
    idx = np.ascontiguousarray(np.asarray(indices).astype(np.int64).astype(np.uint32)).reshape(-1)
    sc = np.ascontiguousarray(scores, dtype=np.float32).reshape(-1)
    gw, gs_, gb = (np.ascontiguousarray(a) for a in gate)
    uw, us, ub = (np.ascontiguousarray(a) for a in up)
    dw, ds, db = (np.ascontiguousarray(a) for a in down)
    E, dff = gw.shape[0], gw.shape[1]
    din = x.size
    assert idx.size == sc.size and gw.shape == uw.shape and dw.shape[:2] == (E, din)
    out = np.empty(din, dtype=np.float32)
    _check(lib().oracle_fused_moe(_ptr(x), _ptr(idx), _ptr(sc), _ptr(gw), _ptr(gs_), _ptr(gb), _ptr(uw),
                                  _ptr(us), _ptr(ub), _ptr(dw), _ptr(ds), _ptr(db), din, dff, idx.size, E,
                                  group_size, gu_bits, d_bits, 1 if act == "geglu" else 0, _ptr(out)),
           "fused_moe")
    return out


# ---- seeded inputs (numpy Philox normal draws in float32, then bf16 RNE) ----

def normal_bf16(shape, std: float, seed: int) -> np.ndarray:
    """Deterministic N(0, std^2) draws rounded to bf16, identical on every host."""
    n = int(np.prod(shape))
    rng = np.random.Generator(np.random.Philox(seed))
    v = rng.standard_normal(n, dtype=np.float32) * np.float32(std)
    return f32_to_bf16(v).reshape(shape)


# ---- fp8 e4m3, mxfp8, nvfp4 -------------------------------------------------

def e4m3_encode(a) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint8)
    lib().oracle_e4m3_encode_n(_ptr(a), _ptr(out), a.size)
    return out


def e4m3_decode(c) -> np.ndarray:
    c = np.ascontiguousarray(c, dtype=np.uint8)
    out = np.empty(c.shape, dtype=np.float32)
    lib().oracle_e4m3_decode_n(_ptr(c), _ptr(out), c.size)
    return out


def _fp_quantize(fn, w_bf16, gs, bits):
    w = np.ascontiguousarray(w_bf16, dtype=np.uint16)
    K = w.shape[-1]
    rows = w.size // K
    wq = np.empty(w.shape[:-1] + (K * bits // 32,), dtype=np.uint32)
    s = np.empty(w.shape[:-1] + (K // gs,), dtype=np.uint8)
    _check(fn(_ptr(w), rows, K, _ptr(wq), _ptr(s)), "fp quantize")
    return wq, s


def _fp_dequantize(fn, wq, scales, bits):
    wq = np.ascontiguousarray(wq, dtype=np.uint32)
    scales = np.ascontiguousarray(scales, dtype=np.uint8)
    K = wq.shape[-1] * 32 // bits
    rows = wq.size // wq.shape[-1]
    out = np.empty(wq.shape[:-1] + (K,), dtype=np.uint16)
    _check(fn(_ptr(wq), _ptr(scales), rows, K, _ptr(out)), "fp dequantize")
    return out


def mxfp8_quantize(w_bf16):
    return _fp_quantize(lib().oracle_mxfp8_quantize, w_bf16, 32, 8)


def mxfp8_dequantize(wq, scales):
    return _fp_dequantize(lib().oracle_mxfp8_dequantize, wq, scales, 8)


def nvfp4_quantize(w_bf16):
    return _fp_quantize(lib().oracle_nvfp4_quantize, w_bf16, 16, 4)


def nvfp4_dequantize(wq, scales):
    return _fp_dequantize(lib().oracle_nvfp4_dequantize, wq, scales, 4)
