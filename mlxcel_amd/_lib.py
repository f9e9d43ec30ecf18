"""ctypes binding of ``libmlxq.so`` (the C ABI in ``include/mlxq.h``).

This is the same binding a Python caller of the reference's FFI would write
(the Rust crate under ``rust/mlxq-sys`` binds the same symbols).  Loading fails loudly when the
library has not been built: there is no fallback path.
"""
from __future__ import annotations

import ctypes
import os

MAX_DIMS = 8
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libmlxq.so")

# mlxq_status
OK, EINVAL, EUNSUPPORTED, EHIP, ENOMEM = 0, 1, 2, 3, 4

# mlxq_dtype (mlx::core::Dtype order)
BOOL, UINT8, UINT16, UINT32, UINT64, INT8, INT16, INT32, INT64 = range(9)
FLOAT16, FLOAT32, FLOAT64, BFLOAT16, COMPLEX64 = 9, 10, 11, 12, 13


class MlxqArray(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("ndim", ctypes.c_int32),
        ("shape", ctypes.c_int64 * MAX_DIMS),
        ("strides", ctypes.c_int64 * MAX_DIMS),
    ]


SYMBOLS = (
    "mlxq_last_error",
    "mlxq_version",
    "mlxq_quantized_matmul",
    "mlxq_quantized_matmul_shape",
    "mlxq_quantized_matmul_multi",
    "mlxq_quantized_linear",
    "mlxq_quantized_matmul_matches_dense_gemm",
    "mlxq_gather_qmm",
    "mlxq_gather_qmm_shape",
    "mlxq_dequantize",
    "mlxq_quantize",
    "mlxq_fused_moe_expert",
    "mlxq_fused_moe_geglu",
    "mlxq_workspace_reserve",
    "mlxq_get_cache_memory",
    "mlxq_clear_cache",
    "mlxq_reload_options",
    "mlxq_quantized_matmul_noalloc",
)

_lib = None


class LibraryNotBuilt(RuntimeError):
    pass


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise LibraryNotBuilt(
            f"{LIB_PATH} is missing: build it with `python -m mlxcel_amd.build` "
            "(the quantized matmul has no CPU fallback)")
    lib = ctypes.CDLL(LIB_PATH)
    A = ctypes.POINTER(MlxqArray)
    P = ctypes.c_void_p
    B = ctypes.c_bool
    I32 = ctypes.c_int32
    S = ctypes.c_char_p
    lib.mlxq_last_error.restype = ctypes.c_char_p
    lib.mlxq_last_error.argtypes = []
    lib.mlxq_version.restype = ctypes.c_char_p
    lib.mlxq_version.argtypes = []
    lib.mlxq_quantized_matmul.argtypes = [A, A, A, A, B, I32, I32, S, A, P]
    lib.mlxq_quantized_matmul_shape.argtypes = [A, A, A, A, B, I32, I32, S, ctypes.POINTER(I32),
                                                ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(I32)]
    AA = ctypes.POINTER(A)
    lib.mlxq_quantized_matmul_multi.argtypes = [A, I32, AA, AA, AA, I32, I32, S, AA, P]
    lib.mlxq_quantized_linear.argtypes = [A, A, A, A, A, I32, I32, S, A, P]
    lib.mlxq_quantized_matmul_matches_dense_gemm.argtypes = [A, A, A, A, I32, I32]
    lib.mlxq_gather_qmm.argtypes = [A, A, A, A, A, A, B, I32, I32, B, S, A, A, P]
    lib.mlxq_gather_qmm_shape.argtypes = [A, A, A, A, A, A, B, I32, I32, S, ctypes.POINTER(I32),
                                          ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(I32)]
    lib.mlxq_dequantize.argtypes = [A, A, A, I32, I32, S, I32, A, P]
    lib.mlxq_quantize.argtypes = [A, I32, I32, S, A, A, A, P]
    lib.mlxq_fused_moe_expert.argtypes = [A] * 12 + [I32] * 6 + [A, P]
    lib.mlxq_fused_moe_geglu.argtypes = [A] * 12 + [I32] * 6 + [A, P]
    lib.mlxq_quantized_matmul_noalloc.argtypes = [A, A, A, A, B, I32, I32, S, A, P]
    lib.mlxq_workspace_reserve.argtypes = [ctypes.c_size_t, P]
    lib.mlxq_get_cache_memory.argtypes = []
    lib.mlxq_clear_cache.argtypes = []
    lib.mlxq_reload_options.argtypes = []
    for name in SYMBOLS[2:]:
        getattr(lib, name).restype = ctypes.c_int
    lib.mlxq_get_cache_memory.restype = ctypes.c_size_t
    lib.mlxq_reload_options.restype = None
    _lib = lib
    return lib


def last_error() -> str:
    return load().mlxq_last_error().decode()
