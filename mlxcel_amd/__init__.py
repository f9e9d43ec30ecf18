"""mlxcel_amd — MI355X (gfx950) quantized-matmul hot path for mlxcel / MLX.

The product is the C-ABI library ``libmlxq.so`` (``include/mlxq.h``); this
package holds its HIP sources (``csrc/``), the build script, and a Python
mirror of the reference operator interface (``ops``).
"""
from .ops import (clear_cache, dequantize, fused_moe_expert, fused_moe_geglu, gather_qmm,  # noqa: F401
                  get_cache_memory, quantize, quantized_linear, quantized_matmul,
                  quantized_matmul_matches_dense_gemm, quantized_matmul_multi, workspace_reserve)
from ._lib import LIB_PATH, load as load_library  # noqa: F401
from . import loader  # noqa: F401,E402  (MLX-quantized safetensors -> device planes)

__all__ = ["quantized_matmul", "quantized_matmul_multi", "quantized_linear",
           "quantized_matmul_matches_dense_gemm", "gather_qmm", "dequantize", "quantize",
           "fused_moe_expert", "fused_moe_geglu", "workspace_reserve", "get_cache_memory", "clear_cache",
           "loader", "load_library", "LIB_PATH"]
