"""MLX-style quantized ops over torch device tensors, backed by ``libmlxq.so``.

Mirrors the reference operator interface (the MLX ops mlxcel binds through
``ffi::quantized_matmul`` / ``ffi::gather_qmm`` / ``ffi::dequantize`` /
``ffi::quantize_weights_*``; src/lib/mlxcel-core/src/lib.rs:1374-1416,
overlays/rocm/mlx/ops.cpp:4955-5008, 5454-5492, 5753-5805, 5841-5948): same
names, argument meaning, defaults and output shapes/dtypes.  Errors follow
MLX's Python binding: argument errors raise ``ValueError`` with the
reference's message; combinations this library does not implement raise
``NotImplementedError``.

Torch is used only for device memory and the current HIP stream; all
arithmetic happens in the HIP kernels.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Sequence

import torch

from . import _lib

_TORCH_TO_MLXQ = {
    torch.bool: _lib.BOOL,
    torch.uint8: _lib.UINT8,
    torch.uint16: _lib.UINT16,
    torch.uint32: _lib.UINT32,
    torch.uint64: _lib.UINT64,
    torch.int8: _lib.INT8,
    torch.int16: _lib.INT16,
    torch.int32: _lib.INT32,
    torch.int64: _lib.INT64,
    torch.float16: _lib.FLOAT16,
    torch.float32: _lib.FLOAT32,
    torch.float64: _lib.FLOAT64,
    torch.bfloat16: _lib.BFLOAT16,
}
_MLXQ_TO_TORCH = {v: k for k, v in _TORCH_TO_MLXQ.items()}


class QuantizedOpError(RuntimeError):
    pass


def _arr(t: Optional[torch.Tensor]):
    if t is None:
        return None
    if t.dim() > _lib.MAX_DIMS:
        raise ValueError(f"[mlxq] at most {_lib.MAX_DIMS} dimensions are supported")
    a = _lib.MlxqArray()
    a.data = t.data_ptr() if t.numel() > 0 else None
    a.dtype = _TORCH_TO_MLXQ.get(t.dtype, -1)
    if a.dtype < 0:
        raise ValueError(f"[mlxq] unsupported tensor dtype {t.dtype}")
    a.ndim = t.dim()
    for i, (s, st) in enumerate(zip(t.shape, t.stride())):
        a.shape[i] = s
        a.strides[i] = st
    return ctypes.byref(a), a  # keep `a` alive with the reference


def _ref(pair):
    return None if pair is None else pair[0]


def _raise(status: int) -> None:
    msg = _lib.last_error()
    if status == _lib.EINVAL:
        raise ValueError(msg)
    if status == _lib.EUNSUPPORTED:
        raise NotImplementedError(msg)
    raise QuantizedOpError(f"status {status}: {msg}")


def _stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _opt(v: Optional[int]) -> int:
    return -1 if v is None else int(v)


def _mode(mode: str) -> bytes:
    return mode.encode() if isinstance(mode, str) else bytes(mode)


def _empty(ndim, shape, dtype, device) -> torch.Tensor:
    return torch.empty(tuple(shape[: ndim.value]), dtype=_MLXQ_TO_TORCH[dtype.value], device=device)


def _device_of(x: torch.Tensor) -> torch.device:
    if x.device.type != "cuda":
        raise ValueError("[mlxq] tensors must live on a HIP device (torch 'cuda' device)")
    return x.device


def quantized_matmul(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
                     biases: Optional[torch.Tensor] = None, transpose: bool = True,
                     group_size: Optional[int] = None, bits: Optional[int] = None,
                     mode: str = "affine", *, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``x @ dequantize(w, scales, biases).T`` (``transpose=True``), as ``mx.quantized_matmul``."""
    lib = _lib.load()
    ax, aw, as_, ab = _arr(x), _arr(w), _arr(scales), _arr(biases)
    gs, b = _opt(group_size), _opt(bits)
    if out is None:
        nd, sh, dt = ctypes.c_int32(), (ctypes.c_int64 * _lib.MAX_DIMS)(), ctypes.c_int32()
        st = lib.mlxq_quantized_matmul_shape(_ref(ax), _ref(aw), _ref(as_), _ref(ab), transpose, gs, b,
                                             _mode(mode), ctypes.byref(nd), sh, ctypes.byref(dt))
        if st:
            _raise(st)
        out = _empty(nd, sh, dt, _device_of(x))
    ao = _arr(out)
    dev = _device_of(x)
    with torch.cuda.device(dev):
        st = lib.mlxq_quantized_matmul(_ref(ax), _ref(aw), _ref(as_), _ref(ab), transpose, gs, b,
                                       _mode(mode), _ref(ao), _stream(dev))
    if st:
        _raise(st)
    return out


def quantized_linear(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: Optional[torch.Tensor] = None,
                     linear_bias: Optional[torch.Tensor] = None, group_size: Optional[int] = None,
                     bits: Optional[int] = None, mode: str = "affine", *,
                     out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The reference's ``quantized_linear_forward``: ``x @ W^T + linear_bias``."""
    lib = _lib.load()
    gs, b = _opt(group_size), _opt(bits)
    ax, aw, as_, ab, alb = _arr(x), _arr(w), _arr(scales), _arr(biases), _arr(linear_bias)
    if out is None:
        nd, sh, dt = ctypes.c_int32(), (ctypes.c_int64 * _lib.MAX_DIMS)(), ctypes.c_int32()
        st = lib.mlxq_quantized_matmul_shape(_ref(ax), _ref(aw), _ref(as_), _ref(ab), True, gs, b, _mode(mode),
                                             ctypes.byref(nd), sh, ctypes.byref(dt))
        if st:
            _raise(st)
        out = _empty(nd, sh, dt, _device_of(x))
    ao = _arr(out)
    dev = _device_of(x)
    with torch.cuda.device(dev):
        st = lib.mlxq_quantized_linear(_ref(ax), _ref(aw), _ref(as_), _ref(ab), _ref(alb), gs, b, _mode(mode),
                                       _ref(ao), _stream(dev))
    if st:
        _raise(st)
    return out


def quantized_matmul_matches_dense_gemm(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
                                        biases: Optional[torch.Tensor] = None, group_size: int = 64,
                                        bits: int = 4) -> bool:
    """The reference's predicate of the same name (no device work)."""
    lib = _lib.load()
    return bool(lib.mlxq_quantized_matmul_matches_dense_gemm(_ref(_arr(x)), _ref(_arr(w)), _ref(_arr(scales)),
                                                             _ref(_arr(biases)), group_size, bits))


def quantized_matmul_multi(x: torch.Tensor, ws: Sequence[torch.Tensor], scales: Sequence[torch.Tensor],
                           biases: Optional[Sequence[Optional[torch.Tensor]]] = None,
                           group_size: Optional[int] = None, bits: Optional[int] = None, mode: str = "affine", *,
                           out: Optional[Sequence[torch.Tensor]] = None) -> list:
    """``[quantized_matmul(x, w_i, s_i, b_i) for i]`` (transpose=True) in one
    call; at decode sizes one launch that reads x once (q/k/v, gate/up)."""
    lib = _lib.load()
    n = len(ws)
    gs, b = _opt(group_size), _opt(bits)
    dev = _device_of(x)
    if out is None:
        out = []
        for w_, s_, b_ in zip(ws, scales, biases if biases is not None else [None] * n):
            nd, sh, dt = ctypes.c_int32(), (ctypes.c_int64 * _lib.MAX_DIMS)(), ctypes.c_int32()
            st = lib.mlxq_quantized_matmul_shape(_ref(_arr(x)), _ref(_arr(w_)), _ref(_arr(s_)), _ref(_arr(b_)),
                                                 True, gs, b, _mode(mode), ctypes.byref(nd), sh, ctypes.byref(dt))
            if st:
                _raise(st)
            out.append(_empty(nd, sh, dt, dev))
    P = ctypes.POINTER(_lib.MlxqArray)

    def ptrs(ts):  # (pointer array, the structs it points to: kept alive by the caller)
        structs = [_arr(t)[1] if t is not None else None for t in ts]
        return (P * n)(*[ctypes.pointer(v) if v is not None else None for v in structs]), structs

    pw, kw = ptrs(ws)
    ps, ks = ptrs(scales)
    po, ko = ptrs(out)
    pb, kb = ptrs(biases) if biases is not None else (None, None)
    ax = _arr(x)
    with torch.cuda.device(dev):
        st = lib.mlxq_quantized_matmul_multi(_ref(ax), n, pw, ps, pb, gs, b, _mode(mode), po, _stream(dev))
    if st:
        _raise(st)
    return list(out)


def gather_qmm(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
               biases: Optional[torch.Tensor] = None, lhs_indices: Optional[torch.Tensor] = None,
               rhs_indices: Optional[torch.Tensor] = None, transpose: bool = True,
               group_size: Optional[int] = None, bits: Optional[int] = None, mode: str = "affine",
               sorted_indices: bool = False, *, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``out[i] = x[lhs[i]] @ dequantize(w[rhs[i]]).T``, as ``mx.gather_qmm``."""
    lib = _lib.load()
    ax, aw, as_, ab = _arr(x), _arr(w), _arr(scales), _arr(biases)
    al, ar = _arr(lhs_indices), _arr(rhs_indices)
    gs, b = _opt(group_size), _opt(bits)
    if out is None:
        nd, sh, dt = ctypes.c_int32(), (ctypes.c_int64 * _lib.MAX_DIMS)(), ctypes.c_int32()
        st = lib.mlxq_gather_qmm_shape(_ref(ax), _ref(aw), _ref(as_), _ref(ab), _ref(al), _ref(ar), transpose,
                                       gs, b, _mode(mode), ctypes.byref(nd), sh, ctypes.byref(dt))
        if st:
            _raise(st)
        out = _empty(nd, sh, dt, _device_of(x))
    ao = _arr(out)
    dev = _device_of(x)
    with torch.cuda.device(dev):
        st = lib.mlxq_gather_qmm(_ref(ax), _ref(aw), _ref(as_), _ref(ab), _ref(al), _ref(ar), transpose, gs, b,
                                 sorted_indices, _mode(mode), None, _ref(ao), _stream(dev))
    if st:
        _raise(st)
    return out


def _default_gs_bits(mode: str, group_size, bits):
    d = {"affine": (64, 4), "mxfp4": (32, 4), "nvfp4": (16, 4), "mxfp8": (32, 8)}.get(mode, (64, 4))
    return (d[0] if group_size is None else group_size), (d[1] if bits is None else bits)


def dequantize(w: torch.Tensor, scales: torch.Tensor, biases: Optional[torch.Tensor] = None,
               group_size: Optional[int] = None, bits: Optional[int] = None, mode: str = "affine",
               dtype: Optional[torch.dtype] = None, *, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``mx.dequantize``; affine output is bit-exact to MLX's CPU graph."""
    lib = _lib.load()
    gs, b = _default_gs_bits(mode, group_size, bits)
    dcode = -1 if dtype is None else _TORCH_TO_MLXQ[dtype]
    if out is None:
        if b <= 0:
            raise ValueError(f"[dequantize] Invalid value for bits: {b}")
        if w.dim() < 1:
            raise ValueError("[dequantize] The matrix to be dequantized must have at least 2 dimension "
                             f"but it has only {w.dim()}.")
        shape = list(w.shape)
        shape[-1] = shape[-1] * 32 // b
        odt = dtype if dtype is not None else (scales.dtype if mode == "affine" else torch.bfloat16)
        out = torch.empty(shape, dtype=odt, device=_device_of(w))
    aw, as_, ab, ao = _arr(w), _arr(scales), _arr(biases), _arr(out)
    dev = _device_of(w)
    with torch.cuda.device(dev):
        st = lib.mlxq_dequantize(_ref(aw), _ref(as_), _ref(ab), gs, b, _mode(mode), dcode, _ref(ao),
                                 _stream(dev))
    if st:
        _raise(st)
    return out


def quantize(w: torch.Tensor, group_size: Optional[int] = None, bits: Optional[int] = None,
             mode: str = "affine") -> Sequence[torch.Tensor]:
    """``mx.quantize``: returns ``(wq, scales, biases)`` (affine) or ``(wq, scales)``."""
    lib = _lib.load()
    gs, b = _default_gs_bits(mode, group_size, bits)
    dev = _device_of(w)
    if w.dim() < 2 or gs <= 0 or b <= 0 or w.shape[-1] % gs or (w.shape[-1] * b) % 32:
        # let the library produce the reference's message
        wq = scales = biases = w.new_empty((0,))
    else:
        qshape = list(w.shape)
        qshape[-1] = w.shape[-1] * b // 32
        sshape = list(w.shape)
        sshape[-1] = w.shape[-1] // gs
        wq = torch.empty(qshape, dtype=torch.uint32, device=dev)
        if mode == "affine":
            scales = torch.empty(sshape, dtype=w.dtype, device=dev)
            biases = torch.empty(sshape, dtype=w.dtype, device=dev)
        else:
            scales = torch.empty(sshape, dtype=torch.uint8, device=dev)
            biases = None
    aw, aq, as_, ab = _arr(w), _arr(wq), _arr(scales), _arr(biases)
    with torch.cuda.device(dev):
        st = lib.mlxq_quantize(_ref(aw), _opt(group_size), _opt(bits), _mode(mode), _ref(aq), _ref(as_),
                               _ref(ab), _stream(dev))
    if st:
        _raise(st)
    return (wq, scales, biases) if mode == "affine" else (wq, scales)


def _fused_moe(fn_name: str, x, indices, gate_w, gate_s, gate_b, up_w, up_s, up_b, down_w, down_s, down_b,
               scores, din: int, dff: int, k: int, gu_bits: int, d_bits: int, group_size: int,
               out: Optional[torch.Tensor]) -> torch.Tensor:
    lib = _lib.load()
    dev = _device_of(x)
    if out is None:
        out = torch.empty(max(int(din), 0), dtype=x.dtype, device=dev)
    arrs = [_arr(t) for t in (x, indices, gate_w, gate_s, gate_b, up_w, up_s, up_b, down_w, down_s, down_b,
                              scores, out)]
    with torch.cuda.device(dev):
        st = getattr(lib, fn_name)(*[_ref(a) for a in arrs[:12]], din, dff, k, gu_bits, d_bits, group_size,
                                   _ref(arrs[12]), _stream(dev))
    if st:
        _raise(st)
    return out


def fused_moe_expert(x, indices, gate_w, gate_s, gate_b, up_w, up_s, up_b, down_w, down_s, down_b, scores,
                     din: int, dff: int, k: int, gu_bits: int, d_bits: int, group_size: int, *,
                     out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The reference's ``fused_moe_expert_kernel`` (SwiGLU experts, one decode
    token): ``sum_j scores[j] * down_e(silu(gate_e(x)) * up_e(x))`` over
    ``e = indices[j]``; returns a ``(din,)`` tensor in x's dtype."""
    return _fused_moe("mlxq_fused_moe_expert", x, indices, gate_w, gate_s, gate_b, up_w, up_s, up_b, down_w,
                      down_s, down_b, scores, din, dff, k, gu_bits, d_bits, group_size, out)


def fused_moe_geglu(x, indices, gate_w, gate_s, gate_b, up_w, up_s, up_b, down_w, down_s, down_b, scores,
                    din: int, dff: int, k: int, gu_bits: int, d_bits: int, group_size: int, *,
                    out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The reference's ``fused_moe_geglu_kernel`` (GeGLU experts: tanh-approximated
    GELU of the gate times up)."""
    return _fused_moe("mlxq_fused_moe_geglu", x, indices, gate_w, gate_s, gate_b, up_w, up_s, up_b, down_w,
                      down_s, down_b, scores, din, dff, k, gu_bits, d_bits, group_size, out)


def workspace_reserve(nbytes: int, device: Optional[torch.device] = None) -> None:
    """Grow the current stream's workspace to ``nbytes`` before a HIP-graph
    capture (a call under capture never allocates; it fails instead)."""
    lib = _lib.load()
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else device
    with torch.cuda.device(dev):
        st = lib.mlxq_workspace_reserve(int(nbytes), _stream(dev))
    if st:
        _raise(st)


def get_cache_memory() -> int:
    """Device bytes held by the library's workspaces (``get_cache_memory``)."""
    return int(_lib.load().mlxq_get_cache_memory())


def clear_cache() -> None:
    """Free every workspace after synchronizing (``clear_memory_cache``)."""
    st = _lib.load().mlxq_clear_cache()
    if st:
        _raise(st)
