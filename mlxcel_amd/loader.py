"""MLX-quantized safetensors checkpoints -> device tensors for this library.

An MLX-quantized model directory holds ``config.json`` (with a
``quantization`` block: ``group_size``, ``bits``, optionally ``mode`` and
per-path overrides) and ``*.safetensors`` files in which every quantized
linear layer ``<prefix>`` is three planes:

* ``<prefix>.weight``  uint32 packed codes ``[..., N, K * bits / 32]``;
* ``<prefix>.scales``  bf16/f16/f32 (affine) or uint8 (block-float: mxfp4
  e8m0, nvfp4, mxfp8) ``[..., N, K / group_size]``;
* ``<prefix>.biases``  affine only, same shape as the scales.

A 2-D weight is a linear layer (``quantized_matmul``); a 3-D weight is a
stack of experts (``gather_qmm``).  The rules for telling the mode and
reconciling the declared ``group_size`` / ``bits`` with the tensor shapes
restate the reference's loader: ``infer_quantization_mode``
(src/lib/mlxcel-core/src/layers.rs:2322-2332), ``infer_plane_quantization_mode``
(:2347-2373), ``reconcile_quantization_layout`` (:2405-2520, with
``infer_quantization_bits`` :1643-1694 and ``infer_quantization_group_size``
:1696-1730), ``validate_quantization_params`` (:1786-1806),
``validate_quantization_mode`` (:2016-2027) and
``validate_quantization_biases`` (:2175-2197); the planes are read as in
``UnifiedLinear::from_weights_with_mode`` (:2745-2800) and the gpt-oss expert
loader (src/models/gpt_oss_common.rs:212-290).  Errors are ``ValueError``
with the reason, raised at load time instead of at the first forward pass.
"""
from __future__ import annotations

import glob
import json
import os
from dataclasses import dataclass
from typing import Dict, Iterable, Optional, Tuple

import torch

from . import ops

SUPPORTED_MODES = ("affine", "mxfp4", "mxfp8", "nvfp4")  # layers.rs:1885
LOADABLE_AFFINE_BITS = (1, 2, 3, 4, 5, 6, 8)  # layers.rs:1933
MAX_GROUP_SIZE = 1 << 20  # layers.rs:2301


def infer_quantization_mode(has_biases: bool, group_size: int, bits: int) -> str:
    """Affine planes carry zero points; the block-float modes are told apart
    by their fixed bits and block (layers.rs:2322-2332)."""
    if has_biases:
        return "affine"
    if bits == 8:
        return "mxfp8"
    if group_size == 16:
        return "nvfp4"
    return "mxfp4"


def validate_quantization_params(group_size: int, bits: int) -> None:
    if not 1 <= bits <= 32:
        raise ValueError(f"quantization.bits ({bits}) must be between 1 and 32")
    if not 1 <= group_size <= MAX_GROUP_SIZE:
        raise ValueError(f"quantization.group_size ({group_size}) must be between 1 and {MAX_GROUP_SIZE}")


def validate_quantization_mode(mode: str) -> None:
    if mode not in SUPPORTED_MODES:
        raise ValueError(f"quantization.mode ({mode!r}) must be one of {', '.join(SUPPORTED_MODES)}")


def validate_quantization_biases(mode: str, has_biases: bool) -> None:
    validate_quantization_mode(mode)
    if mode == "affine" and not has_biases:
        raise ValueError('quantization.mode is "affine" but the checkpoint ships no .biases plane')
    if mode != "affine" and has_biases:
        raise ValueError(f"quantization.mode is {mode!r} but the checkpoint ships a .biases plane")


def _infer_bits(packed_in: int, num_groups: int, group_size: int, caller_bits: int) -> int:
    num, den = packed_in * 32, num_groups * group_size
    if den == 0 or num % den:
        raise ValueError(f"quantized weight shape inconsistency: packed_in={packed_in}, groups={num_groups}, "
                         f"group_size={group_size}: cannot derive integer bits")
    bits = num // den
    if bits != caller_bits and bits not in LOADABLE_AFFINE_BITS:
        raise ValueError(f"quantized weight shape inconsistency: inferred bits={bits} not in "
                         f"{set(LOADABLE_AFFINE_BITS)}")
    return bits


def _infer_group_size(packed_in: int, num_groups: int, bits: int) -> int:
    num, den = packed_in * 32, num_groups * bits
    if den == 0 or num % den:
        raise ValueError(f"quantized weight shape inconsistency: packed_in={packed_in}, groups={num_groups}, "
                         f"bits={bits}: cannot derive integer group_size")
    return num // den


def reconcile_quantization_layout(weight_shape, scales_shape, group_size: int, bits: int,
                                  mode: str) -> Tuple[int, int, bool]:
    """(bits, group_size, reconciled) satisfying
    ``packed_in * 32 == bits * num_groups * group_size``: affine trusts the
    group size and re-derives bits (per-path bit overrides); block-float
    trusts the mode's bits and re-derives the group size (layers.rs:2405-2520)."""
    validate_quantization_params(group_size, bits)
    validate_quantization_mode(mode)
    if not len(weight_shape) or not len(scales_shape):
        return bits, group_size, False
    packed_in, num_groups = int(weight_shape[-1]), int(scales_shape[-1])
    if packed_in <= 0 or num_groups <= 0:
        return bits, group_size, False
    if mode == "affine":
        if group_size == 16 and bits == 4:
            # repacked 16-wide sources: keep 4 bits, recover the real group size
            gs = _infer_group_size(packed_in, num_groups, bits)
            if gs in (32, 64, 128):
                return bits, gs, gs != group_size
        b = _infer_bits(packed_in, num_groups, group_size, bits)
        return b, group_size, b != bits
    if len(weight_shape) < 2 or len(scales_shape) < 2 or 32 % bits:
        return bits, group_size, False
    in_features = packed_in * (32 // bits)
    if in_features % num_groups == 0:
        gs = in_features // num_groups
        return bits, gs, gs != group_size
    return bits, group_size, True


@dataclass
class QuantizedWeight:
    """One quantized plane set on the device: a linear layer (2-D weight) or an
    expert stack (3-D)."""
    weight: torch.Tensor
    scales: torch.Tensor
    biases: Optional[torch.Tensor]
    group_size: int
    bits: int
    mode: str
    reconciled: bool = False

    @property
    def is_experts(self) -> bool:
        return self.weight.dim() == 3

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        """``x @ W^T`` (``quantized_matmul``)."""
        return ops.quantized_matmul(x, self.weight, self.scales, self.biases, True, self.group_size, self.bits,
                                    self.mode)

    def gather(self, x: torch.Tensor, indices: torch.Tensor, sorted_indices: bool = False) -> torch.Tensor:
        """``x @ W[indices]^T`` for an expert stack (``gather_qmm``, rhs indices)."""
        return ops.gather_qmm(x, self.weight, self.scales, self.biases, None, indices, True, self.group_size,
                              self.bits, self.mode, sorted_indices)


def _layer_params(quant: dict, prefix: str) -> Optional[Tuple[int, int, Optional[str]]]:
    """(group_size, bits, mode) for `prefix` from an mlx-lm ``quantization``
    block: per-path entries override the defaults; ``false`` marks a layer
    left unquantized."""
    gs, bits, mode = int(quant.get("group_size", 64)), int(quant.get("bits", 4)), quant.get("mode")
    ov = quant.get(prefix)
    if ov is False:
        return None
    if isinstance(ov, dict):
        gs, bits = int(ov.get("group_size", gs)), int(ov.get("bits", bits))
        mode = ov.get("mode", mode)
    return gs, bits, mode


def load_config(model_dir: str) -> dict:
    path = os.path.join(model_dir, "config.json")
    if not os.path.exists(path):
        return {}
    with open(path) as f:
        return json.load(f)


def load_quantized(paths, config: Optional[dict] = None, device="cuda",
                   ) -> Tuple[Dict[str, QuantizedWeight], Dict[str, torch.Tensor]]:
    """Read MLX-quantized safetensors into ``(quantized planes by prefix,
    other tensors by name)`` on `device`.

    `paths` is a model directory (its ``*.safetensors`` and ``config.json``)
    or an iterable of safetensors files (then `config` gives the
    ``quantization`` block, or its defaults apply: group_size 64, bits 4)."""
    from safetensors import safe_open

    if isinstance(paths, str) and os.path.isdir(paths):
        if config is None:
            config = load_config(paths)
        files = sorted(glob.glob(os.path.join(paths, "*.safetensors")))
    elif isinstance(paths, str):
        files = [paths]
    else:
        files = list(paths)
    quant = dict((config or {}).get("quantization") or (config or {}).get("quantization_config") or {})
    tensors: Dict[str, torch.Tensor] = {}
    for fn in files:
        with safe_open(fn, framework="pt", device="cpu") as f:
            for k in f.keys():
                tensors[k] = f.get_tensor(k)
    planes: Dict[str, QuantizedWeight] = {}
    for name in [k for k in tensors if k.endswith(".scales")]:
        prefix = name[: -len(".scales")]
        wname, bname = prefix + ".weight", prefix + ".biases"
        if wname not in tensors:
            raise ValueError(f"{prefix}: .scales without .weight")
        params = _layer_params(quant, prefix)
        if params is None:
            raise ValueError(f"{prefix}: quantized planes for a layer the config leaves unquantized")
        gs, bits, mode = params
        w, s = tensors.pop(wname), tensors.pop(name)
        b = tensors.pop(bname, None)
        if w.dtype != torch.uint32:
            # safetensors stores MLX's uint32 planes as U32
            raise ValueError(f"{prefix}: .weight must be uint32 (got {w.dtype})")
        if mode is None:
            # the declared pair describes the block only after reconciliation
            declared = infer_quantization_mode(b is not None, gs, bits)
            mode = declared
            if b is None:
                try:
                    rb, rgs, _ = reconcile_quantization_layout(w.shape, s.shape, gs, bits, declared)
                    mode = infer_quantization_mode(False, rgs, rb)
                except ValueError:
                    mode = declared
        validate_quantization_biases(mode, b is not None)
        if mode != "affine":
            bits = {"mxfp4": 4, "nvfp4": 4, "mxfp8": 8}[mode]
        rbits, rgs, rec = reconcile_quantization_layout(w.shape, s.shape, gs, bits, mode)
        planes[prefix] = QuantizedWeight(
            weight=w.to(device).contiguous(), scales=s.to(device).contiguous(),
            biases=None if b is None else b.to(device).contiguous(),
            group_size=rgs, bits=rbits, mode=mode, reconciled=rec)
    rest = {k: v.to(device) for k, v in tensors.items()}
    return planes, rest


def save_quantized(path: str, planes: Dict[str, Tuple[torch.Tensor, ...]], other: Optional[Dict] = None) -> None:
    """Write planes ``{prefix: (weight, scales[, biases])}`` (and plain tensors)
    as one MLX-layout safetensors file."""
    from safetensors.torch import save_file

    out = {}
    for prefix, t in planes.items():
        out[prefix + ".weight"] = t[0].detach().cpu().contiguous()
        out[prefix + ".scales"] = t[1].detach().cpu().contiguous()
        if len(t) > 2 and t[2] is not None:
            out[prefix + ".biases"] = t[2].detach().cpu().contiguous()
    for k, v in (other or {}).items():
        out[k] = v.detach().cpu().contiguous()
    save_file(out, path)


__all__ = ["QuantizedWeight", "load_quantized", "save_quantized", "load_config", "infer_quantization_mode",
           "reconcile_quantization_layout", "validate_quantization_params", "validate_quantization_mode",
           "validate_quantization_biases"]
