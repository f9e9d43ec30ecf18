"""The MLX-quantized safetensors loader (mlxcel_amd/loader.py).

CPU: the reference's own cases for reconciling declared group_size / bits
with the tensor shapes (src/lib/mlxcel-core/src/layers.rs:6994-7160) as
vectors, mode inference (:2322-2332) and bias validation (:2175-2197), and a
synthetic checkpoint directory (config.json + safetensors: affine 4-bit,
a per-path 8-bit override, a shape-reconciled 8-bit plane, an mxfp4 expert
stack stored at group size 32 under a default of 64, a plain tensor) loaded
back with the planes' bytes unchanged.  GPU: the loaded planes drive
quantized_matmul and gather_qmm against the oracle.
"""
import json

import numpy as np
import pytest
import torch

import oracle as orc
from mlxcel_amd import loader

# (weight shape, scales shape, group_size, bits, mode) -> (bits, group_size, reconciled) | error text
RECONCILE_CASES = [
    (([32, 16], [32, 2], 64, 4, "affine"), (4, 64, False)),
    (([32, 32], [32, 2], 64, 4, "affine"), (8, 64, True)),
    (([32, 16], [32, 4], 64, 4, "affine"), (2, 64, True)),
    (([32, 16], [32, 4], 16, 4, "affine"), (4, 32, True)),
    (([32, 16], [32, 2], 16, 4, "affine"), (4, 64, True)),
    (([32, 14], [32, 1], 64, 4, "affine"), "not in"),
    (([32, 17], [32, 2], 64, 4, "affine"), "cannot derive"),
    (([64, 32], [64, 8], 32, 4, "mxfp4"), (4, 32, False)),
    (([64, 32], [64, 8], 64, 4, "mxfp4"), (4, 32, True)),
    (([64, 32], [64, 7], 64, 4, "mxfp4"), (4, 64, True)),
    (([], [], 64, 4, "affine"), (4, 64, False)),
    (([32, 16], [32, 2], 64, 0, "affine"), "bits"),
    (([32, 16], [32, 2], 64, -4, "affine"), "bits"),
    (([32, 16], [32, 2], 64, 33, "affine"), "bits"),
    (([32, 16], [32, 2], 0, 4, "affine"), "group_size"),
    (([32, 16], [32, 2], -64, 4, "affine"), "group_size"),
    (([], [], 64, 0, "mxfp4"), "bits"),
    (([32, 16], [], 0, 4, "mxfp4"), "group_size"),
    (([32, 16], [32, 2], 64, 4, "int4"), "mode"),
]


@pytest.mark.parametrize("args,want", RECONCILE_CASES)
def test_reconcile_quantization_layout_reference_cases(args, want):
    if isinstance(want, str):
        with pytest.raises(ValueError, match=want):
            loader.reconcile_quantization_layout(*args)
    else:
        assert loader.reconcile_quantization_layout(*args) == want


def test_mode_inference_and_bias_rules():
    assert loader.infer_quantization_mode(True, 16, 8) == "affine"
    assert loader.infer_quantization_mode(False, 32, 8) == "mxfp8"
    assert loader.infer_quantization_mode(False, 16, 4) == "nvfp4"
    assert loader.infer_quantization_mode(False, 32, 4) == "mxfp4"
    loader.validate_quantization_biases("affine", True)
    loader.validate_quantization_biases("mxfp4", False)
    with pytest.raises(ValueError, match="no .biases"):
        loader.validate_quantization_biases("affine", False)
    with pytest.raises(ValueError, match="ships a .biases"):
        loader.validate_quantization_biases("mxfp4", True)


def t16(a):
    return torch.from_numpy(np.ascontiguousarray(a).astype(np.int16)).view(torch.bfloat16)


def t32(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32))


def make_checkpoint(tmp_path):
    K = 256
    planes, raw = {}, {}
    q = orc.affine_quantize(orc.normal_bf16((64, K), 0.02, 1), 64, 4)
    planes["model.layers.0.self_attn.q_proj"] = (t32(q[0]), t16(q[1]), t16(q[2]))
    g = orc.affine_quantize(orc.normal_bf16((32, K), 0.02, 2), 64, 8)
    planes["model.layers.0.mlp.gate"] = (t32(g[0]), t16(g[1]), t16(g[2]))
    u = orc.affine_quantize(orc.normal_bf16((48, K), 0.02, 3), 64, 8)  # declared 4-bit by default
    planes["model.layers.0.mlp.up_proj"] = (t32(u[0]), t16(u[1]), t16(u[2]))
    e = orc.mxfp4_quantize(orc.normal_bf16((4, 64, K), 0.02, 4))
    planes["model.layers.0.mlp.experts.down_proj"] = (t32(e[0]), torch.from_numpy(e[1]))
    raw.update(q=q, g=g, u=u, e=e)
    norm = torch.ones(K, dtype=torch.bfloat16)
    loader.save_quantized(str(tmp_path / "model.safetensors"), planes, {"model.norm.weight": norm})
    cfg = {"quantization": {"group_size": 64, "bits": 4, "model.layers.0.mlp.gate": {"group_size": 64, "bits": 8}}}
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    return planes, raw


def test_checkpoint_round_trip(tmp_path):
    planes, _ = make_checkpoint(tmp_path)
    got, rest = loader.load_quantized(str(tmp_path), device="cpu")
    assert set(got) == set(planes) and set(rest) == {"model.norm.weight"}
    want = {
        "model.layers.0.self_attn.q_proj": ("affine", 4, 64, False),
        "model.layers.0.mlp.gate": ("affine", 8, 64, False),
        "model.layers.0.mlp.up_proj": ("affine", 8, 64, True),
        "model.layers.0.mlp.experts.down_proj": ("mxfp4", 4, 32, True),
    }
    for prefix, (mode, bits, gs, rec) in want.items():
        p = got[prefix]
        assert (p.mode, p.bits, p.group_size, p.reconciled) == (mode, bits, gs, rec), prefix
        assert torch.equal(p.weight, planes[prefix][0]) and torch.equal(p.scales, planes[prefix][1])
        assert (p.biases is None) == (len(planes[prefix]) == 2)
    assert got["model.layers.0.mlp.experts.down_proj"].is_experts


def test_checkpoint_errors(tmp_path):
    K = 128
    q = orc.affine_quantize(orc.normal_bf16((16, K), 0.02, 5), 64, 4)
    path = str(tmp_path / "a.safetensors")
    loader.save_quantized(path, {"l": (t32(q[0]), t16(q[1]))})  # affine codes, biases missing
    with pytest.raises(ValueError, match="biases"):
        loader.load_quantized([path], {"quantization": {"group_size": 64, "bits": 4, "mode": "affine"}}, "cpu")
    loader.save_quantized(path, {"l": (t32(q[0]), t16(q[1]), t16(q[2]))})
    with pytest.raises(ValueError, match="group_size"):
        loader.load_quantized([path], {"quantization": {"group_size": 0, "bits": 4}}, "cpu")
    with pytest.raises(ValueError, match="unquantized"):
        loader.load_quantized([path], {"quantization": {"group_size": 64, "bits": 4, "l": False}}, "cpu")


@pytest.mark.gpu
def test_loaded_planes_drive_the_kernels(tmp_path):
    from helpers import TOL, announce, dev_bf16, host_u16, max_rel

    announce("loader_gpu")
    _, raw = make_checkpoint(tmp_path)
    got, _ = loader.load_quantized(str(tmp_path), device="cuda")
    x = orc.normal_bf16((2, 256), 1.0, 6)
    for prefix, key, bits in (("model.layers.0.self_attn.q_proj", "q", 4), ("model.layers.0.mlp.up_proj", "u", 8)):
        y = host_u16(got[prefix](dev_bf16(x)))
        assert max_rel(y, orc.qmm_t_affine(x, *raw[key], 64, bits)) <= TOL
    ex = got["model.layers.0.mlp.experts.down_proj"]
    idx = torch.tensor([[3, 0], [1, 1]], dtype=torch.int32, device="cuda")
    y = host_u16(ex.gather(dev_bf16(x).view(2, 1, 1, 256), idx))
    want = orc.gather_qmm_t(x.reshape(2, 1, 256), *raw["e"], None, np.array([0, 0, 1, 1], np.uint32),
                            np.array([3, 0, 1, 1], np.uint32), mode="mxfp4")
    assert max_rel(y.reshape(4, 64), want.reshape(4, 64)) <= TOL
