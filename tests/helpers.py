"""Shared helpers for the GPU parity tests: build seeded inputs with the oracle
(the checker) on the host, move the same bytes to the device, compare."""
import sys

import numpy as np
import torch

import oracle as orc

TOL = 1e-2  # north-star gate: max|y - y_ref| / max|y_ref|, bf16 output, fp32 accumulate


def setknob(monkeypatch, name, value):
    """Set an MLXQ_* switch for this test; the library latches the switches,
    so re-read them (the conftest re-reads them again before the next test)."""
    monkeypatch.setenv(name, value)
    import mlxcel_amd._lib as L
    L.load().mlxq_reload_options()


def announce(*parts):
    """Name the GPU case before it runs (a fault then still says which case)."""
    print("[gpu case]", *parts, flush=True)
    sys.stdout.flush()


def dev_bf16(a_u16: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a_u16).astype(np.int16)).view(torch.bfloat16).cuda()


def dev_u32(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32)).cuda()


def dev_u8(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint8)).cuda()


def host_u16(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().astype(np.uint16)


def host_f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def max_rel(got_u16: np.ndarray, want_u16: np.ndarray) -> float:
    g = orc.bf16_to_f32(got_u16).astype(np.float64)
    w = orc.bf16_to_f32(want_u16).astype(np.float64)
    return float(np.abs(g - w).max() / max(np.abs(w).max(), 1e-30))


def affine_case(M, N, K, gs, bits, seed, batch=()):
    x = orc.normal_bf16(tuple(batch) + (M, K), 1.0, seed)
    w = orc.normal_bf16((N, K), 0.02, seed + 1)
    wq, s, b = orc.affine_quantize(w, gs, bits)
    return x, wq, s, b


def mxfp4_case(M, N, K, seed, E=None):
    x = orc.normal_bf16((M, K), 1.0, seed)
    shape = (N, K) if E is None else (E, N, K)
    w = orc.normal_bf16(shape, 0.02, seed + 1)
    wq, s = orc.mxfp4_quantize(w)
    return x, wq, s
