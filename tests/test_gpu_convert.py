"""GPU parity for the load-time conversions, bitwise:

* dequantize vs the MLX CPU graph (overlays/rocm/mlx/ops.cpp:5531-5573 affine,
  5646-5695 mxfp4) as restated by the oracle, plus the closed-form mxfp4 table;
* quantize vs the MLX CPU quantizer (overlays/cpu/mlx/backend/cpu/
  quantized.cpp:1233-1305) and the mxfp4 graph quantizer (ops.cpp:5364-5431),
  plus the hand-derived ramp fixtures;
* dequantize(slice) == slice(dequantize) (src/lib/mlxcel-core/src/ffi_tests.rs:5108-5170);
* affine bits 2, 4, 6 (MLX's 3-byte packs of 4 codes) and 8; quantize also
  for float16 / float32 weights and bits 1, 3 and 5 against the oracle's
  typed restatement (pinned in tests/test_oracle_quant_types.py);
* mxfp8 and nvfp4 (e4m3 as the ROCm backend's to_fp8 / from_fp8 evaluate it,
  overlays/rocm/mlx/backend/rocm/quantized/convert_fp8.hip:18-90): quantize
  on wide-range data and the hand fixtures, dequantize over every code and
  every scale.
"""
import os

import numpy as np
import pytest
import torch

import mlxcel_amd as mq
import oracle as orc
from helpers import announce, dev_bf16, dev_u32, dev_u8, host_u16

pytestmark = pytest.mark.gpu
KAT = np.load(os.path.join(os.path.dirname(__file__), "golden", "kat.npz"))


@pytest.mark.parametrize("bits", [2, 4, 6, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_affine_dequantize_bitexact(bits, gs):
    announce("dequant", bits, gs)
    w = orc.normal_bf16((96, 1024), 0.02, 500 + bits + gs)
    wq, s, b = orc.affine_quantize(w, gs, bits)
    got = host_u16(mq.dequantize(dev_u32(wq), dev_bf16(s), dev_bf16(b), gs, bits))
    np.testing.assert_array_equal(got, orc.affine_dequantize(wq, s, b, gs, bits, 2))


def test_affine_dequantize_halfway_fixture():
    announce("dequant_halfway")
    q = (KAT["d2_q"].reshape(-1, 1) * np.array([1, 0, 0, 0, 0, 0, 0, 0], np.uint32)).astype(np.uint32)
    got = host_u16(mq.dequantize(dev_u32(q), dev_bf16(KAT["d2_s"].reshape(-1, 1)),
                                 dev_bf16(KAT["d2_b"].reshape(-1, 1)), 32, 8))
    np.testing.assert_array_equal(got[:, 0], KAT["d2_out"])


def test_mxfp4_dequantize_table_and_random():
    announce("dequant_mxfp4")
    codes = np.zeros((256, 32), np.uint32)
    codes[:, :16] = np.arange(16)
    wq = np.zeros((256, 4), np.uint32)
    for j in range(32):
        wq[:, j // 8] |= codes[:, j] << (4 * (j % 8))
    sc = np.arange(256, dtype=np.uint8).reshape(256, 1)
    got = host_u16(mq.dequantize(dev_u32(wq), dev_u8(sc), None, 32, 4, "mxfp4"))
    np.testing.assert_array_equal(got[:, :16].T, KAT["mxfp4_table"])
    w = orc.normal_bf16((64, 2880), 0.02, 510)
    wq2, sc2 = orc.mxfp4_quantize(w)
    got2 = host_u16(mq.dequantize(dev_u32(wq2), dev_u8(sc2), None, 32, 4, "mxfp4"))
    np.testing.assert_array_equal(got2, orc.mxfp4_dequantize(wq2, sc2))


def test_dequantize_commutes_with_row_slice():
    announce("dequant_slice")
    w = orc.normal_bf16((64, 512), 0.02, 520)
    wq, s, b = orc.affine_quantize(w, 64, 4)
    W, S, B = dev_u32(wq), dev_bf16(s), dev_bf16(b)
    full = host_u16(mq.dequantize(W, S, B))
    part = host_u16(mq.dequantize(W[16:40].contiguous(), S[16:40].contiguous(), B[16:40].contiguous()))
    np.testing.assert_array_equal(full[16:40], part)


@pytest.mark.parametrize("bits", [2, 4, 6, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_affine_quantize_bitexact(bits, gs):
    announce("quant", bits, gs)
    w = orc.normal_bf16((128, 1024), 0.02, 530 + bits + gs)
    wq, s, b = mq.quantize(dev_bf16(w), gs, bits)
    ewq, es, eb = orc.affine_quantize(w, gs, bits)
    np.testing.assert_array_equal(wq.cpu().numpy(), ewq)
    np.testing.assert_array_equal(host_u16(s), es)
    np.testing.assert_array_equal(host_u16(b), eb)
    kw, ks, kb = mq.quantize(dev_bf16(KAT[f"ramp_w_b{bits}_g{gs}"]), gs, bits)
    np.testing.assert_array_equal(kw.cpu().numpy(), KAT[f"ramp_wq_b{bits}_g{gs}"])
    np.testing.assert_array_equal(host_u16(ks), KAT[f"ramp_s_b{bits}_g{gs}"])
    np.testing.assert_array_equal(host_u16(kb), KAT[f"ramp_b_b{bits}_g{gs}"])


TORCH_DT = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}


def typed_weights(dtype, rows, K, seed):
    """(numpy array in the oracle's form, the same values as a device tensor)"""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, K)).astype(np.float32)
    x *= (10.0 ** rng.uniform(-4, 2, (rows, 1))).astype(np.float32)
    x[1] = np.abs(x[1])
    x[2] = -np.abs(x[2])
    x[3] = 0.375
    x[4] = 0.0
    t = torch.from_numpy(x).to(TORCH_DT[dtype])
    if dtype == "bfloat16":
        return t.view(torch.int16).numpy().astype(np.uint16), t.cuda()
    return t.numpy(), t.cuda()


def host_bytes(t):
    return t.cpu().contiguous().view(torch.uint8).numpy()


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_affine_quantize_types_and_widths_bitexact(dtype, bits, gs):
    # every weight type (scales and biases in that type) and width against
    # the oracle's typed restatement of the MLX CPU quantizer, byte for byte
    announce("quant_typed", dtype, bits, gs)
    w, wd = typed_weights(dtype, 64, 512, 900 + 10 * bits + gs)
    wq, s, b = mq.quantize(wd, gs, bits)
    assert s.dtype == TORCH_DT[dtype] and b.dtype == TORCH_DT[dtype]
    ewq, es, eb = orc.affine_quantize_t(w, dtype, gs, bits)
    np.testing.assert_array_equal(wq.cpu().numpy(), ewq)
    np.testing.assert_array_equal(host_bytes(s).reshape(-1), np.asarray(es).reshape(-1).view(np.uint8))
    np.testing.assert_array_equal(host_bytes(b).reshape(-1), np.asarray(eb).reshape(-1).view(np.uint8))


@pytest.mark.parametrize("dtype", ["float16", "float32"])
@pytest.mark.parametrize("bits", [1, 3, 5])
def test_affine_quantize_dequantize_round_trip(dtype, bits):
    # dequantize(quantize(w)) on the GPU equals the MLX graph dequantize of
    # the GPU's codes, bitwise, and each value lies within 1.5 steps of w (the
    # edge snapping can clamp the far extreme by up to a step)
    from oracle import generic as og
    announce("quant_round_trip", dtype, bits)
    gs = 64
    w, wd = typed_weights(dtype, 16, 256, 950 + bits)
    wq, s, b = mq.quantize(wd, gs, bits)
    d = mq.dequantize(wq, s, b, gs, bits).float().cpu().numpy().astype(np.float64)
    s64 = s.float().cpu().numpy().astype(np.float64)
    b64 = b.float().cpu().numpy().astype(np.float64)
    want = og.dequantize_graph(wq.cpu().numpy(), s64, b64, gs, bits, 256, dtype, dtype)
    np.testing.assert_array_equal(d, want)
    wf = wd.float().cpu().numpy().astype(np.float64)
    step = np.repeat(np.abs(s64), gs, axis=1)
    tol = 1.5 * step + 1e-3 * np.abs(wf) + 1e-30
    assert (np.abs(d - wf) <= tol).all()


HAND = sorted({k[len("hand_w_"):] for k in KAT.files if k.startswith("hand_w_")})


@pytest.mark.parametrize("case", HAND)
def test_affine_quantize_hand_cases(case):
    # hand-worked groups: bf16-unrepresentable scales, rint ties, the
    # |w_min| == |w_max| branch, a clamped far extreme
    announce("quant_hand", case)
    bits = int(case.rsplit("_b", 1)[1])
    wq, s, b = mq.quantize(dev_bf16(KAT[f"hand_w_{case}"]), 32, bits)
    np.testing.assert_array_equal(wq.cpu().numpy(), KAT[f"hand_wq_{case}"])
    np.testing.assert_array_equal(host_u16(s), KAT[f"hand_s_{case}"])
    np.testing.assert_array_equal(host_u16(b), KAT[f"hand_b_{case}"])


def test_mxfp4_quantize_hand_cases():
    announce("quant_mxfp4_hand")
    wq, sc = mq.quantize(dev_bf16(KAT["mxfp4_hand_w"]), mode="mxfp4")
    np.testing.assert_array_equal(wq.cpu().numpy(), KAT["mxfp4_hand_wq"])
    np.testing.assert_array_equal(sc.cpu().numpy(), KAT["mxfp4_hand_scales"])


def test_mxfp4_quantize_bitexact():
    announce("quant_mxfp4")
    w = orc.normal_bf16((256, 2880), 0.02, 540)
    wq, sc = mq.quantize(dev_bf16(w), mode="mxfp4")
    ewq, esc = orc.mxfp4_quantize(w)
    np.testing.assert_array_equal(sc.cpu().numpy(), esc)
    np.testing.assert_array_equal(wq.cpu().numpy(), ewq)


def test_quantize_dequantize_roundtrip_full_size():
    # Llama-3-8B gate shape: size-independent property at full size
    announce("roundtrip_full")
    w = torch.randn(14336, 4096, device="cuda", dtype=torch.float32).mul_(0.02).to(torch.bfloat16)
    wq, s, b = mq.quantize(w, 64, 4)
    d = mq.dequantize(wq, s, b, 64, 4).float()
    err = (d - w.float()).abs().reshape(14336, 64, 64)
    assert float((err / s.float().abs().unsqueeze(-1)).max()) <= 1.6


# ---- mxfp8 / nvfp4 (e4m3 via the ROCm backend's to_fp8, convert_fp8.hip:18-90) ----

def wide_bf16(rows, K, seed):
    # N(0, 0.02) rows plus rows spanning 1e-6 .. 1e3 per group, zeros and a
    # few groups with one large outlier (saturation, subnormal codes)
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, K)).astype(np.float32) * np.float32(0.02)
    x[rows // 2:] *= (10.0 ** rng.uniform(-4, 5, (rows - rows // 2, K // 16, 1))).repeat(16, -1).reshape(-1, K) \
        .astype(np.float32)
    x[0, :64] = 0.0
    x[1, 5] = 300.0
    return orc.f32_to_bf16(x)


@pytest.mark.parametrize("mode", ["mxfp8", "nvfp4"])
def test_fp_quantize_bitexact(mode):
    announce("quant", mode)
    w = wide_bf16(96, 2048, 560 + len(mode))
    wq, sc = mq.quantize(dev_bf16(w), mode=mode)
    ewq, esc = (orc.mxfp8_quantize if mode == "mxfp8" else orc.nvfp4_quantize)(w)
    np.testing.assert_array_equal(sc.cpu().numpy(), esc)
    np.testing.assert_array_equal(wq.cpu().numpy(), ewq)


def test_fp_quantize_hand_cases():
    announce("quant_fp_hand")
    for mode in ("mxfp8", "nvfp4"):
        wq, sc = mq.quantize(dev_bf16(KAT[f"{mode}_hand_w"]), mode=mode)
        np.testing.assert_array_equal(wq.cpu().numpy(), KAT[f"{mode}_hand_wq"])
        np.testing.assert_array_equal(sc.cpu().numpy(), KAT[f"{mode}_hand_scales"])


def test_mxfp8_dequantize_every_code_and_scale():
    # all 256 codes under all 256 scales (bf16 subnormal products included)
    announce("dequant_mxfp8_table")
    codes = np.tile(np.arange(256, dtype=np.uint8), (256, 1))
    wq = np.ascontiguousarray(codes).view(np.uint32).reshape(256, 64)
    sc = np.repeat(np.arange(256, dtype=np.uint8)[:, None], 8, 1)
    got = host_u16(mq.dequantize(dev_u32(wq), dev_u8(sc), None, 32, 8, "mxfp8"))
    np.testing.assert_array_equal(got, orc.mxfp8_dequantize(wq, sc))


def test_nvfp4_dequantize_every_code_and_scale():
    announce("dequant_nvfp4_table")
    wq = np.zeros((256, 2), np.uint32)
    for j in range(16):
        wq[:, j // 8] |= np.uint32(j) << np.uint32(4 * (j % 8))
    sc = np.arange(256, dtype=np.uint8).reshape(256, 1)
    got = host_u16(mq.dequantize(dev_u32(wq), dev_u8(sc), None, 16, 4, "nvfp4"))
    np.testing.assert_array_equal(got, orc.nvfp4_dequantize(wq, sc))


@pytest.mark.parametrize("mode", ["mxfp8", "nvfp4"])
def test_fp_dequantize_random_and_roundtrip(mode):
    announce("dequant_fp", mode)
    w = wide_bf16(64, 2880, 570 + len(mode))
    wq, sc = (orc.mxfp8_quantize if mode == "mxfp8" else orc.nvfp4_quantize)(w)
    got = host_u16(mq.dequantize(dev_u32(wq), dev_u8(sc), None, None, None, mode))
    np.testing.assert_array_equal(got, (orc.mxfp8_dequantize if mode == "mxfp8" else orc.nvfp4_dequantize)(wq, sc))
    # quantize -> dequantize on the GPU at a full expert shape, within the
    # format's error: mxfp8 half a 3-bit mantissa step (2^-4 relative, 2^-3
    # bound) plus the truncated subnormal codes (a few 2^-9 * 2^e, below
    # 2^-12 * max|w| of the group); nvfp4, with d the decoded e4m3 scale of
    # the group, half the largest code step (d) or, where |w| / d passed 6
    # (the scale rounded down, or truncated in e4m3's subnormal range),
    # |w| - 6 d
    wd = torch.randn(2880, 5760, device="cuda").mul_(0.02).to(torch.bfloat16)
    q, s = mq.quantize(wd, mode=mode)
    d = mq.dequantize(q, s, None, None, None, mode).float()
    err = (d - wd.float()).abs()
    gs = 32 if mode == "mxfp8" else 16
    amax = wd.float().abs().reshape(2880, -1, gs).amax(-1, keepdim=True).expand(-1, -1, gs).reshape(2880, -1)
    if mode == "mxfp8":
        bound = wd.float().abs() * 2.0 ** -3 + 2.0 ** -12 * amax
    else:
        table = torch.from_numpy(orc.e4m3_decode(np.arange(256, dtype=np.uint8))).cuda()
        dsc = table[s.long()].repeat_interleave(gs, -1)
        bound = torch.maximum(dsc, wd.float().abs() - 6 * dsc) * (1 + 2.0 ** -7)
    assert bool((err <= bound).all())
