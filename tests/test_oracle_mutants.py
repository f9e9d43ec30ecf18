"""The affine quantizer's pins must reject plausible mistakes.

Each case plants one mistake in a copy of the oracle's C source (on the CPU,
in a temporary directory), builds it with gcc, and checks that the fixtures
of tests/test_oracle.py (the hand-worked groups and the numpy restatement on
random data) reject the mutant, while the unmodified source passes them.
"""
import ctypes
import os
import subprocess

import numpy as np
import pytest

import oracle

from test_oracle import GOLD, HAND, codes_bytestream, numpy_affine_quantize, bf16_from_torch, torch_from_bits

SRC = os.path.join(os.path.dirname(oracle.__file__), "mlxq_oracle.c")

MUTANTS = {
    # codes from the bf16-rounded scale and bias (MLX rounds them only when storing)
    "bf16_scale": ("w_el = rintf((w_el - bias) / scale);", "w_el = rintf((w_el - bf(bias)) / bf(scale));"),
    # round half away from zero instead of std::rint in the codes
    "roundf_codes": ("w_el = rintf((w_el - bias) / scale);", "w_el = roundf((w_el - bias) / scale);"),
    # ... and in q0
    "roundf_q0": ("float q0 = rintf(edge / scale);", "float q0 = roundf(edge / scale);"),
    # |w_min| >= |w_max| picks the w_min branch on ties
    "mask_ge": ("int mask = fabsf(w_min) > fabsf(w_max);", "int mask = fabsf(w_min) >= fabsf(w_max);"),
    # codes above 2^bits - 1 not clamped
    "no_clamp": ("w_el = std_min(std_max(w_el, 0.0f), n_bins);", "w_el = std_max(w_el, 0.0f);"),
    # no snapping of the scale to the edge
    "no_snap": ("scale = edge / q0;", "scale = scale;"),
}

MXFP4_MUTANTS = {
    # ties to the last LUT index instead of the first
    "mxfp4_last_min": ("if (d < best_d) {", "if (d <= best_d) {"),
    # no round-up of the e8m0 exponent
    "mxfp4_no_roundup": ("if (decoded < s) e += 1;", "(void)decoded;"),
}


def build(tmp_path, name, mutation):
    src = open(SRC).read()
    if mutation:
        old, new = mutation
        assert src.count(old) == 1, f"mutation site for {name} not found exactly once"
        src = src.replace(old, new)
    d = tmp_path / name
    d.mkdir()
    (d / "mlxq_oracle.c").write_text(src)
    hdr = os.path.join(os.path.dirname(SRC), "mlxq_oracle.h")
    (d / "mlxq_oracle.h").write_text(open(hdr).read())
    so = d / "liboracle.so"
    subprocess.run(["gcc", "-O2", "-std=c11", "-fPIC", "-ffp-contract=off", "-fno-fast-math", "-shared",
                    "-o", str(so), str(d / "mlxq_oracle.c"), "-lm"], check=True)
    lib = ctypes.CDLL(str(so))
    oracle._declare(lib)
    return lib


def quantizer_pins_pass(orc):
    kat = np.load(GOLD)
    for case in HAND:
        bits = int(case.rsplit("_b", 1)[1])
        wq, s, b = orc.affine_quantize(kat[f"hand_w_{case}"], 32, bits)
        if not (np.array_equal(codes_bytestream(wq, bits, 32), codes_bytestream(kat[f"hand_wq_{case}"], bits, 32))
                and np.array_equal(s, kat[f"hand_s_{case}"]) and np.array_equal(b, kat[f"hand_b_{case}"])):
            return False
    rng = np.random.default_rng(5)
    x = rng.standard_normal((16, 256)).astype(np.float32) * np.float32(0.02)
    w = bf16_from_torch(x)
    wf = torch_from_bits(w).float().numpy()
    for bits in (2, 4, 6, 8):
        codes, s, b = numpy_affine_quantize(wf, 64, bits)
        wq, so, bo = orc.affine_quantize(w, 64, bits)
        if not (np.array_equal(codes_bytestream(wq, bits, 256), codes)
                and np.array_equal(so.reshape(-1), bf16_from_torch(s))
                and np.array_equal(bo.reshape(-1), bf16_from_torch(b))):
            return False
    return True


def mxfp4_pins_pass(orc):
    kat = np.load(GOLD)
    wq, sc = orc.mxfp4_quantize(kat["mxfp4_hand_w"])
    return (np.array_equal(codes_bytestream(wq, 4, 96), codes_bytestream(kat["mxfp4_hand_wq"], 4, 96))
            and np.array_equal(sc, kat["mxfp4_hand_scales"]))


FP8_MUTANTS = {
    # round to nearest even instead of half-up
    "e4m3_rne": ("uint32_t m = (frac + 0x80000u) >> 20; /* 3 mantissa bits, half-up */",
                 "uint32_t m = (frac + 0x7FFFFu + ((frac >> 20) & 1u)) >> 20;"),
    # round subnormals to nearest instead of truncating
    "e4m3_sub_round": ("m = (frac | 0x800000u) >> (20 + (1 - be));",
                       "m = ((frac | 0x800000u) + (1u << (19 + (1 - be)))) >> (20 + (1 - be));"),
    # saturate at 448 instead of the NaN code for [464, 496)
    "e4m3_no_nan": ("return sign | (uint8_t)((be & 0xF) << 3) | (uint8_t)(m & 7u);",
                    "return (be == 15 && m == 7) ? (sign | 0x7E) : (sign | (uint8_t)((be & 0xF) << 3) | (uint8_t)(m & 7u));"),
    # underflow one exponent early (2^-9 would become zero)
    "e4m3_underflow": ("if (e < -9) return sign;", "if (e < -8) return sign;"),
}


def fp8_pins_pass(orc):
    kat = np.load(GOLD)
    if not np.array_equal(orc.e4m3_encode(kat["e4m3_hand_in"]), kat["e4m3_hand_code"]):
        return False
    wq, sc = orc.mxfp8_quantize(kat["mxfp8_hand_w"])
    return np.array_equal(wq, kat["mxfp8_hand_wq"]) and np.array_equal(sc, kat["mxfp8_hand_scales"])


@pytest.fixture
def swap_lib(monkeypatch):
    def swap(lib):
        monkeypatch.setattr(oracle, "_lib", lib)
    return swap


def test_unmodified_source_passes(tmp_path, swap_lib):
    swap_lib(build(tmp_path, "original", None))
    assert quantizer_pins_pass(oracle)
    assert mxfp4_pins_pass(oracle)
    assert fp8_pins_pass(oracle)


@pytest.mark.parametrize("name", sorted(MUTANTS))
def test_mutant_is_rejected(tmp_path, swap_lib, name):
    swap_lib(build(tmp_path, name, MUTANTS[name]))
    assert not quantizer_pins_pass(oracle), f"mutant {name} passes the quantizer pins"


@pytest.mark.parametrize("name", sorted(MXFP4_MUTANTS))
def test_mxfp4_mutant_is_rejected(tmp_path, swap_lib, name):
    swap_lib(build(tmp_path, name, MXFP4_MUTANTS[name]))
    assert not mxfp4_pins_pass(oracle), f"mutant {name} passes the mxfp4 pins"


@pytest.mark.parametrize("name", sorted(FP8_MUTANTS))
def test_fp8_mutant_is_rejected(tmp_path, swap_lib, name):
    swap_lib(build(tmp_path, name, FP8_MUTANTS[name]))
    assert not fp8_pins_pass(oracle), f"mutant {name} passes the fp8 pins"
