"""C-ABI checks that need no GPU: the library loads, exports every entry point
include/mlxq.h declares, and validates arguments exactly as the reference op
layer does (overlays/rocm/mlx/ops.cpp:111-179, 4846-5008, 5454-5492,
5494-5805, 5841-5948) before any device work.  Only calls that must fail
validation are made here."""
import ctypes
import os
import re
import subprocess

import pytest

from mlxcel_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mlxq.h")


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(mlxq_[a-z_]+)\s*\(", text)))


def test_header_declares_the_abi():
    assert declared_symbols() == sorted(_lib.SYMBOLS)


def test_library_exports_every_declared_symbol(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r" T (mlxq_\w+)", out))
    missing = set(declared_symbols()) - exported
    assert not missing, f"not exported: {missing}"
    assert lib.mlxq_version().decode().startswith("mlxq ")


def arr(shape, dtype, strides=None):
    a = _lib.MlxqArray()
    a.data = None
    a.dtype = dtype
    a.ndim = len(shape)
    st = strides
    if st is None:
        st, acc = [], 1
        for d in reversed(shape):
            st.insert(0, acc)
            acc *= d
    for i, (d, s) in enumerate(zip(shape, st)):
        a.shape[i] = d
        a.strides[i] = s
    return a


def qmm_shape(lib, x, w, s, b, transpose=True, gs=64, bits=4, mode=b"affine"):
    nd, sh, dt = ctypes.c_int32(), (ctypes.c_int64 * 8)(), ctypes.c_int32()
    st = lib.mlxq_quantized_matmul_shape(ctypes.byref(x), ctypes.byref(w), ctypes.byref(s),
                                         ctypes.byref(b) if b is not None else None, transpose, gs, bits, mode,
                                         ctypes.byref(nd), sh, ctypes.byref(dt))
    return st, tuple(sh[: nd.value]), dt.value


BF, U32, U8, F32, F16, I32 = _lib.BFLOAT16, _lib.UINT32, _lib.UINT8, _lib.FLOAT32, _lib.FLOAT16, _lib.INT32


def test_shape_and_dtype_rules(lib):
    x = arr([3, 1, 4096], BF)
    w = arr([14336, 512], U32)
    s = arr([14336, 64], BF)
    st, shape, dt = qmm_shape(lib, x, w, s, s)
    assert st == 0 and shape == (3, 1, 14336) and dt == BF
    # promotion: x f32 with bf16 scales -> f32 (upstream type rules)
    st, shape, dt = qmm_shape(lib, arr([2, 4096], F32), w, s, s)
    assert st == 0 and dt == F32
    # f16 x with bf16 scales -> f32
    st, _, dt = qmm_shape(lib, arr([2, 4096], F16), w, s, s)
    assert st == 0 and dt == F32
    # defaults from the mode (group_size/bits <= 0)
    st, shape, _ = qmm_shape(lib, x, w, s, s, gs=-1, bits=-1)
    assert st == 0 and shape == (3, 1, 14336)
    # batched x and w broadcast their batch dims
    st, shape, _ = qmm_shape(lib, arr([1, 5, 4096], BF), arr([3, 64, 512], U32), arr([3, 64, 64], BF),
                             arr([3, 64, 64], BF))
    assert st == 0 and shape == (3, 5, 64)
    # mxfp4: uint8 scales, no biases, output follows x
    st, shape, dt = qmm_shape(lib, arr([1, 2880], BF), arr([5760, 360], U32), arr([5760, 90], U8), None,
                              gs=32, bits=4, mode=b"mxfp4")
    assert st == 0 and shape == (1, 5760) and dt == BF


@pytest.mark.parametrize("case,msg", [
    ("bad_mode", "[quantized_matmul] Invalid quantization mode 'int4'."),
    ("no_biases", "[quantized_matmul] Biases must be provided for affine quantization."),
    ("w_dtype", "[quantized_matmul] The weight matrix should be uint32 but received int32"),
    ("sb_shape", "[quantized_matmul] Scales and biases should have the same shape. Received scales with shape "
                 "(14336,64) and biases with (14336,32)"),
    ("gs_bits", "[quantized_matmul] The shapes of the weight and scales are incompatible based on bits and "
                "group_size. w.shape() == (14336,512) and scales.shape() == (14336,64) with group_size=32 and bits=4"),
    ("inner", "[quantized_matmul] Last dimension of first input with shape (..., 4000) does not match the expanded "
              "quantized matrix (4096, 14336) computed from shape (14336,512) with group_size=64, bits=4 and "
              "transpose=true"),
    ("fp_scales", "[quantized_matmul] Scale type must be uint8 but received type bfloat16."),
    ("fp_biases", "[quantized_matmul] Biases must be null for quantization mode 'mxfp4'."),
    ("int_scales", "[quantized_matmul] Only real floating types are supported but scales.dtype() == int32 and "
                   "biases.dtype() == int32."),
    ("x_int", "[quantized_matmul] Only real floating types are supported but x.dtype() == int32."),
    ("batch", "[quantized_matmul] Weight and scales should have the same batch shape. Received weight with shape "
              "(2,64,512), scales with (3,64,64)."),
])
def test_validation_messages(lib, case, msg):
    x = arr([1, 4096], BF)
    w = arr([14336, 512], U32)
    s = arr([14336, 64], BF)
    b = s
    gs, bits, mode = 64, 4, b"affine"
    if case == "bad_mode":
        mode = b"int4"
    elif case == "no_biases":
        b = None
    elif case == "w_dtype":
        w = arr([14336, 512], I32)
    elif case == "sb_shape":
        b = arr([14336, 32], BF)
    elif case == "gs_bits":
        gs = 32
    elif case == "inner":
        x = arr([1, 4000], BF)
    elif case == "fp_scales":
        mode, b, gs = b"mxfp4", None, 32
    elif case == "fp_biases":
        mode, s, b, gs = b"mxfp4", arr([14336, 64], U8), arr([14336, 64], U8), 32
        w = arr([14336, 256], U32)
    elif case == "int_scales":
        s = b = arr([14336, 64], I32)
    elif case == "x_int":
        # int x promotes with bf16 scales in affine mode; fp modes keep x's dtype
        x, mode, b, gs = arr([1, 4096], I32), b"mxfp4", None, 32
        w, s = arr([14336, 512], U32), arr([14336, 128], U8)
    elif case == "batch":
        w, s, b = arr([2, 64, 512], U32), arr([3, 64, 64], BF), arr([3, 64, 64], BF)
    st, _, _ = qmm_shape(lib, x, w, s, b, gs=gs, bits=bits, mode=mode)
    assert st == _lib.EINVAL
    assert _lib.last_error() == msg
    # the compute entry point rejects the same arguments before touching the device
    out = arr([1, 14336], BF)
    st2 = lib.mlxq_quantized_matmul(ctypes.byref(x), ctypes.byref(w), ctypes.byref(s),
                                    ctypes.byref(b) if b is not None else None, True, gs, bits, mode,
                                    ctypes.byref(out), None)
    assert st2 == _lib.EINVAL and _lib.last_error() == msg


def test_out_shape_mismatch_is_rejected(lib):
    x, w, s = arr([2, 4096], BF), arr([64, 512], U32), arr([64, 64], BF)
    out = arr([2, 63], BF)
    st = lib.mlxq_quantized_matmul(ctypes.byref(x), ctypes.byref(w), ctypes.byref(s), ctypes.byref(s), True, 64, 4,
                                   b"affine", ctypes.byref(out), None)
    assert st == _lib.EINVAL and "out must have shape (2,64)" in _lib.last_error()


def gather_shape(lib, x, w, s, b, lhs, rhs, gs=64, bits=4, mode=b"affine"):
    nd, sh, dt = ctypes.c_int32(), (ctypes.c_int64 * 8)(), ctypes.c_int32()
    ref = lambda a: ctypes.byref(a) if a is not None else None  # noqa: E731
    st = lib.mlxq_gather_qmm_shape(ref(x), ref(w), ref(s), ref(b), ref(lhs), ref(rhs), True, gs, bits, mode,
                                   ctypes.byref(nd), sh, ctypes.byref(dt))
    return st, tuple(sh[: nd.value]), dt.value


def test_gather_shapes_and_errors(lib):
    # gpt-oss decode: x [T,1,1,K], rhs [T,4] -> out [T,4,1,N]
    x = arr([16, 1, 1, 2880], BF)
    w = arr([32, 5760, 360], U32)
    s = arr([32, 5760, 90], U8)
    st, shape, dt = gather_shape(lib, x, w, s, None, None, arr([16, 4], U32), gs=32, mode=b"mxfp4")
    assert st == 0 and shape == (16, 4, 1, 5760) and dt == BF
    # sorted path: x [B,1,K], rhs [B]
    st, shape, _ = gather_shape(lib, arr([64, 1, 2880], BF), w, s, None, None, arr([64], U32), gs=32, mode=b"mxfp4")
    assert st == 0 and shape == (64, 1, 5760)
    # non-integral indices
    st, _, _ = gather_shape(lib, x, w, s, None, None, arr([16, 4], F32), gs=32, mode=b"mxfp4")
    assert st == _lib.EINVAL
    assert _lib.last_error() == "[gather_qmm] Got indices with invalid dtype. Indices must be integral."
    # x with one dimension
    st, _, _ = gather_shape(lib, arr([2880], BF), w, s, None, None, arr([4], U32), gs=32, mode=b"mxfp4")
    assert st == _lib.EINVAL
    assert _lib.last_error() == ("[gather_qmm] Input must have at least two dimensions but got input with shape "
                                 "(2880).")
    # indices that do not broadcast
    st, _, _ = gather_shape(lib, x, w, s, None, arr([3], U32), arr([16, 4], U32), gs=32, mode=b"mxfp4")
    assert st == _lib.EINVAL
    assert _lib.last_error() == "[broadcast_shapes] Shapes (3) and (16,4) cannot be broadcast."
    # global scale outside nvfp4
    out = arr([16, 4, 1, 5760], BF)
    gsc = arr([32], F32)
    st = lib.mlxq_gather_qmm(ctypes.byref(x), ctypes.byref(w), ctypes.byref(s), None, None,
                             ctypes.byref(arr([16, 4], U32)), True, 32, 4, False, b"mxfp4", ctypes.byref(gsc),
                             ctypes.byref(out), None)
    assert st == _lib.EINVAL
    assert _lib.last_error() == "[gather_qmm] Global scale is only supported for 'nvfp4' quantization mode."


def test_dequantize_and_quantize_errors(lib):
    w, s = arr([64, 512], U32), arr([64, 64], BF)
    out = arr([64, 4096], BF)
    st = lib.mlxq_dequantize(ctypes.byref(w), ctypes.byref(s), ctypes.byref(arr([64, 32], BF)), 64, 4, b"affine", -1,
                             ctypes.byref(out), None)
    assert st == _lib.EINVAL
    assert _lib.last_error() == "[dequantize] Shape of scales and biases does not match the matrix"
    st = lib.mlxq_dequantize(ctypes.byref(w), ctypes.byref(arr([64, 128], U8)), None, 16, 4, b"mxfp4", -1,
                             ctypes.byref(out), None)
    assert st == _lib.EINVAL
    assert _lib.last_error() == "[dequantize] mxfp4 quantization requires group size 32 but got 16."
    wt = arr([64, 4096], BF)
    q, sc, bi = arr([64, 512], U32), arr([64, 64], BF), arr([64, 64], BF)
    st = lib.mlxq_quantize(ctypes.byref(wt), 48, 4, b"affine", ctypes.byref(q), ctypes.byref(sc), ctypes.byref(bi),
                           None)
    assert st == _lib.EINVAL
    assert _lib.last_error() == ("[quantize] The last dimension of the matrix needs to be divisible by the "
                                 "quantization group size 48. However the provided  matrix has shape (64,4096)")
    st = lib.mlxq_quantize(ctypes.byref(wt), 64, 7, b"affine", ctypes.byref(q), ctypes.byref(sc), ctypes.byref(bi),
                           None)
    assert st == _lib.EINVAL
    assert _lib.last_error() == ("[quantize] The requested number of bits 7 is not supported. The supported bits are "
                                 "1, 2, 3, 4, 5, 6 and 8.")


def test_unimplemented_combinations_say_so(lib):
    # mxfp8 matmuls are valid for MLX but not implemented here (refused before
    # any device work, so the caller can fall back)
    x, w, s = arr([1, 64], BF), arr([64, 16], U32), arr([64, 2], U8)
    out = arr([1, 64], BF)
    st = lib.mlxq_quantized_matmul(ctypes.byref(x), ctypes.byref(w), ctypes.byref(s), None, True, 32, 8,
                                   b"mxfp8", ctypes.byref(out), None)
    assert st == _lib.EUNSUPPORTED and "mxfp8" in _lib.last_error()
    # float64 activations promote the result to float64
    x64, w4, s4 = arr([1, 64], _lib.FLOAT64), arr([64, 8], U32), arr([64, 1], BF)
    out64 = arr([1, 64], _lib.FLOAT64)
    st = lib.mlxq_quantized_matmul(ctypes.byref(x64), ctypes.byref(w4), ctypes.byref(s4), ctypes.byref(s4), True, 64,
                                   4, b"affine", ctypes.byref(out64), None)
    assert st == _lib.EUNSUPPORTED and "float64" in _lib.last_error()


def moe_args(din=256, dff=128, E=4, k=2, gu=4, db=4, gs=64, x_dtype=BF, idx_dtype=_lib.INT32, sc_dtype=_lib.FLOAT32):
    return [arr([din], x_dtype), arr([k], idx_dtype),
            arr([E, dff, din * gu // 32], U32), arr([E, dff, din // gs], BF), arr([E, dff, din // gs], BF),
            arr([E, dff, din * gu // 32], U32), arr([E, dff, din // gs], BF), arr([E, dff, din // gs], BF),
            arr([E, din, dff * db // 32], U32), arr([E, din, dff // gs], BF), arr([E, din, dff // gs], BF),
            arr([k], sc_dtype)]


def call_moe(lib, args, din, dff, k, gu, db, gs, out=None, geglu=False):
    out = out if out is not None else arr([din], BF)
    fn = lib.mlxq_fused_moe_geglu if geglu else lib.mlxq_fused_moe_expert
    return fn(*[ctypes.byref(a) for a in args], din, dff, k, gu, db, gs, ctypes.byref(out), None)


def test_fused_moe_validation(lib):
    # shapes that disagree with din / dff / k are argument errors
    a = moe_args()
    assert call_moe(lib, a, 256, 128, 3, 4, 4, 64) == _lib.EINVAL
    assert "indices must have k elements" in _lib.last_error()
    assert call_moe(lib, a, 256, 192, 2, 4, 4, 64) == _lib.EINVAL
    assert "gate_w must have shape (4,192,32)" in _lib.last_error()
    assert call_moe(lib, a, 256, 128, 2, 4, 4, 64, out=arr([128], BF)) == _lib.EINVAL
    assert call_moe(lib, moe_args(din=96), 96, 128, 2, 4, 4, 64, geglu=True) == _lib.EINVAL
    assert "multiples of group_size" in _lib.last_error()
    # valid for the reference's callers but not implemented: they fall back
    assert call_moe(lib, moe_args(gu=2), 256, 128, 2, 2, 4, 64) == _lib.EUNSUPPORTED
    assert call_moe(lib, moe_args(db=3), 256, 128, 2, 4, 3, 64) == _lib.EUNSUPPORTED
    assert call_moe(lib, moe_args(gs=16), 256, 128, 2, 4, 4, 16) == _lib.EUNSUPPORTED
    assert call_moe(lib, moe_args(x_dtype=_lib.FLOAT16), 256, 128, 2, 4, 4, 64) == _lib.EUNSUPPORTED
    assert call_moe(lib, moe_args(sc_dtype=_lib.INT32), 256, 128, 2, 4, 4, 64) == _lib.EUNSUPPORTED
    assert call_moe(lib, moe_args(idx_dtype=_lib.INT16), 256, 128, 2, 4, 4, 64) == _lib.EUNSUPPORTED
    assert "fused_moe_expert_kernel" in _lib.last_error()


def test_quantized_linear_and_dense_gemm_predicate(lib):
    x, w, s = arr([1, 64], BF), arr([64, 8], U32), arr([64, 1], BF)
    assert lib.mlxq_quantized_matmul_matches_dense_gemm(ctypes.byref(x), ctypes.byref(w), ctypes.byref(s),
                                                        ctypes.byref(s), 64, 4) == 0
    out = arr([1, 64], BF)

    def lin(bias):
        return lib.mlxq_quantized_linear(ctypes.byref(x), ctypes.byref(w), ctypes.byref(s), ctypes.byref(s),
                                         ctypes.byref(bias), 64, 4, b"affine", ctypes.byref(out), None)

    assert lin(arr([32], BF)) == _lib.EUNSUPPORTED and "linear_bias must have shape" in _lib.last_error()
    assert lin(arr([64], F32)) == _lib.EUNSUPPORTED and "dtype" in _lib.last_error()
    # argument errors of the matmul itself come first, with the reference's text
    bad = arr([1, 32], BF)
    st = lib.mlxq_quantized_linear(ctypes.byref(bad), ctypes.byref(w), ctypes.byref(s), ctypes.byref(s), None, 64, 4,
                                   b"affine", ctypes.byref(out), None)
    assert st == _lib.EINVAL


def test_sizes_no_launch_covers_are_refused_before_device_work(lib):
    # what the splits cannot bring below one launch's limits is refused with
    # MLXQ_EUNSUPPORTED (the caller falls back) before any device call
    # one activation row of 2 GiB (2^30 bf16): no row chunk fits a buffer resource
    K = 1 << 30
    x, w, s = arr([1, K], BF), arr([1, K // 8], U32), arr([1, K // 64], BF)
    out = arr([1, 1], BF)
    st = lib.mlxq_quantized_matmul(ctypes.byref(x), ctypes.byref(w), ctypes.byref(s), ctypes.byref(s), True, 64, 4,
                                   b"affine", ctypes.byref(out), None)
    assert st == _lib.EUNSUPPORTED and "reaches 2 GiB" in _lib.last_error()
    # 2^30 gather entries (the chunked gather's flat index lists stay below 2^30)
    B = 1 << 30
    xg, wg, sg, rhs = arr([B, 1, 64], BF), arr([4, 64, 8], U32), arr([4, 64, 1], BF), arr([B], U32)
    outg = arr([B, 1, 64], BF)
    st = lib.mlxq_gather_qmm(ctypes.byref(xg), ctypes.byref(wg), ctypes.byref(sg), ctypes.byref(sg), None,
                             ctypes.byref(rhs), True, 64, 4, False, b"affine", None, ctypes.byref(outg), None)
    assert st == _lib.EUNSUPPORTED and "2^30 index entries" in _lib.last_error()
    # conversions of 2^34 elements (beyond one launch grid)
    rows, Kd = 1 << 20, 1 << 14
    wd, sd, od = arr([rows, Kd // 8], U32), arr([rows, Kd // 64], BF), arr([rows, Kd], BF)
    st = lib.mlxq_dequantize(ctypes.byref(wd), ctypes.byref(sd), ctypes.byref(sd), 64, 4, b"affine", -1,
                             ctypes.byref(od), None)
    assert st == _lib.EUNSUPPORTED and "2^34" in _lib.last_error()
    st = lib.mlxq_quantize(ctypes.byref(od), 64, 4, b"affine", ctypes.byref(wd), ctypes.byref(sd), ctypes.byref(sd),
                           None)
    assert st == _lib.EUNSUPPORTED and "2^34" in _lib.last_error()
