"""GPU checks of the stream-K prefill plan (qmm_tile_kernel's stream-K
instantiation in qmm.hip): more 256 x 256 output tiles than CUs, one
workgroup per CU taking an equal run of the tiles' K-steps laid end to end
(the default plan where the last round holds at most 1/8 of the CUs'
tiles; MLXQ_QMM_STREAMK=L forces runs of L steps at other shapes).  A tile
cut by a run boundary is the sum of two pieces: the next run's first piece
(its tail, saved as fp32 partials) and this run's last piece (its head).  When the tail has not arrived, the head's
workgroup computes it itself; MLXQ_QMM_SK_FALLBACK=1 forces that path for
every cut tile, and since both paths add the same two fp32 pieces once, the
results are bitwise equal.  Results are checked against a float32 product of
the bit-exact dequantized weights (max|y - y_ref| / max|y_ref| <= 1e-2) and
against the plan without stream-K (MLXQ_QMM_STREAMK=0) within the same
bound; repeated calls, calls of other shapes in between and graph replays
check that every launch leaves its counters at 0.
"""
import numpy as np
import pytest
import torch

import mlxcel_amd as mq
from helpers import TOL, announce, host_u16, setknob

pytestmark = pytest.mark.gpu


def make(M, N, K, bits, seed, dt=torch.bfloat16):
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = (torch.randn(N, K, device="cuda", generator=g) * 0.02).to(dt)
    x = torch.randn(M, K, device="cuda", generator=g).to(dt)
    wq, s, b = mq.quantize(w, 64, bits)
    return x, (wq, s, b)


def force_runs(monkeypatch, M, N, K):
    """MLXQ_QMM_STREAMK set to the even run length of this shape (one run per CU)."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    tiles = -(-M // 256) * -(-N // 256)
    setknob(monkeypatch, "MLXQ_QMM_STREAMK", str(-(-tiles * (K // 64) // cus)))


def rel(y, ref):
    return float((y.float() - ref).abs().max() / ref.abs().max())


@pytest.mark.parametrize("mode", ["affine4", "affine8", "float16"])
@pytest.mark.parametrize("M,N,K,forced", [(1536, 12288, 4096, False), (2048, 14336, 4096, True),
                                           (1999, 12200, 2048, True), (4096, 14336, 1024, True),
                                           (1536, 14336, 4096, True)])
def test_streamk_fallback_bitwise_and_vs_dequant(monkeypatch, mode, M, N, K, forced):
    # 288 tiles (1.125 rounds of 256 CUs: the default plan), and forced runs
    # over 448 tiles (1.75 rounds), 384 ragged tiles (1.5), 896 tiles (3.5)
    # with short K, 336 tiles (1.31)
    announce("streamk", mode, M, N, K, forced)
    if forced:
        force_runs(monkeypatch, M, N, K)
    bits = 8 if mode == "affine8" else 4
    dt = torch.float16 if mode == "float16" else torch.bfloat16
    x, w = make(M, N, K, bits, 8100 + M + bits, dt)
    y = mq.quantized_matmul(x, *w, True, 64, bits)
    setknob(monkeypatch, "MLXQ_QMM_SK_FALLBACK", "1")
    y_fb = mq.quantized_matmul(x, *w, True, 64, bits)
    setknob(monkeypatch, "MLXQ_QMM_SK_FALLBACK", "0")
    y_again = mq.quantized_matmul(x, *w, True, 64, bits)
    setknob(monkeypatch, "MLXQ_QMM_STREAMK", "0")
    y_plain = mq.quantized_matmul(x, *w, True, 64, bits)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host_u16(y), host_u16(y_fb))
    np.testing.assert_array_equal(host_u16(y), host_u16(y_again))
    ref = x.float() @ mq.dequantize(*w, 64, bits).float().t()
    assert rel(y, ref) <= TOL
    assert rel(y_plain, ref) <= TOL
    assert rel(y, y_plain.float()) <= TOL


def test_streamk_counters_return_to_zero(monkeypatch):
    # stream-K calls of different run boundaries back to back, the forced
    # fallback in between (the tail then arrives second and resets), each
    # repeated: a counter left at 1 would make a later head add a stale tail
    announce("streamk_sequence")
    shapes = [(2048, 14336, 1024), (1999, 12200, 1024), (1536, 14336, 2048)]
    cases = [make(M, N, K, 4, 8200 + i) for i, (M, N, K) in enumerate(shapes)]
    first = []
    for rep in range(3):
        for j, (x, w) in enumerate(cases):
            force_runs(monkeypatch, *shapes[j])
            setknob(monkeypatch, "MLXQ_QMM_SK_FALLBACK", "1" if (rep + j) % 2 else "0")
            got = host_u16(mq.quantized_matmul(x, *w, True, 64, 4))
            if rep == 0:
                first.append(got)
            else:
                np.testing.assert_array_equal(got, first[j], err_msg=f"case {j} repeat {rep}")


def test_streamk_graph_replays(monkeypatch):
    announce("streamk_graph")
    M, N, K = 2048, 14336, 1024
    force_runs(monkeypatch, M, N, K)
    xs = [make(M, N, K, 4, 8300 + i)[0] for i in range(3)]
    _, w = make(M, N, K, 4, 8300)
    X = xs[0].clone()
    out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        mq.quantized_matmul(X, *w, True, 64, 4, out=out)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        mq.quantized_matmul(X, *w, True, 64, 4, out=out)
    torch.cuda.synchronize()
    for i in (0, 1, 2, 1):
        X.copy_(xs[i])
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(host_u16(out), host_u16(mq.quantized_matmul(X, *w, True, 64, 4)))
