"""HIP-graph capture of the hot path: the C-ABI entry points launch only
kernels on the caller's stream (no allocation, synchronisation or memset once
the workspace exists), so a captured quantized_matmul / gather_qmm replays
the same bits.  Each graph is replayed several times with eager work and
synchronisations in between, and every replay is compared with the eager
result bitwise.
"""
import numpy as np
import pytest
import torch

import mlxcel_amd as mq
import oracle as orc
from helpers import TOL, affine_case, announce, dev_bf16, dev_u32, dev_u8, host_u16, max_rel, mxfp4_case, setknob

pytestmark = pytest.mark.gpu


def capture(fn):
    # The library keeps its scratch per (device, stream): warm up on the
    # stream that is then captured, so the capture itself allocates nothing.
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        fn()
    return g


def replay_and_check(g, out, want_u16, other_work):
    for rep in range(3):
        out.zero_()
        other_work()  # eager work on the same device between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(host_u16(out), want_u16, err_msg=f"replay {rep}")


@pytest.mark.parametrize("kernel,M", [("rs", 1), ("rs", 2), ("fr", 1), ("mfma", 1), ("mfma", 8)])
def test_quantized_matmul_graph(monkeypatch, kernel, M):
    setknob(monkeypatch, "MLXQ_QMV_KERNEL", kernel)
    announce("graph_qmm", kernel, M)
    N, K = 1024, 4096
    x, wq, s, b = affine_case(M, N, K, 64, 4, 1200 + M)
    X, W, S, B = dev_bf16(x), dev_u32(wq), dev_bf16(s), dev_bf16(b)
    out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    eager = host_u16(mq.quantized_matmul(X, W, S, B, True, 64, 4))
    assert max_rel(eager, orc.qmm_t_affine(x, wq, s, b, 64, 4)) <= TOL
    g = capture(lambda: mq.quantized_matmul(X, W, S, B, True, 64, 4, out=out))
    junk = torch.randn(1 << 20, device="cuda")
    replay_and_check(g, out, eager, lambda: junk.mul_(1.0001))


def test_prefill_qmm_graph_with_split_k():
    # the prefill GEMM with K split across workgroups uses the stream's scratch
    announce("graph_qmm_prefill")
    M, N, K = 256, 256, 8192
    x, wq, s, b = affine_case(M, N, K, 64, 4, 1250)
    X, W, S, B = dev_bf16(x), dev_u32(wq), dev_bf16(s), dev_bf16(b)
    out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    eager = host_u16(mq.quantized_matmul(X, W, S, B, True, 64, 4))
    g = capture(lambda: mq.quantized_matmul(X, W, S, B, True, 64, 4, out=out))
    junk = torch.randn(1 << 20, device="cuda")
    replay_and_check(g, out, eager, lambda: junk.mul_(0.999))


def test_gather_qmm_graph():
    announce("graph_gather")
    E, N, K, T = 8, 576, 2880, 2
    x = orc.normal_bf16((T, 1, 1, K), 1.0, 1300)
    w = orc.normal_bf16((E, N, K), 0.02, 1301)
    wq, sc = orc.mxfp4_quantize(w)
    ids = np.array([[3, 0, 7, 5], [1, 3, 6, 2]], np.int32)
    X, W, S, I = dev_bf16(x), dev_u32(wq), dev_u8(sc), torch.from_numpy(ids).cuda()
    out = torch.empty(T, 4, 1, N, dtype=torch.bfloat16, device="cuda")
    eager = host_u16(mq.gather_qmm(X, W, S, None, None, I, True, 32, 4, "mxfp4"))
    g = capture(lambda: mq.gather_qmm(X, W, S, None, None, I, True, 32, 4, "mxfp4", out=out))
    junk = torch.randn(1 << 20, device="cuda")
    replay_and_check(g, out, eager, lambda: junk.add_(1.0))


def test_graph_sees_new_inputs_in_place():
    # a replay reads the captured buffers' current contents
    announce("graph_inplace")
    N, K = 512, 2048
    x1, wq, s, b = affine_case(1, N, K, 64, 4, 1400)
    x2 = orc.normal_bf16((1, K), 1.0, 1401)
    X, W, S, B = dev_bf16(x1), dev_u32(wq), dev_bf16(s), dev_bf16(b)
    out = torch.empty(1, N, dtype=torch.bfloat16, device="cuda")
    g = capture(lambda: mq.quantized_matmul(X, W, S, B, True, 64, 4, out=out))
    X.copy_(dev_bf16(x2))
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    want = host_u16(mq.quantized_matmul(dev_bf16(x2), W, S, B, True, 64, 4))
    np.testing.assert_array_equal(host_u16(out), want)


def test_capture_without_warmup_gets_a_status_and_an_intact_capture():
    # a call that needs workspace on a stream under capture returns
    # MLXQ_ENOMEM (no allocation, no synchronize) and the capture goes on
    announce("graph_no_warmup")
    M, N, K = 256, 256, 8192
    x, wq, s, b = affine_case(M, N, K, 64, 4, 1260)
    X, W, S, B = dev_bf16(x), dev_u32(wq), dev_bf16(s), dev_bf16(b)
    out = torch.zeros(M, N, dtype=torch.bfloat16, device="cuda")
    marker = torch.zeros(4, device="cuda")
    st = torch.cuda.Stream()  # never used: its workspace is empty
    g = torch.cuda.CUDAGraph()
    err = None
    with torch.cuda.graph(g, stream=st):
        try:
            mq.quantized_matmul(X, W, S, B, True, 64, 4, out=out)
        except mq.ops.QuantizedOpError as e:
            err = str(e)
        marker.add_(1.0)
    assert err is not None and "captured" in err, err
    for rep in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert float(marker[0]) == rep + 1
    # reserving up front makes the same capture work
    eager = host_u16(mq.quantized_matmul(X, W, S, B, True, 64, 4))
    st2 = torch.cuda.Stream()
    with torch.cuda.stream(st2):
        mq.workspace_reserve(64 << 20)
    torch.cuda.synchronize()
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2, stream=st2):
        mq.quantized_matmul(X, W, S, B, True, 64, 4, out=out)
    junk = torch.randn(1 << 20, device="cuda")
    replay_and_check(g2, out, eager, lambda: junk.mul_(0.5))


def test_replay_after_the_workspace_grew():
    # a graph captured with a small workspace still replays correctly after a
    # larger call on the same stream replaced the workspace (the old buffer
    # is kept, not freed)
    announce("graph_ws_growth")
    M, N, K = 8, 2048, 4096  # 5-16-row decode kernel: K-range partials in the workspace
    x, wq, s, b = affine_case(M, N, K, 64, 4, 1270)
    X, W, S, B = dev_bf16(x), dev_u32(wq), dev_bf16(s), dev_bf16(b)
    out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    eager = host_u16(mq.quantized_matmul(X, W, S, B, True, 64, 4))
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        mq.quantized_matmul(X, W, S, B, True, 64, 4, out=out)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        mq.quantized_matmul(X, W, S, B, True, 64, 4, out=out)
    held = mq.get_cache_memory()
    # a split-K prefill with much larger partials on the same stream
    M2, N2, K2 = 512, 4096, 14336
    x2, wq2, s2, b2 = affine_case(M2, N2, K2, 64, 4, 1271)
    X2, W2, S2, B2 = dev_bf16(x2), dev_u32(wq2), dev_bf16(s2), dev_bf16(b2)
    with torch.cuda.stream(st):
        big = mq.quantized_matmul(X2, W2, S2, B2, True, 64, 4)
    torch.cuda.synchronize()
    assert mq.get_cache_memory() >= held
    junk = torch.randn(1 << 22, device="cuda")
    replay_and_check(g, out, eager, lambda: junk.mul_(1.5))
    want_big = host_u16(mq.quantized_matmul(X2, W2, S2, B2, True, 64, 4))
    np.testing.assert_array_equal(host_u16(big), want_big)


def test_capture_with_strided_x_after_a_reserve():
    # a strided activation is copied into the stream's staging buffer first;
    # mlxq_workspace_reserve grows that buffer too, so a capture right after
    # a reserve (no eager warm-up on the stream) allocates nothing
    announce("graph_strided_reserve")
    M, N, K = 256, 256, 8192  # prefill with split K: scratch and staging both used
    x, wq, s, b = affine_case(M, N, K, 64, 4, 1280)
    W, S, B = dev_u32(wq), dev_bf16(s), dev_bf16(b)
    wide = torch.zeros(M, 2 * K, dtype=torch.bfloat16, device="cuda")
    wide[:, ::2] = dev_bf16(x)
    X = wide[:, ::2]  # stride 2 along K: needs the staging copy
    assert not X.is_contiguous()
    out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    eager = host_u16(mq.quantized_matmul(X.contiguous(), W, S, B, True, 64, 4))
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        mq.workspace_reserve(64 << 20)
    torch.cuda.synchronize()
    held = mq.get_cache_memory()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        mq.quantized_matmul(X, W, S, B, True, 64, 4, out=out)
    assert mq.get_cache_memory() == held
    junk = torch.randn(1 << 20, device="cuda")
    replay_and_check(g, out, eager, lambda: junk.mul_(0.25))
