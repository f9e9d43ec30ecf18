"""mlxq_quantized_matmul_noalloc: the no-allocation variant of
mlxq_quantized_matmul, called through the C-ABI.  Its output must be the
existing entry point's, bit for bit (same kernels, same plan), on two calls in
a row (the second smaller, so stale scratch contents from the first would
show), for routes that use scratch (5-16-row decode partials, split-K
prefill) and one that does not; it must not grow any workspace; a call
needing more scratch than the fixed array returns MLXQ_ENOMEM; and a fresh
process whose first library call is a noalloc call under HIP-graph capture
(the scratch address resolved while the stream captures) replays it with new
activations bitwise equal to the eager entry point."""
import ctypes
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

import mlxcel_amd as mq
from mlxcel_amd import _lib
from mlxcel_amd.ops import _arr, _ref
from helpers import affine_case, announce, dev_bf16, dev_u32, host_u16, setknob

pytestmark = pytest.mark.gpu


def noalloc(X, W, S, B, out, stream):
    lib = _lib.load()
    ax, aw, as_, ab, ao = _arr(X), _arr(W), _arr(S), _arr(B), _arr(out)
    return lib.mlxq_quantized_matmul_noalloc(_ref(ax), _ref(aw), _ref(as_), _ref(ab), True, 64, 4, b"affine",
                                             _ref(ao), ctypes.c_void_p(stream.cuda_stream))


def case(M, N, K, seed):
    x, wq, s, b = affine_case(M, N, K, 64, 4, seed)
    return dev_bf16(x), dev_u32(wq), dev_bf16(s), dev_bf16(b)


# (large call, smaller call): decode 5-16 rows (K-range partials), prefill
# with split K (fp32 partials), decode 1 row (no scratch)
PAIRS = [
    ((16, 4096, 8192), (6, 1024, 2048)),
    ((256, 512, 8192), (64, 256, 4096)),
    ((1, 4096, 4096), (1, 512, 1024)),
]


@pytest.mark.parametrize("pair", PAIRS, ids=["mid", "prefill_splitk", "qmv"])
def test_noalloc_matches_quantized_matmul_twice(pair):
    st = torch.cuda.Stream()
    calls = []
    for i, (M, N, K) in enumerate(pair):
        X, W, S, B = case(M, N, K, 3000 + 10 * M + i)
        want = host_u16(mq.quantized_matmul(X, W, S, B, True, 64, 4))  # the existing entry point
        out = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
        calls.append((M, N, K, X, W, S, B, want, out))
    torch.cuda.synchronize()
    held = mq.get_cache_memory()
    for i, (M, N, K, X, W, S, B, want, out) in enumerate(calls):
        announce("noalloc", i, M, N, K)
        assert noalloc(X, W, S, B, out, st) == _lib.OK, _lib.last_error()
        st.synchronize()
        np.testing.assert_array_equal(host_u16(out), want, err_msg=f"call {i} {M}x{N}x{K}")
    # no workspace was created or grown for `st`
    assert mq.get_cache_memory() == held


def test_noalloc_rejects_calls_beyond_its_scratch(monkeypatch):
    # a forced 4-way K split of a 2048 x 4096 output needs 128 MiB of partials
    setknob(monkeypatch, "MLXQ_QMM_KSPLIT", "4")
    announce("noalloc_too_big")
    M, N, K = 2048, 4096, 4096
    X, W, S, B = case(M, N, K, 3100)
    out = torch.zeros(M, N, dtype=torch.bfloat16, device="cuda")
    st = torch.cuda.Stream()
    torch.cuda.synchronize()
    assert noalloc(X, W, S, B, out, st) == _lib.ENOMEM
    assert "scratch" in _lib.last_error()
    st.synchronize()
    assert float(out.float().abs().max()) == 0.0  # nothing ran


# Run in a fresh process, so the captured call is the first call into the
# library there: the device address of the fixed scratch is resolved while
# the stream is being captured.
CAPTURE_FIRST = r"""
import ctypes, sys
import numpy as np, torch
sys.path.insert(0, sys.argv[1]); sys.path.insert(0, sys.argv[1] + "/tests")
import mlxcel_amd as mq
from mlxcel_amd import _lib
from mlxcel_amd.ops import _arr, _ref
from helpers import affine_case, dev_bf16, dev_u32, host_u16
M, N, K = 16, 4096, 8192  # 5-16-row decode kernel with K-range partials in the scratch
x, wq, s, b = affine_case(M, N, K, 64, 4, 3200)
X, W, S, B = dev_bf16(x), dev_u32(wq), dev_bf16(s), dev_bf16(b)
out = torch.zeros(M, N, dtype=torch.bfloat16, device="cuda")
lib = _lib.load()
args = [_arr(t) for t in (X, W, S, B, out)]
st = torch.cuda.Stream()
torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g, stream=st):
    rc = lib.mlxq_quantized_matmul_noalloc(*[_ref(a) for a in args[:4]], True, 64, 4, b"affine", _ref(args[4]),
                                           ctypes.c_void_p(st.cuda_stream))
assert rc == _lib.OK, _lib.last_error()
assert mq.get_cache_memory() == 0  # nothing allocated by the library in this process
for rep in range(3):
    x2, _, _, _ = affine_case(M, N, K, 64, 4, 3300 + rep)  # new activations, same buffer
    X.copy_(dev_bf16(x2))
    out.zero_()
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    want = host_u16(mq.quantized_matmul(X, W, S, B, True, 64, 4))
    np.testing.assert_array_equal(host_u16(out), want, err_msg=f"replay {rep}")
print("capture-first noalloc: 3 replays bitwise equal", flush=True)
"""


def test_noalloc_first_call_under_capture_in_a_fresh_process():
    announce("noalloc_capture_first (subprocess)")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", CAPTURE_FIRST, root], capture_output=True, text=True, timeout=300)
    print(r.stdout[-2000:], r.stderr[-4000:], flush=True)
    assert r.returncode == 0, r.stderr[-4000:]
    assert "3 replays bitwise equal" in r.stdout
