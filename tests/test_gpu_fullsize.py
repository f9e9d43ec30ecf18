"""The BASELINE configurations at their real shapes, checked through
size-independent references:

* configs[3], mxfp4 gather_qmm MoE (gpt-oss-20b-like): 32 experts, hidden
  2880, gate/up 5760 and down 2880, T in {1, 16, 256} tokens with top-4
  distinct experts drawn uniformly per token, sorted by expert when
  T * 4 >= 64 (the reference caller's rule, src/models/gpt_oss.rs:317-345)
  and as [T, 4] index arrays otherwise -- the routes and index layouts the
  benchmark times.  Reference: per expert, the float32 product of its
  bit-exact dequantized weights with its activation rows.
* configs[4], the Qwen3-8B-shaped decoder (36 layers, hidden 4096, 32/8
  heads, intermediate 12288, vocab 151936, 4-bit g64) at batch 1 and 16: a
  512-token prompt and 4 greedy decode steps, every projection call checked
  on the decoder's actual input against the float32 product of the
  dequantized weights (free-running, two decoders that differ only in the
  projections drift apart through 36 bf16 layers of random weights: 0.12
  relative on the prefill logits), then a graph-replayed decode step against
  the eager step, bitwise.

max|y - y_ref| / max|y_ref| <= 1e-2 for every gather and projection call.
"""
import os
import sys

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import bench  # noqa: E402
import mlxcel_amd as mq  # noqa: E402
from helpers import TOL, announce  # noqa: E402
from test_gpu_e2e import rel  # noqa: E402

pytestmark = pytest.mark.gpu

E, H, I2 = 32, 2880, 5760


@pytest.fixture(scope="module")
def experts():
    gu = bench.make_mxfp4(E, I2, H, 3060)
    dn = bench.make_mxfp4(E, H, H, 3070)
    deq = lambda w: mq.dequantize(w[0], w[1], None, 32, 4, "mxfp4").float()  # [E, N, K]
    return {"gate_up": (gu, deq(gu)), "down": (dn, deq(dn))}


@pytest.mark.parametrize("T", [1, 16, 256])
@pytest.mark.parametrize("proj", ["gate_up", "down"])
def test_gather_qmm_gpt_oss_shapes(experts, T, proj):
    announce("fullsize_gather", proj, T)
    (wq, sc), wd = experts[proj]
    N = wq.shape[1]
    rng = np.random.default_rng(3080 + T)
    ids = np.stack([rng.permutation(E)[:4] for _ in range(T)]).astype(np.int32)
    x = bench.randn_bf16((T, 1, 1, H), 3090 + T)
    if T * 4 >= 64:
        order = np.argsort(ids.reshape(-1), kind="stable")
        rhs = ids.reshape(-1)[order]
        xs = x.reshape(T, 1, H)[torch.from_numpy(order // 4).cuda()]  # [4T, 1, H]
        y = mq.gather_qmm(xs, wq, sc, None, None, torch.from_numpy(rhs).cuda(), True, 32, 4, "mxfp4",
                          sorted_indices=True).reshape(4 * T, N)
        xrows = xs.reshape(4 * T, H)
    else:
        rhs = ids.reshape(-1)
        y = mq.gather_qmm(x, wq, sc, None, None, torch.from_numpy(ids).cuda(), True, 32, 4,
                          "mxfp4").reshape(4 * T, N)
        xrows = x.reshape(T, H).repeat_interleave(4, 0)
    ref = torch.empty(4 * T, N, device="cuda")
    for e in np.unique(rhs):
        rows = torch.from_numpy(np.nonzero(rhs == e)[0]).cuda()
        ref[rows] = xrows[rows].float() @ wd[e].t()
    err = float((y.float() - ref).abs().max() / ref.abs().max())
    assert err <= TOL, err


class CheckedDecoder(bench.QuantDecoder):
    """The library decoder with every projection call checked against the
    float32 product of the bit-exact dequantized weights on the same input."""

    worst = 0.0
    calls = 0

    def _check(self, x, w, y):
        wd = mq.dequantize(*w, self.gs, self.bits).float()
        ref = x.float() @ wd.t()
        CheckedDecoder.worst = max(CheckedDecoder.worst, rel(y, ref))
        CheckedDecoder.calls += 1

    def qmm(self, x, w):
        y = super().qmm(x, w)
        self._check(x, w, y)
        return y

    def qmm_n(self, x, ws):
        ys = super().qmm_n(x, ws)
        for w, y in zip(ws, ys):
            self._check(x, w, y)
        return ys


@pytest.mark.parametrize("batch", [1, 16])
def test_qwen3_8b_shaped_decoder(batch):
    # The decoder at its real shape: a 512-token prompt (every projection on
    # the prefill GEMM) and 4 greedy decode steps (the decode kernels at 1 or
    # 16 rows; q/k/v and gate/up as one multi-projection launch), every one of
    # the 36 x 7 projection calls per pass and the 151936-wide LM head checked
    # on its actual input, then the graph-replayed decode step against the
    # eager step, bitwise.  (Free-running, two decoders that differ only in
    # these projections drift apart through 36 bf16 layers of random weights:
    # 0.12 relative on the prefill logits, so the check is per call.)
    announce("fullsize_decoder", batch)
    shape = bench.QwenShape()  # 36 layers, hidden 4096, vocab 151936
    S, steps, T = 512, 4, 576
    m = CheckedDecoder(shape, batch, T, seed=21)
    G = shape.nq // shape.nkv
    g = torch.Generator(device="cuda").manual_seed(22)
    prompt = torch.randint(0, shape.vocab, (batch, S), device="cuda", generator=g)
    CheckedDecoder.worst, CheckedDecoder.calls = 0.0, 0
    with torch.no_grad():
        logits = m.prefill(prompt)
        print(f"[fullsize decoder] batch {batch} prefill: {CheckedDecoder.calls} projections, "
              f"worst rel err {CheckedDecoder.worst:.3e}", flush=True)
        assert CheckedDecoder.calls == 36 * 7 + 1 and CheckedDecoder.worst <= TOL
        tok = torch.argmax(logits, -1)
        ar = torch.arange(T, device="cuda")
        for i in range(steps):
            CheckedDecoder.worst, CheckedDecoder.calls = 0.0, 0
            pos = torch.full((), S + i, dtype=torch.int64, device="cuda")
            mask = torch.where(ar[None, :] <= pos, 0.0, float("-inf")).expand(G, T)
            logits = m.forward(tok, pos, 1, T, mask)
            print(f"[fullsize decoder] batch {batch} decode step {i}: worst rel err {CheckedDecoder.worst:.3e}",
                  flush=True)
            assert CheckedDecoder.calls == 36 * 7 + 1 and CheckedDecoder.worst <= TOL
            tok = torch.argmax(logits, -1)
        # graph replay == eager step, bitwise (the plain library decoder)
        p = bench.QuantDecoder.__new__(bench.QuantDecoder)
        p.__dict__.update(m.__dict__)
        p.tok = tok.clone()
        p.pos = torch.full((), S + steps, dtype=torch.int64, device="cuda")
        kc = [k.clone() for k in p.kc]
        vc = [v.clone() for v in p.vc]
        gm = p.decode_graph(T)
        gm.replay()
        torch.cuda.synchronize()
        graph_logits = p.logits.clone()
        for i in range(len(p.layers)):
            p.kc[i].copy_(kc[i])
            p.vc[i].copy_(vc[i])
        pos = torch.full((), S + steps, dtype=torch.int64, device="cuda")
        mask = torch.where(ar[None, :] <= pos, 0.0, float("-inf")).expand(G, T)
        assert torch.equal(graph_logits, p.forward(tok, pos, 1, T, mask))
