"""GPU check of the end-to-end decode harness in bench.py (
Qwen3-8B shape, here at a small size): every linear layer of the decoder
runs through this library's quantized_matmul; the same decoder with each
quantized_matmul replaced by the float32 product of the bit-exact
dequantized weights (rounded to bf16 like the kernel's output) must give
the same logits within max|l - l_ref| / max|l_ref| <= 5e-2, for the prompt
(prefill GEMM path) and for graph-replayed decode steps (decode path),
and the graph replays must agree with eager steps.

The bound is wider than the 1e-2 each quantized_matmul is held to (tests/
test_gpu_qmv*.py, test_gpu_qmm.py): the whole network runs in bf16 (residual
stream, norms, attention), so single-ulp differences of the products compound
over the layers, and the prefill GEMM rounds its weights once, bf16(s*q + b),
where dequantize follows MLX's CPU graph, bf16(bf16(q*s) + b).
"""
import os
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import bench  # noqa: E402
import mlxcel_amd as mq  # noqa: E402
from helpers import announce  # noqa: E402

pytestmark = pytest.mark.gpu
E2E_TOL = 5e-2


class DequantDecoder(bench.QuantDecoder):
    """The same decoder with the quantized matmul done as a float32 product of
    the dequantized weights."""

    def qmm(self, x, w):
        wd = mq.dequantize(*w, self.gs, self.bits).float()
        return (x.float() @ wd.t()).to(torch.bfloat16)

    def qmm_n(self, x, ws):
        return [self.qmm(x, w) for w in ws]


def rel(a, b):
    a, b = a.float(), b.float()
    return float((a - b).abs().max() / b.abs().max())


@pytest.mark.parametrize("batch,rows_case", [(1, "decode M=1"), (12, "decode M=12")])
def test_decoder_matches_dequantized_reference(batch, rows_case):
    announce("e2e_decoder", batch)
    shape = bench.QwenShape(layers=2, hidden=512, nq=8, nkv=2, hd=64, inter=1024, vocab=2000)
    m = bench.QuantDecoder(shape, batch, 96, seed=5)
    r = DequantDecoder(shape, batch, 96, seed=5)
    g = torch.Generator(device="cuda").manual_seed(6)
    prompt = torch.randint(0, shape.vocab, (batch, 80), device="cuda", generator=g)
    lm, lr = m.prefill(prompt), r.prefill(prompt)
    assert rel(lm, lr) <= E2E_TOL
    for d in (m, r):
        d.tok = torch.argmax(lm, -1)
        d.pos = torch.full((), 80, dtype=torch.int64, device="cuda")
    gm, gr = m.decode_graph(96), r.decode_graph(96)
    for _ in range(4):
        gm.replay()
        gr.replay()
        torch.cuda.synchronize()
        assert rel(m.logits, r.logits) <= E2E_TOL
        r.tok.copy_(m.tok)  # teacher forcing: both continue from the same token


def test_graph_replay_matches_eager_step():
    announce("e2e_graph_vs_eager")
    shape = bench.QwenShape(layers=2, hidden=256, nq=4, nkv=2, hd=64, inter=512, vocab=1000)
    m = bench.QuantDecoder(shape, 2, 64, seed=7)
    prompt = torch.randint(0, shape.vocab, (2, 40), device="cuda", generator=torch.Generator(device="cuda").manual_seed(8))
    toks, _, _ = m.generate(prompt, 8, bucket=16)
    # eager: prefill then the same greedy steps without graphs
    e = bench.QuantDecoder(shape, 2, 64, seed=7)
    logits = e.prefill(prompt)
    tok = torch.argmax(logits, -1)
    G = shape.nq // shape.nkv
    for i in range(8):
        assert torch.equal(tok, toks[:, i])
        pos = torch.full((), 40 + i, dtype=torch.int64, device="cuda")
        T = ((40 + i + 1 + 15) // 16) * 16
        ar = torch.arange(T, device="cuda")
        mask = torch.where(ar[None, :] <= pos, 0.0, float("-inf")).expand(G, T)
        tok = torch.argmax(e.forward(tok, pos, 1, T, mask), -1)


def test_multi_projection_decoder_is_bitwise_the_separate_calls():
    # q/k/v and gate/up through quantized_matmul_multi (one launch each at
    # decode) against one quantized_matmul call per projection
    announce("e2e_multi_vs_separate")
    shape = bench.QwenShape(layers=2, hidden=512, nq=8, nkv=2, hd=64, inter=1024, vocab=2000)
    g = torch.Generator(device="cuda").manual_seed(9)
    prompt = torch.randint(0, shape.vocab, (1, 40), device="cuda", generator=g)
    a = bench.QuantDecoder(shape, 1, 64, seed=10, multi=True)
    b = bench.QuantDecoder(shape, 1, 64, seed=10, multi=False)
    ta, _, _ = a.generate(prompt, 6, bucket=16)
    tb, _, _ = b.generate(prompt, 6, bucket=16)
    assert torch.equal(ta, tb)
    assert torch.equal(a.logits, b.logits)
