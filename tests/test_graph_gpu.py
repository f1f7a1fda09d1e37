"""A whole layer step (forward and backward, bf16 masters quantized per call,
top-8 routing so that the gathered GEMMs run) captured in a HIP graph: every
replay gives the eager step's output and gradients bit for bit, with eager
steps and synchronizations between the replays (a captured memset or a
library call that writes differently on replay would show here)."""

import math

import pytest
import torch

import mlops_amd

pytestmark = pytest.mark.gpu


def test_layer_step_replays_bitwise_in_a_graph(device):
    g = torch.Generator().manual_seed(11)
    tokens, hidden, inter, experts, top_k = 512, 512, 256, 16, 8
    x = torch.randn(tokens, hidden, generator=g).to(torch.bfloat16).to(device)
    res = torch.randn(tokens, hidden, generator=g).to(torch.bfloat16).to(device)
    dy = torch.randn(tokens, hidden, generator=g).to(torch.bfloat16).to(device)
    wr = (torch.randn(experts, hidden, generator=g) / math.sqrt(hidden)).to(device)
    w13 = (torch.randn(experts, 2 * inter, hidden, generator=g) * 0.02).to(torch.bfloat16).to(device)
    w2 = (torch.randn(experts, hidden, inter, generator=g) * 0.02).to(torch.bfloat16).to(device)
    leaves = [t.requires_grad_(True) for t in (x, wr, w13, w2)]
    daux = torch.full((), 0.01, device=device)
    holder = {}

    def step():
        for t in leaves:
            t.grad = None
        out, aux, _, _ = mlops_amd.moe(x, res, wr, w13, w2, top_k=top_k,
                                       routing_mode="topk_then_softmax",
                                       compute_precision="fp8_block")
        torch.autograd.backward([out, aux], [dy, daux])
        holder["out"] = out.detach()

    def results():
        return [holder["out"].clone()] + [t.grad.clone() for t in leaves]

    for _ in range(2):
        step()
    torch.cuda.synchronize()
    want = results()

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    # The graph's own output tensors (an eager step below rebinds .grad).
    captured = [holder["out"]] + [t.grad for t in leaves]
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for got, ref in zip(captured, want):
            assert torch.equal(got, ref)
        step()
        torch.cuda.synchronize()
        for got, ref in zip(results(), want):
            assert torch.equal(got, ref)
