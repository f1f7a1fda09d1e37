"""The two-region composed form (``mi355x.moe.composed``) on the GPU.

Its regions run the fused operator's kernels. The bf16 ``dh`` that crosses
the region boundary is quantized by the row and transposing quantizers, which
equal the fused SwiGLU backward's own quantizers byte for byte. So every
output and gradient must equal the fused operator's **bitwise**. The fused
operator is itself pinned against the CPU oracle (tests/test_moe_gpu.py).
Also checked:
* the prepare region recomputed under activation checkpointing changes no
  gradient (the rematerialization this form exists for);
* the donating finish VJP equals the functional one, with ``grad_h13``
  written over ``h13``;
* fake-tensor schemas of all five operators;
* selection: the fused operator stays the default, the composed one is used
  when forced.
"""

import math

import pytest
import torch
import torch.utils.checkpoint

import mlops_amd
from mlops_amd import BlockFP8Weight
from mlops_amd import kernels as K
from mlops_amd.dispatch import explain_implementation, use_implementation
from mlops_amd.providers.mi355x import moe_composed as C

pytestmark = pytest.mark.gpu

FUSED, COMPOSED = "mi355x.moe.block_fp8", "mi355x.moe.composed"


def _inputs(device, tokens=256, hidden=512, experts=8, inter=256, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(tokens, hidden, generator=g).to(torch.bfloat16)
    res = torch.randn(tokens, hidden, generator=g).to(torch.bfloat16)
    wr = torch.randn(experts, hidden, generator=g) / math.sqrt(hidden)
    w13 = (torch.randn(experts, 2 * inter, hidden, generator=g) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn(experts, hidden, inter, generator=g) * 0.02).to(torch.bfloat16)
    dy = torch.randn(tokens, hidden, generator=g).to(torch.bfloat16)
    return [t.to(device) for t in (x, res, wr, w13, w2, dy)]


def _run(implementation, x, res, wr, w13, w2, dy, *, containers=True, **kw):
    x = x.clone().requires_grad_(True)
    res = res.clone().requires_grad_(True)
    wr = wr.clone().requires_grad_(True)
    if containers:
        w13 = BlockFP8Weight.quantize(w13).detach().requires_grad_(True)
        w2 = BlockFP8Weight.quantize(w2).detach().requires_grad_(True)
    else:
        w13 = w13.clone().requires_grad_(True)
        w2 = w2.clone().requires_grad_(True)
        kw.setdefault("compute_precision", "fp8_block")
    with use_implementation("moe", implementation):
        out, aux, counts, psum = mlops_amd.moe(x, res, wr, w13, w2, **kw)
    torch.autograd.backward([out, aux, psum],
                           [dy, torch.ones_like(aux) * 0.1, torch.full_like(psum, 0.01)])
    return dict(out=out.detach(), aux=aux.detach(), counts=counts, psum=psum.detach(),
                gx=x.grad, gres=res.grad, gr=wr.grad, g13=w13.grad, g2=w2.grad)


def _assert_equal(a, b):
    for key in a:
        assert torch.equal(a[key], b[key]), key


@pytest.mark.parametrize("mode,kw", [
    ("topk_then_softmax", {}),
    ("softmax_then_topk", dict(swiglu_limit=4.0)),
    ("sigmoid_noaux_tc", dict(n_group=4, topk_group=2, routed_scaling=2.5,
                              lengths=(100, 156))),
])
def test_composed_equals_fused_bitwise(device, mode, kw):
    args = _inputs(device, seed=3)
    fused = _run(FUSED, *args, top_k=2, routing_mode=mode, **kw)
    composed = _run(COMPOSED, *args, top_k=2, routing_mode=mode, **kw)
    _assert_equal(fused, composed)


def test_composed_equals_fused_with_per_call_weights(device):
    """Plain bf16 masters, quantized per call (the C3 bench's weights)."""
    args = _inputs(device, tokens=384, hidden=256, experts=16, inter=128, seed=4)
    fused = _run(FUSED, *args, containers=False, top_k=4, routing_mode="topk_then_softmax")
    composed = _run(COMPOSED, *args, containers=False, top_k=4,
                    routing_mode="topk_then_softmax")
    _assert_equal(fused, composed)


def test_default_selection_is_fused_and_composed_when_forced(device):
    x, res, wr, w13, w2, _ = _inputs(device, tokens=32, seed=5)
    opts = dict(top_k=2, routing_mode="topk_then_softmax", compute_precision="fp8_block")
    assert explain_implementation("moe", x, res, wr, w13, w2, **opts).selected == FUSED
    with use_implementation("moe", COMPOSED):
        assert explain_implementation("moe", x, res, wr, w13, w2, **opts).selected == COMPOSED


def test_checkpointed_prepare_region_matches(device):
    """The prepare region recomputed in backward (what AOT rematerialization
    does with it) gives the same gradients, bitwise: it is deterministic and
    the finish region is not replayed."""
    x, res, wr, w13, w2, dy = _inputs(device, seed=6)
    w13c = BlockFP8Weight.quantize(w13).detach()
    w2c = BlockFP8Weight.quantize(w2).detach()
    rows = x.shape[0]

    def prepare(xv, wrv, w13v):
        outs = C._prepare_op(xv, wrv, w13v, torch.empty(0, device=device), 2,
                             "topk_then_softmax", 1, 1, 1.0, [rows], "float32", None, [])
        return outs[0], outs[4], outs[6], outs[7], outs[8], outs[9]

    def step(checkpointed):
        xv = x.clone().requires_grad_(True)
        wrv = wr.clone().requires_grad_(True)
        w13v = w13c.detach().requires_grad_(True)
        w2v = w2c.detach().requires_grad_(True)
        if checkpointed:
            aux, weights, order, offsets, slots, h13 = torch.utils.checkpoint.checkpoint(
                prepare, xv, wrv, w13v, use_reentrant=False)
        else:
            aux, weights, order, offsets, slots, h13 = prepare(xv, wrv, w13v)
        out = C._finish_op(h13, w2v, weights, order, offsets, slots, res, 2, None, None, [])
        torch.autograd.backward([out, aux], [dy, torch.ones_like(aux) * 0.1])
        return dict(out=out.detach(), gx=xv.grad, gr=wrv.grad, g13=w13v.grad, g2=w2v.grad)

    _assert_equal(step(False), step(True))


def _finish_state(device, seed=7):
    x, res, wr, w13, w2, dy = _inputs(device, seed=seed)
    w13q, w13s = K.quantize_weight_blocks(w13)
    w2q, w2s = K.quantize_weight_blocks(w2)
    rows = x.shape[0]
    outs = C._prepare_op(x, wr, w13q, torch.empty(0, device=device), 2, "topk_then_softmax", 1,
                         1, 1.0, [rows], "float32", None, [w13s])
    return x, res, wr, (w13q, w13s), (w2q, w2s), dy, outs


def test_donating_finish_vjp_matches_functional(device):
    _, _, _, _, (w2q, w2s), dy, outs = _finish_state(device)
    (_, _, _, _, weights, _, order, offsets, slots, h13) = outs
    ops = torch.ops.mlops_mi355x
    args = (weights, order, offsets, slots, 2, None, 4.0, [w2s], True)
    grad_h13, grad_w2, grad_rw, grad_res = ops.moe_mi355x_finish_bwd(dy, h13, w2q, *args)
    donated = h13.clone()
    d_w2, d_rw, d_res = ops.moe_mi355x_finish_bwd_donate_h13(dy, donated, w2q, *args)
    assert torch.equal(donated, grad_h13)
    assert not torch.equal(donated, h13)
    assert torch.equal(d_w2, grad_w2) and torch.equal(d_rw, grad_rw)
    assert torch.equal(d_res, grad_res) and torch.equal(grad_res, dy)
    # grad_route_weights is <r, act> of each assignment, gathered to [T, k].
    assert grad_rw.shape == weights.shape and grad_rw.dtype == weights.dtype


def test_opcheck_composed_ops(device):
    x, res, wr, (w13q, w13s), (w2q, w2s), dy, outs = _finish_state(device, seed=8)
    rows = x.shape[0]
    ops = torch.ops.mlops_mi355x
    prep = (x, wr, w13q, torch.empty(0, device=device), 2, "topk_then_softmax", 1, 1, 1.0,
            [rows], "float32", None, [w13s])
    torch.library.opcheck(ops.moe_mi355x_prepare_fwd.default, prep,
                          test_utils=("test_faketensor",))
    (aux, counts, psum, logits, weights, ids, order, offsets, slots, h13) = outs
    fin = (h13, w2q, weights, order, offsets, slots, res, 2, None, None, [w2s])
    torch.library.opcheck(ops.moe_mi355x_finish_fwd.default, fin,
                          test_utils=("test_faketensor",))
    fin_b = (dy, h13, w2q, weights, order, offsets, slots, 2, None, None, [w2s], True)
    torch.library.opcheck(ops.moe_mi355x_finish_bwd.default, fin_b,
                          test_utils=("test_faketensor",))
    prep_b = (torch.zeros((), device=device), torch.zeros_like(psum), torch.zeros_like(weights),
              torch.zeros_like(h13), x, wr, w13q, logits, weights, ids, order, offsets, slots, 2,
              "topk_then_softmax", [rows], None, [w13s], True, True)
    torch.library.opcheck(ops.moe_mi355x_prepare_bwd.default, prep_b,
                          test_utils=("test_faketensor",))


@pytest.mark.parametrize("containers", [True, False])
def test_composed_fp8_current_equals_the_fused_operator(device, containers):
    """The composed form at fp8_current (RowFP8Weight containers, or bf16
    masters quantized per call) equals mi355x.moe.fp8_current bitwise."""
    from mlops_amd import RowFP8Weight

    x, res, wr, w13, w2, dy = _inputs(device, seed=12)
    results = []
    for implementation in ("mi355x.moe.fp8_current", COMPOSED):
        xv = x.clone().requires_grad_(True)
        wrv = wr.clone().requires_grad_(True)
        if containers:
            a = RowFP8Weight.quantize(w13, interleaved=True).detach().requires_grad_(True)
            b = RowFP8Weight.quantize(w2).detach().requires_grad_(True)
            kw = {}
        else:
            a, b = w13.clone().requires_grad_(True), w2.clone().requires_grad_(True)
            kw = dict(compute_precision="fp8_current")
        with use_implementation("moe", implementation):
            out, aux, counts, psum = mlops_amd.moe(xv, res, wrv, a, b, top_k=2,
                                                   routing_mode="softmax_then_topk",
                                                   swiglu_limit=3.0, **kw)
        torch.autograd.backward([out, aux], [dy, torch.ones_like(aux) * 0.1])
        results.append(dict(out=out.detach(), aux=aux.detach(), counts=counts, gx=xv.grad,
                            gr=wrv.grad, g13=a.grad, g2=b.grad))
    _assert_equal(*results)
