"""Expert LoRA (``mlops_amd.lora.expert_lora``) on the MI355X block-FP8 path.

* Against the reference's native form on the dequantized base weights
  (``oracle.native_moe(..., lora=...)``, fp32 autograd on the CPU), with the
  reference's FP8 bounds for expert LoRA (tests/test_sonicmoe_lora.py:336-343:
  8e-2 relative Frobenius), for a frozen FP8 base and for trained masters,
  at aligned and unaligned ranks.
* With zero B factors it is ``mlops_amd.moe`` (tests/test_sonicmoe_lora.py
  :159-193): the forward bitwise, the gradients to summation order.
"""

import math

import pytest
import torch

import mlops_amd
from mlops_amd import BlockFP8Weight, RowFP8Weight
from mlops_amd.lora import expert_lora
from oracle import moe_oracle as O
from tests.conftest import frob_rel

TOKENS, WIDTH, EXPERTS, INTER, TOP_K, SCALE = 256, 512, 8, 256, 2, 0.5
BOUND = 8e-2


def _inputs(device, rank, seed):
    g = torch.Generator().manual_seed(seed)

    def rnd(*shape, s=1.0, dtype=torch.float32):
        return (torch.randn(*shape, generator=g) * s).to(dtype).to(device)

    x, res = rnd(TOKENS, WIDTH, dtype=torch.bfloat16), rnd(TOKENS, WIDTH, dtype=torch.bfloat16)
    wr = rnd(EXPERTS, WIDTH, s=WIDTH ** -0.5)
    w13 = rnd(EXPERTS, 2 * INTER, WIDTH, s=WIDTH ** -0.5, dtype=torch.bfloat16)
    w2 = rnd(EXPERTS, WIDTH, INTER, s=INTER ** -0.5, dtype=torch.bfloat16)
    a13, b13 = rnd(EXPERTS, rank, WIDTH, s=WIDTH ** -0.5), rnd(EXPERTS, 2 * INTER, rank, s=rank ** -0.5)
    a2, b2 = rnd(EXPERTS, rank, INTER, s=INTER ** -0.5), rnd(EXPERTS, WIDTH, rank, s=rank ** -0.5)
    dy = rnd(TOKENS, WIDTH, dtype=torch.bfloat16)
    return x, res, wr, w13, w2, a13, b13, a2, b2, dy


def _leaf(t):
    return t.detach().clone().requires_grad_(True)


def _run_gpu(x, res, wr, w13, w2, a13, b13, a2, b2, dy, *, train_base, mode, limit=None,
             current=False):
    x, wr, res = _leaf(x), _leaf(wr), _leaf(res)
    factors = [_leaf(t) for t in (a13, b13, a2, b2)]
    if train_base:
        w13, w2 = _leaf(w13), _leaf(w2)
        precision = "fp8_current" if current else "fp8_block"
    elif current:
        w13, w2 = RowFP8Weight.quantize(w13, interleaved=True), RowFP8Weight.quantize(w2)
        precision = None
    else:
        w13, w2, precision = BlockFP8Weight.quantize(w13), BlockFP8Weight.quantize(w2), None
    out, aux, counts, psum = expert_lora(
        x, res, wr, w13, w2, *factors, top_k=TOP_K, routing_mode=mode, scale=SCALE,
        swiglu_limit=limit, compute_precision=precision)
    trainable = [x, wr, *factors] + ([w13, w2] if train_base else [])
    *grads, grad_res = torch.autograd.grad((out.float() * dy.float()).sum() + 0.3 * aux,
                                           trainable + [res])
    # The residual passes straight through: its gradient is the output cotangent.
    assert torch.equal(grad_res, dy.to(grad_res.dtype))
    return out.detach(), aux.detach(), counts, psum.detach(), grads


def _dequantized_rows(w):
    data, _, scale, _ = O.quantize_weights_current(w)
    return data.float() * scale[..., None]


def _run_oracle(x, res, wr, w13, w2, a13, b13, a2, b2, dy, *, train_base, mode, limit=None,
                current=False):
    cpu = lambda t: t.detach().cpu()
    # The base as the GPU path's forward sees it: its FP8 values, dequantized
    # (per 128x128 block, or per row for fp8_current).
    if current:
        w13d, w2d = _dequantized_rows(cpu(w13).float()), _dequantized_rows(cpu(w2).float())
    else:
        w13d = O.dequantize_blocks(*O.quantize_blocks(cpu(w13).float()))
        w2d = O.dequantize_blocks(*O.quantize_blocks(cpu(w2).float()))
    xl, wrl = _leaf(cpu(x)), _leaf(cpu(wr))
    w13l, w2l = _leaf(w13d), _leaf(w2d)
    factors = [_leaf(cpu(t)) for t in (a13, b13, a2, b2)]
    out, aux, counts, psum = O.native_moe(xl, cpu(res), wrl, w13l, w2l, top_k=TOP_K,
                                          routing_mode=mode, swiglu_limit=limit,
                                          lora=(*factors, SCALE))
    trainable = [xl, wrl, *factors] + ([w13l, w2l] if train_base else [])
    grads = torch.autograd.grad((out.float() * cpu(dy).float()).sum() + 0.3 * aux, trainable)
    return out.detach(), aux.detach(), counts, psum.detach(), grads


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["topk_then_softmax", "softmax_then_topk", "sigmoid_noaux_tc"])
@pytest.mark.parametrize("rank,train_base", [(16, False), (7, True), (1, False), (80, False)])
def test_expert_lora_matches_native_on_dequantized_weights(device, mode, rank, train_base):
    case = _inputs(device, rank, seed=rank)
    out, aux, counts, psum, grads = _run_gpu(*case, train_base=train_base, mode=mode)
    r_out, r_aux, r_counts, r_psum, r_grads = _run_oracle(*case, train_base=train_base, mode=mode)
    assert torch.equal(counts.cpu(), r_counts)
    assert frob_rel(out.cpu().float(), r_out.float()) < 4e-2
    assert abs(aux.item() - r_aux.item()) < 1e-4 * max(1.0, abs(r_aux.item()))
    assert frob_rel(psum.cpu(), r_psum) < 1e-4
    names = ["x", "router", "a13", "b13", "a2", "b2"] + (["w13", "w2"] if train_base else [])
    for name, g, r in zip(names, grads, r_grads, strict=True):
        assert g.shape == r.shape, name
        err = frob_rel(g.cpu().float(), r.float())
        assert err < BOUND, f"{name}: relative error {err:.3e}"
    # Factor gradients come back at the factors' dtype, base ones at bf16.
    assert all(g.dtype == torch.float32 for g in grads[2:6])
    if train_base:
        assert grads[6].dtype == grads[7].dtype == torch.bfloat16


@pytest.mark.gpu
@pytest.mark.parametrize("rank,train_base", [(16, False), (7, True)])
def test_expert_lora_on_an_fp8_current_base(device, rank, train_base):
    """A per-row FP8 base (RowFP8Weight containers, or masters quantized per
    call at fp8_current), as the reference's SonicMoE LoRA serves it: against
    the native form on the dequantized rows at the same bounds."""
    case = _inputs(device, rank, seed=30 + rank)
    kw = dict(train_base=train_base, mode="softmax_then_topk", current=True)
    out, aux, counts, psum, grads = _run_gpu(*case, **kw)
    r_out, r_aux, r_counts, r_psum, r_grads = _run_oracle(*case, **kw)
    assert torch.equal(counts.cpu(), r_counts)
    assert frob_rel(out.cpu().float(), r_out.float()) < 4e-2
    names = ["x", "router", "a13", "b13", "a2", "b2"] + (["w13", "w2"] if train_base else [])
    for name, g, r in zip(names, grads, r_grads, strict=True):
        assert g.shape == r.shape, name
        err = frob_rel(g.cpu().float(), r.float())
        assert err < BOUND, f"{name}: relative error {err:.3e}"


@pytest.mark.gpu
def test_zero_b_factors_are_mlops_moe_at_fp8_current(device):
    x, res, wr, w13, w2, a13, b13, a2, b2, dy = _inputs(device, 16, seed=6)
    b13, b2 = torch.zeros_like(b13), torch.zeros_like(b2)
    w13c, w2c = RowFP8Weight.quantize(w13, interleaved=True), RowFP8Weight.quantize(w2)
    options = dict(top_k=TOP_K, routing_mode="softmax_then_topk", swiglu_limit=2.75)

    def run(lora):
        xl, wrl = _leaf(x), _leaf(wr)
        if lora:
            outs = expert_lora(xl, res, wrl, w13c, w2c, a13, b13, a2, b2, scale=SCALE, **options)
        else:
            outs = mlops_amd.moe(xl, res, wrl, w13c, w2c, **options)
        grads = torch.autograd.grad((outs[0].float() * dy.float()).sum() + 0.3 * outs[1],
                                    [xl, wrl])
        return [o.detach() for o in outs], grads

    (outs, grads), (ref_outs, ref_grads) = run(True), run(False)
    for a, b in zip(outs, ref_outs, strict=True):
        assert torch.equal(a, b)
    for a, b in zip(grads, ref_grads, strict=True):
        assert frob_rel(a.float(), b.float()) < 1e-3


@pytest.mark.gpu
def test_the_limit_reaches_the_lora_path(device):
    """As tests/test_sonicmoe_lora.py:377-403 checks its FP8 base: FP8 moves
    pre-activations by a few percent, enough to cross a limit inside the bulk
    of them and move a gradient by whole elements, so parity with the native
    form is taken at a limit far out (4.0, still clipping a few), and a tight
    limit (0.75) must change the output and the hidden rows' gradient."""
    case = _inputs(device, 16, seed=21)
    got = _run_gpu(*case, train_base=False, mode="softmax_then_topk", limit=4.0)
    ref = _run_oracle(*case, train_base=False, mode="softmax_then_topk", limit=4.0)
    assert frob_rel(got[0].cpu().float(), ref[0].float()) < 4e-2
    for g, r in zip(got[4], ref[4], strict=True):
        assert frob_rel(g.cpu().float(), r.float()) < BOUND
    clamped = _run_gpu(*case, train_base=False, mode="softmax_then_topk", limit=0.75)
    plain = _run_gpu(*case, train_base=False, mode="softmax_then_topk")
    assert frob_rel(clamped[0].float(), plain[0].float()) > 5e-2
    assert frob_rel(clamped[4][0].float(), plain[4][0].float()) > 5e-2


@pytest.mark.gpu
def test_zero_b_factors_are_mlops_moe(device):
    x, res, wr, w13, w2, a13, b13, a2, b2, dy = _inputs(device, 16, seed=5)
    b13, b2 = torch.zeros_like(b13), torch.zeros_like(b2)
    w13c, w2c = BlockFP8Weight.quantize(w13), BlockFP8Weight.quantize(w2)
    options = dict(top_k=TOP_K, routing_mode="sigmoid_noaux_tc", n_group=2, topk_group=1,
                   routed_scaling=1.5, lengths=(96, 160), swiglu_limit=2.75)

    def run(lora):
        xl, wrl = _leaf(x), _leaf(wr)
        if lora:
            outs = expert_lora(xl, res, wrl, w13c, w2c, a13, b13, a2, b2, scale=SCALE, **options)
        else:
            outs = mlops_amd.moe(xl, res, wrl, w13c, w2c, **options)
        grads = torch.autograd.grad((outs[0].float() * dy.float()).sum() + 0.3 * outs[1],
                                    [xl, wrl])
        return [o.detach() for o in outs], grads

    (outs, grads), (ref_outs, ref_grads) = run(True), run(False)
    for a, b in zip(outs, ref_outs, strict=True):
        assert torch.equal(a, b)
    for a, b in zip(grads, ref_grads, strict=True):
        assert frob_rel(a.float(), b.float()) < 1e-3


def test_unknown_implementations_are_refused():
    t = torch.zeros(1)
    with pytest.raises(ValueError, match="unknown expert LoRA implementation"):
        expert_lora(t, t, t, t, t, t, t, t, t, top_k=1, routing_mode="softmax_then_topk",
                    scale=1.0, implementation="sonicmoe")
    with pytest.raises(ValueError, match="swiglu_limit must be positive"):
        expert_lora(t, t, t, t, t, t, t, t, t, top_k=1, routing_mode="softmax_then_topk",
                    scale=1.0, swiglu_limit=0.0)


def test_cpu_tensors_are_refused_with_the_reason():
    x = torch.zeros(4, 128, dtype=torch.bfloat16)
    wr = torch.zeros(2, 128)
    w13, w2 = torch.zeros(2, 256, 128), torch.zeros(2, 128, 128)
    a, b = torch.zeros(2, 4, 128), torch.zeros(2, 256, 4)
    with pytest.raises(ValueError, match="does not apply here"):
        expert_lora(x, x, wr, w13, w2, a, b, torch.zeros(2, 4, 128), torch.zeros(2, 128, 4),
                    top_k=1, routing_mode="softmax_then_topk", scale=1.0,
                    compute_precision="fp8_block")


@pytest.mark.gpu
def test_expert_lora_at_mixtral_widths(device):
    """C5's widths (H = 4096, I = 14336, E = 8, top-2, rank 16) on a frozen
    block-FP8 base, with C5's factor scales (A ~ N(0, 0.01), B = 0.1 N(0, 1),
    bf16) and its +2 logit on expert 0, at 128 tokens so the CPU oracle
    finishes: every output and gradient against the native form on the
    dequantized base at the reference's FP8 bounds
    (tests/test_sonicmoe_lora.py:336-343). K = 4096 and 14336 take the LoRA
    accumulator-start GEMMs and the routed rank products through their long-K
    loops."""
    tokens, width, experts, inter, top_k, rank, scale = 128, 4096, 8, 14336, 2, 16, 2.0
    g = torch.Generator().manual_seed(55)
    x = torch.randn(tokens, width, generator=g).to(torch.bfloat16)
    res = torch.randn(tokens, width, generator=g).to(torch.bfloat16)
    wr = torch.randn(experts, width, generator=g) / math.sqrt(width)
    x[:, 0], wr[:, 0], wr[0, 0] = 1.0, 0.0, 2.0  # logits + 2 on expert 0
    factors = [(torch.randn(*shape, generator=g) * std).to(torch.bfloat16)
               for shape, std in (((experts, rank, width), 0.01), ((experts, 2 * inter, rank), 0.1),
                                  ((experts, rank, inter), 0.01), ((experts, width, rank), 0.1))]
    dy = torch.randn(tokens, width, generator=g).to(torch.bfloat16)
    gd = torch.Generator(device=device).manual_seed(56)  # 1.4G weight values: drawn on the GPU
    w13 = (torch.randn(experts, 2 * inter, width, generator=gd, device=device) * 0.02).bfloat16()
    w2 = (torch.randn(experts, width, inter, generator=gd, device=device) * 0.02).bfloat16()
    mode = "topk_then_softmax"

    # GPU: frozen containers, gradients for x, the router and the factors.
    xg, wrg = _leaf(x.to(device)), _leaf(wr.to(device))
    fg = [_leaf(f.to(device)) for f in factors]
    w13c, w2c = BlockFP8Weight.quantize(w13), BlockFP8Weight.quantize(w2)
    del w13, w2
    out, aux, counts, psum = expert_lora(xg, res.to(device), wrg, w13c, w2c, *fg, top_k=top_k,
                                         routing_mode=mode, scale=scale)
    grads = torch.autograd.grad((out.float() * dy.to(device).float()).sum() + 0.3 * aux,
                                [xg, wrg, *fg])
    grads = [t.cpu() for t in grads]
    out, counts = out.detach().cpu(), counts.cpu()
    assert int(counts[0]) == int(counts.max()) > tokens // 2  # the +2 logit on expert 0

    # Oracle on the CPU, on the base the GPU forward multiplies: the
    # containers' e4m3 blocks (bit-exact to the oracle's block quantizer,
    # tested elsewhere) dequantized, as per-expert frozen tensors.
    comps = [c.components() for c in (w13c, w2c)]
    w13d, w2d = ([O.dequantize_blocks(d[e:e + 1].cpu(), s[e:e + 1].cpu())[0]
                  for e in range(experts)] for d, s in comps)
    del w13c, w2c, comps
    xl, wrl = _leaf(x), _leaf(wr)
    fl = [_leaf(f.float()) for f in factors]
    r_out, r_aux, r_counts, _ = O.native_moe(xl, res, wrl, w13d, w2d, top_k=top_k,
                                             routing_mode=mode, lora=(*fl, scale))
    r_grads = torch.autograd.grad((r_out.float() * dy.float()).sum() + 0.3 * r_aux, [xl, wrl, *fl])
    assert torch.equal(counts, r_counts)
    assert frob_rel(out.float(), r_out.detach().float()) < 4e-2
    for name, a, b in zip(["x", "router", "a13", "b13", "a2", "b2"], grads, r_grads, strict=True):
        assert a.shape == b.shape, name
        err = frob_rel(a.float(), b.float())
        assert err < BOUND, f"{name}: relative error {err:.3e}"


@pytest.mark.gpu
@pytest.mark.filterwarnings("ignore:Synchronization debug mode")
@pytest.mark.parametrize("precision", ["fp8_block", "fp8_current"])
def test_no_host_synchronization(device, precision):
    """The reference's provider contract (docs/PROVIDERS.md:64-69): no
    device-to-host synchronization in forward or backward. torch's sync debug
    mode turns any synchronizing call (``.item()``, ``.tolist()``, ``nonzero``,
    a blocking copy) into an error; expert LoRA and ``mlops_amd.moe`` run
    forward and backward under it."""
    x, res, wr, w13, w2, a13, b13, a2, b2, dy = _inputs(device, 16, seed=8)
    factors = [_leaf(t) for t in (a13, b13, a2, b2)]
    if precision == "fp8_current":
        w13c, w2c = RowFP8Weight.quantize(w13, interleaved=True), RowFP8Weight.quantize(w2)
    else:
        w13c, w2c = BlockFP8Weight.quantize(w13), BlockFP8Weight.quantize(w2)
    torch.cuda.synchronize(device)
    previous = torch.cuda.get_sync_debug_mode()
    torch.cuda.set_sync_debug_mode("error")
    try:
        with pytest.raises(RuntimeError):  # the mode is live: .item() is refused
            torch.ones(1, device=device).sum().item()
        xl, wrl = _leaf(x), _leaf(wr)
        out, aux, _, _ = expert_lora(xl, res, wrl, w13c, w2c, *factors, top_k=TOP_K,
                                     routing_mode="softmax_then_topk", scale=SCALE)
        torch.autograd.backward([out, aux], [dy, torch.ones_like(aux)])
        xm, wrm = _leaf(x), _leaf(wr)
        out, aux, _, _ = mlops_amd.moe(xm, res, wrm, w13c, w2c, top_k=TOP_K,
                                       routing_mode="softmax_then_topk")
        torch.autograd.backward([out, aux], [dy, torch.ones_like(aux)])
    finally:
        torch.cuda.set_sync_debug_mode(previous)
    assert all(f.grad is not None for f in factors) and xm.grad is not None
