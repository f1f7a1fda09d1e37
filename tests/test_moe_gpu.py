"""Layer-level parity of ``mlops_amd.moe`` (block-FP8 on the MI355X provider).

* Against the CPU oracle at the provider's own quantization points
  (``oracle.fp8_moe_forward/backward``): routing, counts and the permutation
  bit-exact given the same fp32 logits; outputs and gradients within 1e-2
  relative Frobenius (bf16 roundings and summation order only).
* Against the reference's native path on the dequantized weights
  (``oracle.native_moe``, fp32 autograd): the reference's own bounds for
  block-FP8 vs bf16 (tests/test_sonicmoe_block_fp8.py:350-368): output 4e-2,
  gradients 8e-2 (relative Frobenius).
* Contracts: explicit forward/backward equal autograd bitwise; repeat runs
  bitwise equal; frozen weights skip their gradients; opcheck of the op pair.
"""

import math

import pytest
import torch

import mlops_amd
from mlops_amd import BlockFP8Weight
from mlops_amd import kernels as K
from mlops_amd.dispatch import capture_dispatch, weight_gradients_at
from oracle import moe_oracle as O
from tests.conftest import frob_rel, max_rel

pytestmark = pytest.mark.gpu


def _inputs(device, tokens=256, hidden=512, experts=8, inter=1024, seed=0, std=0.02):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(tokens, hidden, generator=g).to(torch.bfloat16)
    res = torch.randn(tokens, hidden, generator=g).to(torch.bfloat16)
    wr = torch.randn(experts, hidden, generator=g) / math.sqrt(hidden)
    w13 = (torch.randn(experts, 2 * inter, hidden, generator=g) * std).to(torch.bfloat16)
    w2 = (torch.randn(experts, hidden, inter, generator=g) * std).to(torch.bfloat16)
    dy = torch.randn(tokens, hidden, generator=g).to(torch.bfloat16)
    return [t.to(device) for t in (x, res, wr, w13, w2, dy)]


def _run(x, res, wr, w13, w2, dy, **kw):
    x = x.clone().requires_grad_(True)
    res = res.clone().requires_grad_(True)
    wr = wr.clone().requires_grad_(True)
    w13c = BlockFP8Weight.quantize(w13).detach().requires_grad_(True)
    w2c = BlockFP8Weight.quantize(w2).detach().requires_grad_(True)
    out, aux, counts, psum = mlops_amd.moe(x, res, wr, w13c, w2c, **kw)
    torch.autograd.backward([out, aux], [dy, torch.ones_like(aux) * 0.1])
    assert torch.equal(res.grad, dy)  # d residual is the output cotangent
    return dict(out=out.detach(), aux=aux.detach(), counts=counts, psum=psum.detach(),
                gx=x.grad, gr=wr.grad, g13=w13c.grad, g2=w2c.grad, w13c=w13c, w2c=w2c)


@pytest.mark.parametrize("mode", ["topk_then_softmax", "softmax_then_topk", "sigmoid_noaux_tc"])
def test_layer_matches_fp8_oracle(device, mode):
    x, res, wr, w13, w2, dy = _inputs(device, seed=1)
    top_k = 2
    r = _run(x, res, wr, w13, w2, dy, top_k=top_k, routing_mode=mode)
    w13q, w13s = r["w13c"].components()
    w2q, w2s = r["w2c"].components()
    cpu = lambda t: t.detach().cpu()
    from mlops_amd import router
    logits = router.router_logits(x, wr).cpu()
    fwd = O.fp8_moe_forward(cpu(x), cpu(res), cpu(wr), cpu(w13q), cpu(w13s), cpu(w2q), cpu(w2s),
                            top_k=top_k, routing_mode=mode, logits=logits)
    assert torch.equal(r["counts"].cpu(), fwd["counts"])
    assert frob_rel(r["out"].cpu().float(), fwd["out"].float()) < 1e-2
    assert abs(r["aux"].item() - fwd["aux"].item()) < 1e-4 * max(1, abs(fwd["aux"].item()))
    assert max_rel(r["psum"].cpu(), fwd["prob_sum"]) < 1e-4
    bwd = O.fp8_moe_backward(fwd, cpu(x), cpu(dy), cpu(wr), cpu(w13q), cpu(w13s), cpu(w2q),
                             cpu(w2s), top_k=top_k, routing_mode=mode,
                             grad_aux=torch.tensor(0.1), grad_prob_sum=None)
    assert frob_rel(r["g2"].cpu().float(), bwd["dw2"]) < 1e-2
    assert frob_rel(r["g13"].cpu().float(), bwd["dw13"]) < 1e-2
    assert frob_rel(r["gx"].cpu().float(), bwd["grad_x"].float()) < 1e-2
    assert frob_rel(r["gr"].cpu().float(), bwd["grad_router"]) < 1e-2


def test_layer_matches_native_on_dequantized_weights(device):
    """BASELINE config 1 shapes (T=256, H=512, E=8, k=2, I=1024)."""
    x, res, wr, w13, w2, dy = _inputs(device, seed=2)
    r = _run(x, res, wr, w13, w2, dy, top_k=2, routing_mode="topk_then_softmax")
    w13d = r["w13c"].dequantize().detach().float().cpu().requires_grad_(True)
    w2d = r["w2c"].dequantize().detach().float().cpu().requires_grad_(True)
    xr = x.detach().float().cpu().requires_grad_(True)
    wrr = wr.detach().cpu().requires_grad_(True)
    out, aux, counts, psum = O.native_moe(xr, res.float().cpu(), wrr, w13d, w2d, top_k=2,
                                          routing_mode="topk_then_softmax")
    torch.autograd.backward([out, aux], [dy.float().cpu(), torch.tensor(0.1)])
    assert torch.equal(r["counts"].cpu(), counts)
    assert frob_rel(r["out"].cpu().float(), out.detach()) < 4e-2
    assert frob_rel(r["gx"].cpu().float(), xr.grad) < 8e-2
    assert frob_rel(r["g13"].cpu().float(), w13d.grad) < 8e-2
    assert frob_rel(r["g2"].cpu().float(), w2d.grad) < 8e-2
    assert frob_rel(r["gr"].cpu().float(), wrr.grad) < 8e-2


def test_plain_weights_quantized_per_call_and_dispatch(device):
    x, res, wr, w13, w2, dy = _inputs(device, tokens=64, hidden=256, experts=4, inter=256, seed=3)
    w13p = w13.clone().requires_grad_(True)
    with capture_dispatch() as trace:
        out, *_ = mlops_amd.moe(x, res, wr, w13p, w2, top_k=2, routing_mode="topk_then_softmax",
                                compute_precision="fp8_block")
    assert trace == {"moe": {"mi355x.moe.block_fp8": 1}}
    out.backward(dy)
    assert w13p.grad is not None and w13p.grad.shape == w13.shape
    with pytest.raises(RuntimeError, match="no supported implementation"):
        mlops_amd.moe(x, res, wr, w13, w2, top_k=2, routing_mode="topk_then_softmax")


def test_explicit_surface_equals_autograd_bitwise(device):
    x, res, wr, w13, w2, dy = _inputs(device, tokens=128, hidden=256, experts=8, inter=256, seed=4)
    r = _run(x, res, wr, w13, w2, dy, top_k=2, routing_mode="softmax_then_topk")
    w13c, w2c = r["w13c"].detach(), r["w2c"].detach()
    fwd = mlops_amd.explicit.moe.forward(x, res, wr, w13c, w2c, top_k=2,
                                         routing_mode="softmax_then_topk")
    assert len(fwd) == 11
    assert torch.equal(fwd[0], r["out"])
    (out, aux, counts, psum, logits, weights, ids, order, offsets, slots, h13) = fwd
    grads = mlops_amd.explicit.moe.backward(
        dy, torch.tensor(0.1, device=device), torch.zeros_like(psum), x, wr, w13c, w2c, logits,
        weights, ids, order, offsets, slots, h13, top_k=2, routing_mode="softmax_then_topk",
        lengths=(x.shape[0],))
    gx, gres, gr, g13, g2 = grads
    assert torch.equal(gx, r["gx"]) and torch.equal(gr, r["gr"])
    assert torch.equal(g13, r["g13"]) and torch.equal(g2, r["g2"])
    assert torch.equal(gres, dy)


def test_bitwise_repeatable(device):
    x, res, wr, w13, w2, dy = _inputs(device, tokens=512, hidden=512, experts=16, inter=256, seed=5)
    a = _run(x, res, wr, w13, w2, dy, top_k=4, routing_mode="topk_then_softmax")
    b = _run(x, res, wr, w13, w2, dy, top_k=4, routing_mode="topk_then_softmax")
    for key in ("out", "aux", "psum", "gx", "gr", "g13", "g2"):
        assert torch.equal(a[key], b[key]), key


def test_frozen_weights_skip_gradients(device):
    x, res, wr, w13, w2, dy = _inputs(device, tokens=64, hidden=256, experts=4, inter=256, seed=6)
    xg = x.clone().requires_grad_(True)
    w13c = BlockFP8Weight.quantize(w13)
    w2c = BlockFP8Weight.quantize(w2)
    out, *_ = mlops_amd.moe(xg, res, wr, w13c, w2c, top_k=2, routing_mode="topk_then_softmax")
    out.backward(dy)
    assert xg.grad is not None and w13c.grad is None and w2c.grad is None


def test_weight_gradients_at_fp32(device):
    x, res, wr, w13, w2, dy = _inputs(device, tokens=64, hidden=256, experts=4, inter=256, seed=7)
    with weight_gradients_at(torch.float32):
        r = _run(x, res, wr, w13, w2, dy, top_k=2, routing_mode="topk_then_softmax")
    # the container's logical dtype is bf16: autograd delivers bf16 grads
    assert r["g13"].dtype == torch.bfloat16 and r["g13"].shape == w13.shape


def test_swiglu_limit_and_shared_expert(device):
    x, res, wr, w13, w2, dy = _inputs(device, tokens=128, hidden=256, experts=4, inter=256, seed=8)
    g = torch.Generator().manual_seed(9)
    sw13 = (torch.randn(512, 256, generator=g) * 0.02).to(torch.bfloat16).to(device)
    sw2 = (torch.randn(256, 256, generator=g) * 0.02).to(torch.bfloat16).to(device)
    w13c, w2c = BlockFP8Weight.quantize(w13), BlockFP8Weight.quantize(w2)
    out, *_ = mlops_amd.moe(x, res, wr, w13c, w2c, top_k=2, routing_mode="topk_then_softmax",
                            swiglu_limit=0.01, shared_w13=sw13, shared_w2=sw2)
    xd = x.float().cpu()
    ref, *_ = O.native_moe(xd, res.float().cpu(), wr.cpu(), w13c.dequantize().float().cpu(),
                           w2c.dequantize().float().cpu(), top_k=2,
                           routing_mode="topk_then_softmax", swiglu_limit=0.01)
    sh = xd @ sw13.float().cpu().t()
    gte, up = sh[:, :256].clamp(max=0.01), sh[:, 256:].clamp(-0.01, 0.01)
    ref = ref.float() + (torch.nn.functional.silu(gte) * up) @ sw2.float().cpu().t()
    assert frob_rel(out.float().cpu(), ref) < 4e-2


def test_opcheck_forward_op(device):
    x, res, wr, w13, w2, dy = _inputs(device, tokens=32, hidden=256, experts=4, inter=128, seed=10)
    w13q, w13s = K.quantize_weight_blocks(w13)
    w2q, w2s = K.quantize_weight_blocks(w2)
    op = torch.ops.mlops_mi355x.moe_mi355x_block_fp8_fwd.default
    args = (x, res, wr, w13q, w2q, torch.empty(0, device=device), 2, "topk_then_softmax", 1, 1,
            1.0, [32], "float32", None, None, [w13s, w2s])
    # opcheck's schema test multiplies every tensor input, which torch does not
    # implement for float8; the fake-tensor test runs through opcheck and the
    # schema's no-mutation promise is checked on the input bytes directly.
    torch.library.opcheck(op, args, test_utils=("test_faketensor",))
    tensors = [a for a in args if isinstance(a, torch.Tensor)] + list(args[-1])
    before = [t.clone().view(torch.uint8) if t.numel() else t.clone() for t in tensors]
    outs = op(*args)
    assert len(outs) == 11
    for b, t in zip(before, tensors):
        assert torch.equal(b, t.view(torch.uint8) if t.numel() else t)
    bwd = torch.ops.mlops_mi355x.moe_mi355x_block_fp8_bwd.default
    (out, aux, counts, psum, logits, weights, ids, order, offsets, slots, h13) = outs
    bargs = (dy, torch.zeros((), device=device), torch.zeros_like(psum), x, wr, w13q, w2q, logits,
             weights, ids, order, offsets, slots, h13, 2, "topk_then_softmax", [32], None, None,
             True, True, True, True, [w13s, w2s])
    torch.library.opcheck(bwd, bargs, test_utils=("test_faketensor",))
    # The autograd path asks for no residual copy: an empty placeholder.
    quiet = bargs[:-2] + (False, bargs[-1])
    torch.library.opcheck(bwd, quiet, test_utils=("test_faketensor",))
    full, empty = bwd(*bargs), bwd(*quiet)
    assert torch.equal(full[1], dy) and empty[1].numel() == 0
    for u, v in zip(full[:1] + full[2:], empty[:1] + empty[2:]):
        assert torch.equal(u, v)


def test_qwen3_shape_properties(device):
    """Config 3 shapes (T=16384, H=2048, I=768, E=128, k=8): size-independent
    checks -- plan invariants, finite outputs, sampled rows of the up GEMM
    against fp64, and token sums of the backward."""
    tokens, hidden, inter, experts, top_k = 16384, 2048, 768, 128, 8
    x, res, wr, w13, w2, dy = _inputs(device, tokens, hidden, experts, inter, seed=11)
    w13c, w2c = BlockFP8Weight.quantize(w13), BlockFP8Weight.quantize(w2)
    fwd = mlops_amd.explicit.moe.forward(x, res, wr, w13c, w2c, top_k=top_k,
                                         routing_mode="topk_then_softmax")
    out, aux, counts, psum, logits, weights, ids, order, offsets, slots, h13 = fwd
    assert int(counts.sum()) == tokens * top_k
    assert torch.all(offsets[1:] >= offsets[:-1]) and int(offsets[-1]) == tokens * top_k
    flat = torch.arange(tokens * top_k, device=device, dtype=torch.int32)
    assert torch.equal(slots.reshape(-1)[order.long()], flat)
    sorted_ids = ids.reshape(-1)[order.long()]
    assert torch.all(sorted_ids[1:] >= sorted_ids[:-1])
    assert torch.isfinite(out.float()).all() and torch.isfinite(h13.float()).all()
    # sampled rows of h13 against fp64 of the GPU-quantized operands
    xq, xs = K.permute_quantize(x, slots)
    w13q, w13s = w13c.components()
    sample = torch.linspace(0, tokens * top_k - 1, 64).long()
    a = O.dequantize_rows(xq[sample].cpu(), xs[:, sample].cpu()).double()
    wd = O.dequantize_blocks(w13q.cpu(), w13s.cpu()).double()
    rows_e = torch.searchsorted(offsets.cpu().long(), sample, right=True) - 1
    for i, row in enumerate(sample.tolist()):
        e = int(rows_e[i])
        want = a[i] @ wd[e].t()
        want = torch.stack((want[:inter], want[inter:]), -1).reshape(-1)
        assert max_rel(h13[row].cpu(), want) < 1e-2
    grads = mlops_amd.explicit.moe.backward(
        dy, torch.zeros((), device=device), torch.zeros_like(psum), x, wr, w13c, w2c, logits,
        weights, ids, order, offsets, slots, h13, top_k=top_k, routing_mode="topk_then_softmax",
        lengths=(tokens,))
    for gtensor in grads:
        assert torch.isfinite(gtensor.float()).all()


def test_qwen3_full_shape_sampled_tokens_against_oracle(device):
    """Config 3 at full size (T=16384, H=2048, I=768, E=128, k=8) against the
    fp8 oracle on a subset S of the tokens: the two least-loaded experts'
    tokens plus 64 spread tokens. The GPU runs the whole layer; its backward
    takes the upstream gradient masked to S with zero aux / probability-sum
    cotangents, so every gradient is a sum over S. The oracle then runs on S
    alone, with the GPU's fp32 logits of S (routing is per token): its rows of
    the two experts are exactly the GPU's, in the same order, so their 128-row
    quantization blocks agree, and it gives the GPU's ``out[S]``,
    ``grad_x[S]``, the full router gradient and both experts' weight
    gradients, each within 1e-2 relative Frobenius."""
    tokens, hidden, inter, experts, top_k = 16384, 2048, 768, 128, 8
    x, res, wr, w13, w2, dy = _inputs(device, tokens, hidden, experts, inter, seed=12)
    w13c, w2c = BlockFP8Weight.quantize(w13), BlockFP8Weight.quantize(w2)
    mode = "topk_then_softmax"
    fwd = mlops_amd.explicit.moe.forward(x, res, wr, w13c, w2c, top_k=top_k, routing_mode=mode)
    out, aux, counts, psum, logits, weights, ids, order, offsets, slots, h13 = fwd
    cnt = counts.cpu().clone()
    cnt[cnt == 0] = tokens * top_k
    e1, e2 = (int(e) for e in torch.argsort(cnt, stable=True)[:2])
    ids_c = ids.cpu()
    mask = ((ids_c == e1) | (ids_c == e2)).any(1)
    mask[torch.linspace(0, tokens - 1, 64).long()] = True
    sample = torch.nonzero(mask).squeeze(1)
    dy_masked = dy * mask.to(device)[:, None].to(dy.dtype)
    d_h2, _, d_router, d_w13, d_w2 = mlops_amd.explicit.moe.backward(
        dy_masked, torch.zeros((), device=device), torch.zeros_like(psum), x, wr, w13c, w2c,
        logits, weights, ids, order, offsets, slots, h13, top_k=top_k, routing_mode=mode,
        lengths=(tokens,))

    cpu = lambda t: t.detach().cpu()
    w13q, w13s = (cpu(t) for t in w13c.components())
    w2q, w2s = (cpu(t) for t in w2c.components())
    xs, sl = cpu(x)[sample], cpu(logits)[sample]
    ofwd = O.fp8_moe_forward(xs, cpu(res)[sample], cpu(wr), w13q, w13s, w2q, w2s, top_k=top_k,
                             routing_mode=mode, logits=sl)
    assert torch.equal(ofwd["ids"], ids_c[sample])
    assert frob_rel(cpu(out)[sample].float(), ofwd["out"].float()) < 1e-2
    obwd = O.fp8_moe_backward(ofwd, xs, cpu(dy)[sample], cpu(wr), w13q, w13s, w2q, w2s,
                              top_k=top_k, routing_mode=mode)
    assert frob_rel(cpu(d_h2)[sample].float(), obwd["grad_x"].float()) < 1e-2
    assert frob_rel(cpu(d_router).float(), obwd["grad_router"]) < 1e-2
    for e in (e1, e2):
        assert int(ofwd["counts"][e]) == int(counts[e]) > 0
        assert frob_rel(cpu(d_w2[e]).float(), obwd["dw2"][e]) < 1e-2, e
        assert frob_rel(cpu(d_w13[e]).float(), obwd["dw13"][e]) < 1e-2, e


def test_per_call_transposed_weights_match_containers_bitwise(device, monkeypatch):
    """Weights quantized per call and pre-built containers give the same
    results bit for bit; at widths that are multiples of 256 neither writes a
    transposed copy (the input-gradient GEMMs read the weights as stored)."""
    from mlops_amd import kernels as K

    calls = []
    original = K.transpose_fp8
    monkeypatch.setattr(K, "transpose_fp8", lambda data: calls.append(1) or original(data))
    x, res, wr, w13, w2, dy = _inputs(device, tokens=256, hidden=256, experts=4, inter=256,
                                      seed=9)
    results = []
    for per_call in (True, False):
        xg = x.clone().requires_grad_(True)
        if per_call:
            a, b = w13.clone().requires_grad_(True), w2.clone().requires_grad_(True)
        else:
            a = BlockFP8Weight.quantize(w13).detach().requires_grad_(True)
            b = BlockFP8Weight.quantize(w2).detach().requires_grad_(True)
        calls.clear()
        out, *_ = mlops_amd.moe(xg, res, wr, a, b, top_k=2, routing_mode="topk_then_softmax",
                                compute_precision="fp8_block")
        out.backward(dy)
        assert len(calls) == 0
        results.append((out, xg.grad, a.grad, b.grad))
    for u, v in zip(*results):
        assert torch.equal(u.float(), v.float())


def test_per_call_transposed_copy_follows_the_kmajor_width(device, monkeypatch):
    """The per-call quantizer writes the transposed copy exactly for a weight
    whose last axis (the N of its K-major input-gradient GEMM) is not a
    multiple of 256: w2 [E, H, I] with I = 384 gets it, w13 [E, 2I, H] with
    H = 256 does not; the backward then transposes nothing itself, and the
    results equal those of pre-built containers bit for bit."""
    from mlops_amd import kernels as K

    flags, calls = [], []
    quantize, transpose = K.quantize_weight_blocks, K.transpose_fp8
    monkeypatch.setattr(K, "quantize_weight_blocks",
                        lambda w, transposed=False: flags.append((w.shape[2], transposed))
                        or quantize(w, transposed=transposed))
    monkeypatch.setattr(K, "transpose_fp8", lambda data: calls.append(1) or transpose(data))
    x, res, wr, w13, w2, dy = _inputs(device, tokens=256, hidden=256, experts=4, inter=384,
                                      seed=11)
    results = []
    for per_call in (True, False):
        xg = x.clone().requires_grad_(True)
        if per_call:
            a, b = w13.clone().requires_grad_(True), w2.clone().requires_grad_(True)
        else:
            a = BlockFP8Weight.quantize(w13).detach().requires_grad_(True)
            b = BlockFP8Weight.quantize(w2).detach().requires_grad_(True)
        flags.clear()
        calls.clear()
        out, *_ = mlops_amd.moe(xg, res, wr, a, b, top_k=2, routing_mode="topk_then_softmax",
                                compute_precision="fp8_block")
        out.backward(dy)
        if per_call:
            assert sorted(flags) == [(256, False), (384, True)]
            assert len(calls) == 0
        results.append((out, xg.grad, a.grad, b.grad))
    for u, v in zip(*results):
        assert torch.equal(u.float(), v.float())


def test_forced_zipf_top1_at_c4_width_matches_fp8_oracle(device):
    """The C4 benchmark's own workload form -- top-1 slots whose experts are
    forced from an i.i.d. Zipf(1.2) draw through the routing override, at
    the DeepSeek-V3 shard widths (H=7168, I=2048, 32 experts, weights
    N(0, 0.006)) -- on 384 slots, against the block-FP8 oracle. The oracle
    routes through logits raised by 100 at the forced experts (top-1 under
    topk_then_softmax: the route weight is 1 and carries no logit gradient
    either way). Several experts receive no slot."""
    import numpy as np

    from mlops_amd import router
    from mlops_amd.routing import routing_override

    tokens, hidden, inter, experts = 384, 7168, 2048, 32
    x, res, wr, w13, w2, dy = _inputs(device, tokens, hidden, experts, inter, seed=31, std=0.006)
    p = np.arange(1, experts + 1, dtype=np.float64) ** -1.2
    draw = np.random.default_rng(7).choice(experts, size=(tokens, 1), p=p / p.sum())
    ids = torch.from_numpy(draw.astype(np.int32)).to(device)
    xg = x.clone().requires_grad_(True)
    w13c = BlockFP8Weight.quantize(w13).detach().requires_grad_(True)
    w2c = BlockFP8Weight.quantize(w2).detach().requires_grad_(True)
    with routing_override([ids]):
        out, _aux, counts, _psum = mlops_amd.moe(xg, res, wr, w13c, w2c, top_k=1,
                                                 routing_mode="topk_then_softmax")
    out.backward(dy)
    want_counts = torch.bincount(ids.long().cpu().reshape(-1), minlength=experts)
    assert torch.equal(counts.cpu().long(), want_counts)
    assert int((want_counts == 0).sum()) > 0
    cpu = lambda t: t.detach().cpu()
    w13q, w13s = w13c.components()
    w2q, w2s = w2c.components()
    logits = router.router_logits(x, wr).cpu()
    logits[torch.arange(tokens), ids.long().cpu()[:, 0]] += 100.0
    fwd = O.fp8_moe_forward(cpu(x), cpu(res), cpu(wr), cpu(w13q), cpu(w13s), cpu(w2q), cpu(w2s),
                            top_k=1, routing_mode="topk_then_softmax", logits=logits)
    assert torch.equal(fwd["counts"], want_counts)
    assert frob_rel(cpu(out).float(), fwd["out"].float()) < 1e-2
    bwd = O.fp8_moe_backward(fwd, cpu(x), cpu(dy), cpu(wr), cpu(w13q), cpu(w13s), cpu(w2q),
                             cpu(w2s), top_k=1, routing_mode="topk_then_softmax")
    assert frob_rel(cpu(xg.grad).float(), bwd["grad_x"].float()) < 1e-2
    for e in range(experts):
        if int(want_counts[e]) == 0:
            assert float(w13c.grad[e].abs().max()) == 0.0
            continue
        assert frob_rel(cpu(w13c.grad[e]).float(), bwd["dw13"][e]) < 1e-2, e
        assert frob_rel(cpu(w2c.grad[e]).float(), bwd["dw2"][e]) < 1e-2, e


@pytest.mark.parametrize("shape", [
    # BASELINE config 4 (DeepSeek-V3 shard: H=7168, I=2048, 32 local experts,
    # k=8, Zipf(1.2)-skewed routing, weights N(0, 0.006)) at 512 tokens.
    dict(tokens=512, hidden=7168, inter=2048, experts=32, top_k=8, std=0.006, skew="zipf"),
    # BASELINE config 5 (Mixtral: H=4096, I=14336, E=8, k=2, logits + 2 on
    # expert 0) at 256 tokens.
    dict(tokens=256, hidden=4096, inter=14336, experts=8, top_k=2, std=0.02, skew="expert0"),
], ids=["deepseek_v3_shard", "mixtral_8x7b"])
def test_large_shapes_match_native_on_gpu(device, shape):
    """Layer fwd+bwd at the C4 / C5 widths against the reference's native
    path (oracle.native_moe, fp32, on the GPU) on the dequantized weights."""
    t, h, i, e, k = (shape[n] for n in ("tokens", "hidden", "inter", "experts", "top_k"))
    x, res, wr, w13, w2, dy = _inputs(device, t, h, e, i, seed=21, std=shape["std"])
    # Skewed routing: a constant input column times per-expert router offsets.
    x[:, 0] = 1.0
    if shape["skew"] == "zipf":
        wr[:, 0] = 1.2 * torch.log(1.0 / torch.arange(1, e + 1, device=device, dtype=torch.float32))
    else:
        wr[:, 0] = 0.0
        wr[0, 0] = 2.0
    r = _run(x, res, wr, w13, w2, dy, top_k=k, routing_mode="topk_then_softmax")
    w13d = [w.requires_grad_(True) for w in r["w13c"].dequantize().detach().float()]
    w2d = [w.requires_grad_(True) for w in r["w2c"].dequantize().detach().float()]
    xr = x.detach().float().requires_grad_(True)
    wrr = wr.detach().clone().requires_grad_(True)
    out, aux, counts, psum = O.native_moe(xr, res.float(), wrr, w13d, w2d, top_k=k,
                                          routing_mode="topk_then_softmax")
    torch.autograd.backward([out, aux], [dy.float(), torch.tensor(0.1, device=device)])
    # logits from different GEMM orders may flip a near-tie: allow one route
    assert int((r["counts"] - counts).abs().sum()) <= 2
    assert frob_rel(r["out"].float(), out.detach()) < 4e-2
    assert frob_rel(r["gx"].float(), xr.grad) < 8e-2
    assert frob_rel(r["g13"].float(), torch.stack([w.grad for w in w13d])) < 8e-2
    assert frob_rel(r["g2"].float(), torch.stack([w.grad for w in w2d])) < 8e-2
    assert frob_rel(r["gr"].float(), wrr.grad) < 8e-2


@pytest.mark.parametrize("tokens,experts,top_k", [
    (333, 16, 2),    # an odd token count; half the experts get no rows
    (1, 8, 2),       # one token
    (64, 64, 32),    # the largest top_k
    (96, 512, 4),    # the largest expert count, most experts empty
])
def test_layer_edge_shapes_match_fp8_oracle(device, tokens, experts, top_k):
    """Ragged and empty inputs at the layer: the upper half of the experts
    never wins (a constant hidden feature with a strongly negative router
    weight), so their weight gradients must be exactly zero; everything else
    matches the fp8 oracle as in test_layer_matches_fp8_oracle."""
    x, res, wr, w13, w2, dy = _inputs(device, tokens=tokens, hidden=256, experts=experts,
                                      inter=256, seed=11)
    x[:, 0] = 1.0
    wr[:, 0] = 0.0
    if top_k <= experts // 2:
        wr[experts // 2:, 0] = -30.0
    mode = "softmax_then_topk"
    r = _run(x, res, wr, w13, w2, dy, top_k=top_k, routing_mode=mode)
    w13q, w13s = r["w13c"].components()
    w2q, w2s = r["w2c"].components()
    cpu = lambda t: t.detach().cpu()
    from mlops_amd import router
    logits = router.router_logits(x, wr).cpu()
    fwd = O.fp8_moe_forward(cpu(x), cpu(res), cpu(wr), cpu(w13q), cpu(w13s), cpu(w2q), cpu(w2s),
                            top_k=top_k, routing_mode=mode, logits=logits)
    assert torch.equal(r["counts"].cpu(), fwd["counts"])
    assert frob_rel(r["out"].cpu().float(), fwd["out"].float()) < 1e-2
    bwd = O.fp8_moe_backward(fwd, cpu(x), cpu(dy), cpu(wr), cpu(w13q), cpu(w13s), cpu(w2q),
                             cpu(w2s), top_k=top_k, routing_mode=mode,
                             grad_aux=torch.tensor(0.1), grad_prob_sum=None)
    assert frob_rel(r["gx"].cpu().float(), bwd["grad_x"].float()) < 1e-2
    assert frob_rel(r["gr"].cpu().float(), bwd["grad_router"]) < 1e-2
    used = r["counts"].cpu() > 0
    assert frob_rel(r["g13"].cpu().float()[used], bwd["dw13"][used]) < 1e-2
    assert frob_rel(r["g2"].cpu().float()[used], bwd["dw2"][used]) < 1e-2
    if top_k <= experts // 2:
        assert not bool(used[experts // 2:].any())
        assert bool((r["g13"][~used.to(device)] == 0).all())
        assert bool((r["g2"][~used.to(device)] == 0).all())


def test_protocol_container_equals_block_fp8_weight(device):
    """The same e4m3 blocks in a container class that only carries the
    reference's component protocol (tests/foreign_container.py): every output
    and gradient bitwise equal to BlockFP8Weight's, trained containers
    included (their gradients arrive on the foreign leaves)."""
    from tests.foreign_container import ProtocolBlockWeight

    x, res, wr, w13, w2, dy = _inputs(device, tokens=192, hidden=256, experts=8, inter=256,
                                      seed=41)

    def run(make):
        xl, wrl = x.clone().requires_grad_(True), wr.clone().requires_grad_(True)
        c13 = make(*BlockFP8Weight.quantize(w13).components()).requires_grad_(True)
        c2 = make(*BlockFP8Weight.quantize(w2).components()).requires_grad_(True)
        out, aux, counts, psum = mlops_amd.moe(xl, res, wrl, c13, c2, top_k=2,
                                               routing_mode="softmax_then_topk")
        torch.autograd.backward([out, aux], [dy, torch.ones_like(aux) * 0.1])
        return [out, aux, counts, psum, xl.grad, wrl.grad, c13.grad, c2.grad]

    with capture_dispatch() as trace:
        theirs = run(lambda d, s: ProtocolBlockWeight(d, s, dtype=torch.bfloat16))
    assert trace == {"moe": {"mi355x.moe.block_fp8": 1}}
    ours = run(lambda d, s: BlockFP8Weight(d, s, dtype=torch.bfloat16))
    for a, b in zip(theirs, ours, strict=True):
        assert a is not None and torch.equal(a, b)


@pytest.mark.parametrize("precision", ["fp8_block", "fp8_current"])
def test_gathered_token_rows_equal_permuted_copy_in_the_layer(device, monkeypatch, precision):
    """From top_k 4 the up projection and r = dy @ W2 read the token rows
    quantized once (gathered GEMMs); below, a permuted copy. Forcing either
    path on the same top-4 layer gives bitwise the same outputs and
    gradients (bf16 masters quantized per call)."""
    from mlops_amd.providers.mi355x import moe as fused

    x, res, wr, w13, w2, dy = _inputs(device, tokens=384, hidden=512, experts=8, inter=256,
                                      seed=7)

    calls = []
    for name in ("gemm_gathered", "gemm_rowwise_gathered"):
        original = getattr(K, name)

        def counted(*args, _original=original, **kwargs):
            calls.append(1)
            return _original(*args, **kwargs)

        monkeypatch.setattr(K, name, counted)

    def run(threshold):
        monkeypatch.setattr(fused, "GATHER_MIN_TOP_K", threshold)
        leaves = [t.clone().requires_grad_(True) for t in (x, wr, w13, w2)]
        out, aux, counts, psum = mlops_amd.moe(leaves[0], res, leaves[1], leaves[2], leaves[3],
                                               top_k=4, routing_mode="softmax_then_topk",
                                               compute_precision=precision)
        grads = torch.autograd.grad([out, aux], leaves, [dy, torch.ones_like(aux) * 0.1])
        return [out, aux, counts, psum, *grads]

    gathered = run(4)
    assert len(calls) == 2  # the up projection and r = dy @ W2
    permuted = run(10**9)
    assert len(calls) == 2
    names = ["out", "aux", "counts", "psum", "x", "router", "w13", "w2"]
    for name, a, b in zip(names, gathered, permuted, strict=True):
        assert torch.equal(a, b), name
