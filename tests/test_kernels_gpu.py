"""Kernel-level parity of the HIP entry points against the CPU oracle.

Bar: bit-exact for routing ids, the permutation (order / offsets / slots /
counts), every e4m3 byte and fp32 scale of the quantizers; GEMMs within
1e-2 worst-relative (per expert) of the fp64 product of the same
dequantized operands (the reference's own bound,
tests/test_block_fp8_transpose_gemm.py:486-531); fp32 router math within
1e-5 relative.
"""

import numpy as np
import pytest
import torch

from mlops_amd import kernels as K
from oracle import moe_oracle as O
from tests.conftest import frob_rel, max_rel, worst_cell_rel

pytestmark = pytest.mark.gpu


def _bytes(t):
    return t.detach().cpu().view(torch.uint8)


def _zipf_ids(tokens, top_k, experts, s, seed):
    rng = np.random.default_rng(seed)
    p = 1.0 / np.arange(1, experts + 1) ** s
    p /= p.sum()
    ids = np.stack([rng.choice(experts, size=top_k, replace=False, p=p) for _ in range(tokens)])
    return torch.from_numpy(ids.astype(np.int32))


# ------------------------------------------------------------------ router
@pytest.mark.parametrize("mode", ["topk_then_softmax", "softmax_then_topk", "sigmoid_noaux_tc"])
@pytest.mark.parametrize("experts,top_k", [(128, 8), (8, 2), (300, 6), (256, 8), (512, 32), (64, 1),
                                            (128, 16), (128, 17), (16, 16), (100, 3)])
def test_router_topk_matches_oracle(device, mode, experts, top_k):
    g = torch.Generator().manual_seed(experts + top_k)
    logits = torch.randn(1000, experts, generator=g)
    logits[3] = 0.0          # all tied
    logits[4, 1] = logits[4, experts - 1] = 4.0  # tie at the top
    w, ids = K.router_topk(logits.to(device), top_k, mode, routed_scaling=1.3)
    ow, oids = O.route(logits, top_k, mode, routed_scaling=1.3)
    assert torch.equal(ids.cpu(), oids)
    assert max_rel(w.cpu(), ow) < 1e-5


@pytest.mark.parametrize("mode", ["topk_then_softmax", "sigmoid_noaux_tc"])
@pytest.mark.parametrize("experts,top_k", [(128, 8), (300, 6)])
def test_router_topk_nan_and_signed_zero(device, mode, experts, top_k):
    """torch.sort's order on the awkward values: NaN ahead of every number,
    -0 equal to +0 (ties to the lower id), -inf last among numbers."""
    g = torch.Generator().manual_seed(5)
    logits = torch.randn(64, experts, generator=g)
    logits[0, 7] = float("nan")
    logits[1, [3, 9]] = float("nan")
    logits[2] = float("-inf")
    logits[2, 11] = 0.5
    logits[3] = 0.0
    logits[3, ::2] = -0.0
    logits[4, : experts - 2] = float("-inf")
    _, ids = K.router_topk(logits.to(device), top_k, mode)
    _, oids = O.route(logits, top_k, mode)
    assert torch.equal(ids.cpu(), oids)


def test_router_topk_group_limited(device):
    g = torch.Generator().manual_seed(11)
    logits = torch.randn(777, 64, generator=g)
    bias = torch.randn(64, generator=g) * 0.05
    w, ids = K.router_topk(logits.to(device), 6, "sigmoid_noaux_tc", bias=bias.to(device),
                           n_group=8, topk_group=3, routed_scaling=2.5)
    ow, oids = O.route(logits, 6, "sigmoid_noaux_tc", bias=bias, n_group=8, topk_group=3,
                       routed_scaling=2.5)
    assert torch.equal(ids.cpu(), oids)
    assert max_rel(w.cpu(), ow) < 1e-5


def test_router_forced_ids(device):
    g = torch.Generator().manual_seed(12)
    logits = torch.randn(50, 16, generator=g)
    forced = torch.stack([torch.randperm(16, generator=g)[:4] for _ in range(50)]).int()
    for mode in ("topk_then_softmax", "softmax_then_topk", "sigmoid_noaux_tc"):
        w, ids = K.router_topk(logits.to(device), 4, mode, forced_ids=forced.to(device))
        ow, oids = O.route(logits, 4, mode, forced_ids=forced)
        assert torch.equal(ids.cpu(), forced)
        assert max_rel(w.cpu(), ow) < 1e-5


@pytest.mark.parametrize("mode,lengths,experts,top_k", [
    ("topk_then_softmax", None, 32, 4),
    ("softmax_then_topk", None, 32, 4),
    ("topk_then_softmax", (300, 200), 32, 4),         # softmax aux over all segments
    ("sigmoid_noaux_tc", (100, 37, 363), 32, 4),
    ("softmax_then_topk", (77, 250, 173), 512, 8),   # 8 logits per lane, odd segments
    ("sigmoid_noaux_tc", (201, 299), 512, 6),
    ("topk_then_softmax", None, 64, 32),               # top_k near the lane limit
    ("sigmoid_noaux_tc", (13, 487), 64, 32),
    ("topk_then_softmax", None, 128, 8),               # two expert slots per lane
    ("softmax_then_topk", (250, 250), 200, 8),         # four slots per lane, masked tail
    ("sigmoid_noaux_tc", None, 256, 8),
])
def test_router_stats_and_backward(device, mode, lengths, experts, top_k):
    g = torch.Generator().manual_seed(13 + experts + top_k)
    tokens = 500
    lengths = (tokens,) if lengths is None else lengths
    logits = torch.randn(tokens, experts, generator=g)
    w, ids = O.route(logits, top_k, mode)
    aux, psum, seg_counts, seg_offsets = K.router_stats(logits.to(device), ids.to(device), top_k,
                                                        mode, lengths)
    oaux, ocounts, opsum = O.routing_statistics(logits, ids, mode, lengths, experts)
    assert abs(aux.item() - oaux.item()) <= 1e-5 * max(1.0, abs(oaux.item()))
    assert max_rel(psum.cpu(), opsum) < 1e-5
    assert torch.equal(seg_counts.cpu().sum(0).long(), ocounts)
    # backward: route-weight cotangent arrives as per-sorted-row dscore
    order, offsets, slots = O.sort_assignments(ids, experts)
    dscore = torch.randn(tokens * top_k, generator=g)
    gw = dscore[slots.reshape(-1).long()].view(tokens, top_k)
    ga = torch.tensor(0.3)
    gps = torch.randn(experts, generator=g)
    grad = K.router_backward(logits.to(device), w.to(device), ids.to(device), dscore.to(device),
                             slots.to(device), mode, grad_aux=ga.to(device),
                             grad_prob_sum=gps.to(device), offsets=offsets.to(device),
                             seg_offsets=seg_offsets, seg_counts=seg_counts)
    want = O.routing_gradient(ga, gps, gw, w, ids, logits, mode, lengths)
    assert max_rel(grad.cpu(), want) < 1e-5
    # the split form: [hi | mid] bf16 pieces of the same fp32 gradient, as
    # torch's casts make them
    pieces = K.router_backward(logits.to(device), w.to(device), ids.to(device),
                               dscore.to(device), slots.to(device), mode, grad_aux=ga.to(device),
                               grad_prob_sum=gps.to(device), offsets=offsets.to(device),
                               seg_offsets=seg_offsets, seg_counts=seg_counts, pieces=True).cpu()
    hi = grad.cpu().to(torch.bfloat16)
    assert torch.equal(pieces[:, :experts], hi)
    assert torch.equal(pieces[:, experts:], (grad.cpu() - hi.float()).to(torch.bfloat16))


@pytest.mark.parametrize("tokens,experts,hidden", [
    (16384, 128, 2048),   # C3's router
    (1000, 32, 256),      # ragged last step
    (37, 8, 512),         # one step, most expert rows masked
    (700, 200, 768),      # E not a multiple of the 128-row tile
    (513, 256, 256),      # two expert tiles
    (0, 16, 256),         # no tokens: zeros
])
def test_router_weight_grad_matches_fp64(device, tokens, experts, hidden):
    """dW = hi^T x + mid^T x (bf16 pieces, fp32 sums) against fp64 on the same
    bf16 operands, and equal to the pieces' fp32 cotangent within the bf16
    split's resolution."""
    g = torch.Generator().manual_seed(tokens + experts)
    grad = torch.randn(tokens, experts, generator=g) * 1e-3
    hi = grad.to(torch.bfloat16)
    mid = (grad - hi.float()).to(torch.bfloat16)
    pieces = torch.cat([hi, mid], 1)
    x = torch.randn(tokens, hidden, generator=g).to(torch.bfloat16)
    got = K.router_weight_grad(pieces.to(device), x.to(device)).cpu()
    want = hi.double().t() @ x.double() + mid.double().t() @ x.double()
    assert got.dtype == torch.float32 and got.shape == (experts, hidden)
    if tokens == 0:
        assert torch.count_nonzero(got) == 0
        return
    assert (got.double() - want).abs().max() <= 1e-5 * want.abs().max()
    # the split carries the fp32 cotangent to ~2^-16 relative
    exact = grad.double().t() @ x.double()
    assert (got.double() - exact).abs().max() <= 1e-4 * exact.abs().max()


# ------------------------------------------------------------------ permute
@pytest.mark.parametrize("tokens,top_k,experts,kind", [
    (16384, 8, 128, "uniform"),      # Qwen3-30B-A3B routing shape
    (4096, 8, 32, "zipf"),           # skewed, some experts empty
    (1, 3, 4, "uniform"),
    (777, 2, 1, "uniform"),          # one expert
    (5000, 1, 512, "uniform"),       # max experts
])
def test_permute_plan_bit_exact(device, tokens, top_k, experts, kind):
    if kind == "zipf":
        ids = _zipf_ids(tokens, top_k, experts, 1.2, seed=tokens)
    else:
        g = torch.Generator().manual_seed(tokens + experts)
        if top_k <= experts:
            ids = torch.stack([torch.randperm(experts, generator=g)[:top_k] for _ in range(tokens)]).int() \
                if tokens < 5000 else torch.randint(0, experts, (tokens, top_k), generator=g).int()
        else:
            ids = torch.randint(0, experts, (tokens, top_k), generator=g).int()
    counts, offsets, order, slots = K.permute_plan(ids.to(device), experts)
    oorder, ooffsets, oslots = O.sort_assignments(ids, experts)
    assert torch.equal(order.cpu(), oorder)
    assert torch.equal(offsets.cpu(), ooffsets)
    assert torch.equal(slots.cpu(), oslots)
    assert torch.equal(counts.cpu(), torch.bincount(ids.reshape(-1).long(), minlength=experts))


def test_permute_quantize_bit_exact(device):
    g = torch.Generator().manual_seed(14)
    tokens, width, top_k, experts = 700, 1024, 4, 16
    x = (torch.randn(tokens, width, generator=g) * 2).to(torch.bfloat16)
    x[7, :128] = 0  # zero group
    x[8, 5] = 300.0  # outlier
    ids = torch.stack([torch.randperm(experts, generator=g)[:top_k] for _ in range(tokens)]).int()
    order, offsets, slots = O.sort_assignments(ids, experts)
    q, s = K.permute_quantize(x.to(device), slots.to(device))
    oq, os_ = O.quantize_rows_1x128(x[order.long() // top_k])
    assert torch.equal(_bytes(q), oq.view(torch.uint8))
    assert torch.equal(s.cpu(), os_)


@pytest.mark.parametrize("gate_up", [False, True])
def test_quantize_rows_bit_exact(device, gate_up):
    g = torch.Generator().manual_seed(15)
    x = (torch.randn(333, 1536, generator=g) * 0.1).to(torch.bfloat16)
    q, s = K.quantize_rows(x.to(device), gate_up=gate_up)
    src = x[:, O.gate_up_columns(1536)] if gate_up else x
    oq, os_ = O.quantize_rows_1x128(src)
    assert torch.equal(_bytes(q), oq.view(torch.uint8))
    assert torch.equal(s.cpu(), os_)


@pytest.mark.parametrize("limit", [None, 0.5])
def test_swiglu_quantize(device, limit):
    g = torch.Generator().manual_seed(16)
    h = torch.randn(257, 2 * 768, generator=g).to(torch.bfloat16)
    q, s = K.swiglu_quantize(h.to(device), limit)
    act = O.swiglu(h, limit)
    oq, os_ = O.quantize_rows_1x128(act)
    # exp() differs in the last ulp between libraries: scales agree to 1e-6,
    # bytes agree except where a value sits on a rounding boundary.
    assert max_rel(s.cpu(), os_) < 1e-6
    same = (_bytes(q) == oq.view(torch.uint8)).float().mean().item()
    assert same > 0.999
    assert max_rel(O.dequantize_rows(q.cpu(), s.cpu()), O.dequantize_rows(oq, os_)) < 0.07


@pytest.mark.parametrize("shape,dtype", [((4, 256, 384), torch.bfloat16),
                                         ((3, 208, 144), torch.float32)])
def test_quantize_weight_blocks_bit_exact(device, shape, dtype):
    g = torch.Generator().manual_seed(17)
    w = (torch.randn(*shape, generator=g) * 0.02).to(dtype)
    w[0, :128, :128] = 0
    w[1, 0, 0] = 2.0 ** 14 * 0.02
    data, scale, data_t = K.quantize_weight_blocks(w.to(device), transposed=True)
    od, os_ = O.quantize_blocks(w)
    assert torch.equal(_bytes(data), od.view(torch.uint8))
    assert torch.equal(scale.cpu(), os_)
    assert torch.equal(_bytes(data_t), od.transpose(1, 2).contiguous().view(torch.uint8))
    assert torch.equal(_bytes(K.transpose_fp8(data)), _bytes(data_t))


@pytest.mark.parametrize("gather,gate_up", [(False, False), (True, False), (False, True)])
def test_quantize_transpose_bit_exact(device, gather, gate_up):
    g = torch.Generator().manual_seed(18)
    experts, top_k, tokens, width = 6, 2, 400, 512
    ids = torch.stack([torch.randperm(experts, generator=g)[:top_k] for _ in range(tokens)]).int()
    ids[ids == 4] = 5  # expert 4 empty
    order, offsets, slots = O.sort_assignments(ids, experts)
    if gather:
        src = torch.randn(tokens, width, generator=g).to(torch.bfloat16)
        rows = src[order.long() // top_k]
        qt, st, padded = K.quantize_transpose(src.to(device), offsets.to(device), tokens * top_k,
                                              gather=order.to(device), gather_div=top_k)
    else:
        rows = torch.randn(tokens * top_k, width, generator=g).to(torch.bfloat16)
        src = rows
        qt, st, padded = K.quantize_transpose(rows.to(device), offsets.to(device), tokens * top_k,
                                              gate_up=gate_up)
    if gate_up:
        rows = rows[:, O.gate_up_columns(width)]
    oq, os_, total = O.quantize_transpose_padded(rows, offsets, padded)
    assert torch.equal(_bytes(qt)[:, :total], oq.view(torch.uint8)[:, :total])
    assert torch.equal(st.cpu()[: total // 128], os_[: total // 128])


# ------------------------------------------------------------------- GEMMs
def _ragged(counts):
    offs = [0]
    for c in counts:
        offs.append(offs[-1] + c)
    return torch.tensor(offs, dtype=torch.int32)


def _block_factors(g, shape, exponents):
    """A power of two per 128x128 block of a ``[E, R, C]`` weight, 2**e with e
    uniform over ``exponents``, and one all-zero block (the last expert's
    last block row, first block column), as the reference's block-weight
    helper builds them (tests/test_block_fp8_transpose_gemm.py:431-444)."""
    experts, r, c = shape
    lo, hi = exponents
    blocks = (experts, -(-r // 128), -(-c // 128))
    e = torch.randint(lo, hi + 1, blocks, generator=g).double()
    f = torch.exp2(e).float()
    if f.numel() > 1:
        f[-1, -1, 0] = 0.0
    return f.repeat_interleave(128, 1).repeat_interleave(128, 2)[:, :r, :c]


def _gemm_case(device, counts, n, k, *, seed, transposed=False, interleave=False,
               exponents=(-3, 3), addend=False, lora_rank=0):
    g = torch.Generator().manual_seed(seed)
    experts = len(counts)
    offsets = _ragged(counts)
    rows = int(offsets[-1])
    x = torch.randn(rows, k, generator=g).to(torch.bfloat16)
    wshape = (experts, k, n) if transposed else (experts, n, k)
    # Block scales a few powers of two apart (or 2^-14..2^14), so every
    # block's scale shows in every output cell.
    w = torch.randn(*wshape, generator=g) * 0.02 * _block_factors(g, wshape, exponents)
    xq, xs = K.quantize_rows(x.to(device))
    if transposed:
        wd, ws, wt = K.quantize_weight_blocks(w.to(device), transposed=True)
        wq_kernel = wt
    else:
        wd, ws = K.quantize_weight_blocks(w.to(device))
        wq_kernel = wd
    c = torch.randn(rows, n, generator=g).to(torch.bfloat16) if addend else None
    lora = None
    if lora_rank:
        zz = (torch.randn(rows, lora_rank, generator=g) * 0.5).to(torch.bfloat16)
        bb = (torch.randn(experts, n, lora_rank, generator=g) * 0.1).to(torch.bfloat16)
        lora = (zz.to(device), bb.to(device))
    out = K.gemm(xq, xs, wq_kernel, ws, offsets.to(device), transposed_scale=transposed,
                 interleave=interleave, addend=None if c is None else c.to(device), lora=lora)
    want = O.grouped_gemm(xq.cpu(), xs.cpu(), wd.cpu(), ws.cpu(), offsets, transposed=transposed,
                          interleave=interleave)
    if c is not None:
        want = want + c.double()
    if lora_rank:
        # The rank term in weight-row order (gate rows, then up rows), then
        # in the output's column order.
        term = torch.zeros(rows, n, dtype=torch.float64)
        for e in range(experts):
            lo, hi = int(offsets[e]), int(offsets[e + 1])
            term[lo:hi] = zz[lo:hi].double() @ bb[e].double().t()
        if interleave:
            term = term.view(rows, 2, n // 2).transpose(1, 2).reshape(rows, n)
        want = want + term
    return out.cpu(), want, offsets


COUNTS = [0, 70, 131, 15, 260]  # an empty expert, partial row tiles (reference COUNTS)


@pytest.mark.parametrize("case", [
    dict(counts=COUNTS, n=256, k=512),                                  # block scales 2^-3..2^3
    dict(counts=COUNTS, n=384, k=1024, exponents=(-14, 14)),            # extreme scales, zero block
    dict(counts=COUNTS, n=256, k=1024, exponents=(-14, 14), transposed=True),
    dict(counts=COUNTS, n=512, k=1024, exponents=(-14, 14), interleave=True),
    dict(counts=[129, 64, 257], n=256, k=384, interleave=True),         # gate/up interleaved output
    dict(counts=[100, 200, 0, 33], n=256, k=512, transposed=True),      # input-gradient orientation
    dict(counts=[90, 190], n=128, k=256, addend=True),                  # LoRA-style addend
    dict(counts=COUNTS, n=256, k=512, lora_rank=16),                    # rank term, empty expert
    dict(counts=[129, 64, 257], n=512, k=384, interleave=True, lora_rank=32),  # gate/up order
    dict(counts=[100, 200, 0, 33], n=256, k=512, transposed=True, lora_rank=16),  # input gradient
])
def test_grouped_gemm_matches_fp64(device, case):
    """Worst relative Frobenius error over (expert, 128-column) cells < 1e-2,
    the reference's GEMM metric (tests/test_block_fp8_transpose_gemm.py:
    390-406), so a block 2^28 times smaller than its neighbours is still
    checked at its own magnitude."""
    out, want, offsets = _gemm_case(device, seed=sum(case["counts"]) + case["k"], **case)
    assert torch.isfinite(out).all()
    assert worst_cell_rel(out, want, offsets.tolist()) < 1e-2


@pytest.mark.parametrize("tokens,top_k,experts,k,n,form", [
    (2000, 4, 16, 512, 512, "up"),           # gate/up interleave, partial row tiles
    (1000, 3, 8, 128, 256, "plain"),         # one K step: the next tile's rows at once
    (777, 2, 5, 1024, 768, "kmajor"),        # input gradient through a K-major weight
    (16384, 8, 128, 2048, 1536, "up"),       # C3's up projection
    (16384, 8, 128, 2048, 768, "kmajor"),    # C3's input gradient through W2
    (600, 16, 64, 256, 512, "up"),           # top-16: slot order / 16 in the kernel
])
def test_grouped_gemm_gathered_matches_permuted_copy(device, tokens, top_k, experts, k, n, form):
    """Token rows quantized once and read through the routed rows' tokens
    (a_rows = order // top_k) give the same bytes as the routed-row GEMM on
    the permuted copy; the per-token quantization equals the permuted one."""
    g = torch.Generator().manual_seed(tokens + k + n)
    logits = torch.randn(tokens, experts, generator=g)
    logits[:, 1] -= 30.0  # expert 1 empty
    x = torch.randn(tokens, k, generator=g).to(torch.bfloat16).to(device)
    _, ids = K.router_topk(logits.to(device), top_k, "topk_then_softmax")
    _, offsets, order, slots = K.permute_plan(ids, experts)
    a_rows = (order // top_k).to(torch.int32)
    xq, xs = K.permute_quantize(x, slots)
    tq, ts = K.quantize_token_rows(x)
    assert torch.equal(_bytes(tq[a_rows.long()]), _bytes(xq))
    assert torch.equal(ts[a_rows.long()].t().cpu(), xs.cpu())
    w = (torch.randn(experts, n, k, generator=g) * 0.02).to(torch.bfloat16).to(device)
    if form == "kmajor":
        wk = w.transpose(1, 2).contiguous()              # [E, K, N] as stored
        wq, ws = K.quantize_weight_blocks(wk)
        want = K.gemm_kmajor(xq, xs, wq, ws, offsets)
        got = K.gemm_gathered(tq, ts, a_rows, wq, ws, offsets, kmajor=True)
        # The plan's slot order itself, divided by top_k in the kernel.
        got_slots = K.gemm_gathered(tq, ts, order, wq, ws, offsets, kmajor=True, rows_div=top_k)
    else:
        wq, ws = K.quantize_weight_blocks(w)
        inter = form == "up"
        want = K.gemm(xq, xs, wq, ws, offsets, interleave=inter)
        got = K.gemm_gathered(tq, ts, a_rows, wq, ws, offsets, interleave=inter)
        got_slots = K.gemm_gathered(tq, ts, order, wq, ws, offsets, interleave=inter,
                                    rows_div=top_k)
    assert torch.equal(got.cpu(), want.cpu())
    assert torch.equal(got_slots.cpu(), want.cpu())


@pytest.mark.parametrize("form", ["up", "kmajor"])
def test_grouped_gemm_gathered_matches_fp64(device, form):
    """The gathered GEMMs on the C3 hot path (the interleaved up projection
    and r = dy @ W2 through the K-major weight) checked directly against the
    fp64 product of the dequantized operands, under the reference's metric
    (worst relative Frobenius error over (expert, 128-column) cells < 1e-2,
    tests/test_block_fp8_transpose_gemm.py:390-406): weight block scales
    2^-14..2^14 with an all-zero block, an empty expert, partial row blocks,
    and one token row scaled by 2^12 (its 1x128 scales ~4096 times its
    neighbours', read token-major through each of its routed rows)."""
    tokens, top_k, experts = 700, 4, 6
    k, n = (512, 768) if form == "up" else (1024, 512)
    g = torch.Generator().manual_seed(41 + k)
    logits = torch.randn(tokens, experts, generator=g)
    logits[:, 2] -= 30.0  # expert 2 empty
    x = torch.randn(tokens, k, generator=g)
    x[17] *= 2.0 ** 12
    x = x.to(torch.bfloat16).to(device)
    _, ids = K.router_topk(logits.to(device), top_k, "topk_then_softmax")
    _, offsets, order, _ = K.permute_plan(ids, experts)
    a_rows = (order // top_k).to(torch.int32)
    tq, ts = K.quantize_token_rows(x)
    wshape = (experts, k, n) if form == "kmajor" else (experts, n, k)
    w = torch.randn(*wshape, generator=g) * 0.02 * _block_factors(g, wshape, (-14, 14))
    wq, ws = K.quantize_weight_blocks(w.to(device))
    got = K.gemm_gathered(tq, ts, a_rows, wq, ws, offsets, interleave=form == "up",
                          kmajor=form == "kmajor").cpu()
    rows = a_rows.long().cpu()
    xq, xs = tq.cpu()[rows], ts.cpu()[rows].t().contiguous()
    want = O.grouped_gemm(xq, xs, wq.cpu(), ws.cpu(), offsets.cpu(),
                          transposed=form == "kmajor", interleave=form == "up")
    bounds = offsets.cpu().tolist()
    assert bounds[3] == bounds[2]  # the empty expert
    assert torch.isfinite(got).all()
    assert worst_cell_rel(got, want, bounds) < 1e-2


@pytest.mark.parametrize("tokens,top_k,experts,k,n", [
    (1500, 4, 16, 512, 512),
    (16384, 8, 128, 2048, 1536),             # C3's up projection at fp8_current
])
def test_rowwise_gemm_gathered_matches_permuted_copy(device, tokens, top_k, experts, k, n):
    """The row-scaled GEMM on token rows read through the routed rows equals
    the one on the permuted copy bit for bit (per-row descales in the epilogue
    taken from the tokens)."""
    g = torch.Generator().manual_seed(tokens + n)
    logits = torch.randn(tokens, experts, generator=g)
    logits[:, 2] -= 30.0
    x = torch.randn(tokens, k, generator=g).to(torch.bfloat16).to(device)
    _, ids = K.router_topk(logits.to(device), top_k, "topk_then_softmax")
    _, offsets, order, slots = K.permute_plan(ids, experts)
    a_rows = (order // top_k).to(torch.int32)
    xq, xs = K.permute_quantize_current(x, slots)
    tq, ts = K.quantize_rows_current(x)
    assert torch.equal(_bytes(tq[a_rows.long()]), _bytes(xq))
    assert torch.equal(ts[a_rows.long()].cpu(), xs.cpu())
    w = (torch.randn(experts, n, k, generator=g) * 0.02).to(torch.bfloat16).to(device)
    wq, _, wsc, _ = K.quantize_weights_current(w)
    want = K.gemm_rowwise(xq, xs, wq, wsc, offsets)
    got = K.gemm_rowwise_gathered(tq, ts, a_rows, wq, wsc, offsets)
    assert torch.equal(got.cpu(), want.cpu())
    got_slots = K.gemm_rowwise_gathered(tq, ts, order, wq, wsc, offsets, rows_div=top_k)
    assert torch.equal(got_slots.cpu(), want.cpu())


@pytest.mark.parametrize("counts,k,n", [
    (COUNTS, 512, 256),                      # empty expert, partial row tiles
    ([300, 0, 520, 45], 1536, 2048),         # C3's input gradient through W13 (K = 2I)
    ([129, 64, 257], 2048, 768),             # C3's input gradient through W2 (N = I)
    ([40, 700], 14336, 4096),                # Mixtral's K, the large-weight tile order
])
def test_grouped_gemm_kmajor_matches_transposed_copy(device, counts, k, n):
    """The input-gradient GEMM on the weight as stored ([E, K, N], fragments
    through ds_read_b64_tr_b8) is bitwise the GEMM on its transposed copy
    (same products, same MFMA K grouping), including extreme block scales and
    a zero block."""
    g = torch.Generator().manual_seed(k + n + sum(counts))
    offsets = _ragged(counts)
    rows, experts = int(offsets[-1]), len(counts)
    x = torch.randn(rows, k, generator=g).to(torch.bfloat16).to(device)
    w = (torch.randn(experts, k, n, generator=g) * 0.02)
    w[0, :128, :128] *= 2.0 ** 12
    w[-1, 128:256, :128] = 0.0
    xq, xs = K.quantize_rows(x)
    wq, ws, wt = K.quantize_weight_blocks(w.to(device), transposed=True)
    off = offsets.to(device)
    want = K.gemm(xq, xs, wt, ws, off, transposed_scale=True)
    got = K.gemm_kmajor(xq, xs, wq, ws, off)
    assert torch.equal(got, want)


def test_grouped_gemm_baseline_config2_row_blocks(device):
    """The BASELINE single-GEMM config (E=8, K=4096, N=2048, M_e ~ U{256..4096}
    step 128) under the reference's per-cell metric: each expert's first and
    last full 256-row blocks (every output column of them) against fp64,
    worst relative Frobenius error over (block, 128-column) cells < 1e-2."""
    rng = np.random.default_rng(2)
    counts = (rng.integers(2, 33, size=8) * 128).tolist()
    g = torch.Generator().manual_seed(3)
    offsets = _ragged(counts)
    rows = int(offsets[-1])
    x = torch.randn(rows, 4096, generator=g).to(torch.bfloat16).to(device)
    w = (torch.randn(8, 2048, 4096, generator=g) * 0.02).to(device)
    xq, xs = K.quantize_rows(x)
    wq, ws = K.quantize_weight_blocks(w)
    out = K.gemm(xq, xs, wq, ws, offsets.to(device)).cpu()
    a = O.dequantize_rows(xq.cpu(), xs.cpu()).double()
    wd = O.dequantize_blocks(wq.cpu(), ws.cpu()).double()
    worst = 0.0
    for e in range(8):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        for start in sorted({lo, hi - 256}):
            sel = slice(start, start + 256)
            want = a[sel] @ wd[e].t()
            worst = max(worst, worst_cell_rel(out[sel], want, [0, 256]))
    assert worst < 1e-2


@pytest.mark.parametrize("interleave", [False, True])
def test_grouped_gemm_large_weight_tile_order(device, interleave):
    """Experts whose weight is 24 MB or more (N x K e4m3 bytes) run in the
    grouped tile order: 8 N tiles x all the expert's row blocks, unrotated.
    N = 6400 gives groups of 8, 8, 8 and 1 N tiles; an empty expert and
    partial row blocks are included. Every output element is checked
    against the dequantized oracle operands multiplied in fp32."""
    counts, n, k = [300, 0, 520, 45], 6400, 4096
    assert n * k >= 24 << 20
    g = torch.Generator().manual_seed(17)
    offsets = _ragged(counts)
    rows = int(offsets[-1])
    x = torch.randn(rows, k, generator=g).to(torch.bfloat16).to(device)
    w = (torch.randn(len(counts), n, k, generator=g) * 0.02).to(torch.bfloat16).to(device)
    xq, xs = K.quantize_rows(x)
    wq, ws = K.quantize_weight_blocks(w)
    out = K.gemm(xq, xs, wq, ws, offsets.to(device), interleave=interleave)
    a = O.dequantize_rows(xq.cpu(), xs.cpu()).float().to(device)
    for e, count in enumerate(counts):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        if hi == lo:
            continue
        wd = O.dequantize_blocks(wq[e:e + 1].cpu(), ws[e:e + 1].cpu())[0].float().to(device)
        want = a[lo:hi] @ wd.t()
        if interleave:  # output columns 2j, 2j + 1 = gate j, up j
            want = want.view(hi - lo, 2, n // 2).transpose(1, 2).reshape(hi - lo, n)
        assert max_rel(out[lo:hi].float(), want) < 1e-2, e
        assert worst_cell_rel(out[lo:hi], want, [0, hi - lo]) < 1e-2, e


def test_rowwise_gemm_large_weight_tile_order(device):
    """The row-scaled kernel in the grouped tile order (same shape rule)."""
    counts, n, k = [0, 260, 700], 6400, 4096
    g = torch.Generator().manual_seed(19)
    offsets = _ragged(counts)
    rows = int(offsets[-1])
    x = torch.randn(rows, k, generator=g).to(torch.bfloat16).to(device)
    w = (torch.randn(len(counts), n, k, generator=g) * 0.02).to(torch.bfloat16).to(device)
    xq, xs = K.quantize_rows_current(x)
    wq, _, wsc, _ = K.quantize_weights_current(w)
    out = K.gemm_rowwise(xq, xs, wq, wsc, offsets.to(device))
    a = xq.float() * xs[:, None]
    for e, count in enumerate(counts):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        if hi == lo:
            continue
        want = a[lo:hi] @ (wq[e].float() * wsc[e][:, None]).t()
        assert max_rel(out[lo:hi].float(), want) < 1e-2, e


# (256, 384): general kernel; (512, 768): the pipelined hardware-scaled one.
@pytest.mark.parametrize("features", [(256, 384), (512, 768)])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_wgrad_matches_fp64(device, out_dtype, features):
    g = torch.Generator().manual_seed(19)
    counts = [0, 300, 50, 129]
    offsets = _ragged(counts)
    rows = int(offsets[-1])
    p_rows = torch.randn(rows, features[0], generator=g).to(torch.bfloat16)
    q_rows = torch.randn(rows, features[1], generator=g).to(torch.bfloat16)
    p_rows[7] *= 1e4  # spread the per-block scales over many binades
    q_rows[:, 5] *= 1e-5
    pt, pts, padded = K.quantize_transpose(p_rows.to(device), offsets.to(device), rows)
    qt, qts, _ = K.quantize_transpose(q_rows.to(device), offsets.to(device), rows, padded=padded)
    out = K.wgrad(pt, pts, qt, qts, offsets.to(device), out_dtype=out_dtype).cpu()
    want = O.wgrad(pt.cpu(), pts.cpu(), qt.cpu(), qts.cpu(), offsets)
    assert torch.all(out[0] == 0)
    tol = 1e-4 if out_dtype == torch.float32 else 1e-2  # fp32 accumulation order
    for e in range(1, 4):
        assert max_rel(out[e], want[e]) < tol, e
        # per (128-row, 128-column) cell, as the reference measures GEMMs
        assert worst_cell_rel(out[e], want[e], list(range(0, features[0] + 1, 128))) < tol, e


def test_combine_and_token_sum(device):
    g = torch.Generator().manual_seed(20)
    tokens, top_k, width, experts = 300, 3, 768, 8
    ids = torch.stack([torch.randperm(experts, generator=g)[:top_k] for _ in range(tokens)]).int()
    order, offsets, slots = O.sort_assignments(ids, experts)
    y = torch.randn(tokens * top_k, width, generator=g).to(torch.bfloat16)
    w = torch.rand(tokens, top_k, generator=g)
    res = torch.randn(tokens, width, generator=g).to(torch.bfloat16)
    out = K.combine(y.to(device), slots.to(device), w.to(device), res.to(device)).cpu()
    want = O.combine(y, slots, w, res)
    # one fp32 sum rounded once; summation order may move the last bf16 bit
    assert max_rel(out.float(), want.float()) < 1e-2
    assert (out == want).float().mean().item() > 0.99
    s = K.unpermute_sum(y.to(device), slots.to(device)).cpu()
    assert (s == O.unpermute_sum(y, slots)).float().mean().item() > 0.99


@pytest.mark.parametrize("limit", [None, 0.7])
def test_routed_swiglu_backward(device, limit):
    g = torch.Generator().manual_seed(21)
    rows, width, tokens, top_k = 256, 384, 128, 2
    r = torch.randn(rows, width, generator=g).to(torch.bfloat16)
    h = torch.randn(rows, 2 * width, generator=g).to(torch.bfloat16)
    weights = torch.rand(tokens, top_k, generator=g)
    order = torch.randperm(rows, generator=g).int()
    dh, ap, ds = K.routed_swiglu_backward(r.to(device), h.to(device), weights.reshape(-1).to(device),
                                          order.to(device), limit)
    score = weights.reshape(-1)[order.long()]
    ods, odh, oap = O.routed_swiglu_backward(r, h, score, limit)
    assert max_rel(ds.cpu(), ods) < 1e-4
    assert max_rel(dh.cpu().float(), odh) < 1e-2
    assert max_rel(ap.cpu().float(), oap) < 1e-2


@pytest.mark.parametrize("limit", [None, 0.7])
@pytest.mark.parametrize("rows,width", [(256, 384), (37, 1152), (1, 128)])
def test_routed_swiglu_backward_rows_matches_unfused(device, limit, rows, width):
    """The routed backward with dh row-quantized in the same pass writes the
    plain kernel's dh, a' and dscore, and the row quantizer's bytes and scales
    on that dh (widths past one 1024-column chunk, ragged row counts)."""
    g = torch.Generator().manual_seed(rows + width)
    r = torch.randn(rows, width, generator=g).to(torch.bfloat16).to(device)
    h = torch.randn(rows, 2 * width, generator=g).to(torch.bfloat16).to(device)
    h[0] *= 40.0
    weights = torch.rand(rows, generator=g).to(device)
    order = torch.randperm(rows, generator=g).int().to(device)
    dh, ap, ds, dhq, dhs = K.routed_swiglu_backward_rows(r, h, weights, order, limit)
    dh_ref, ap_ref, ds_ref = K.routed_swiglu_backward(r, h, weights, order, limit)
    q_ref, s_ref = K.quantize_rows(dh_ref, gate_up=True)
    assert torch.equal(dh, dh_ref) and torch.equal(ap, ap_ref) and torch.equal(ds, ds_ref)
    assert torch.equal(_bytes(dhq), _bytes(q_ref))
    assert torch.equal(dhs, s_ref)


@pytest.mark.parametrize("limit", [None, 0.7])
def test_swiglu_bwd_quantize_matches_unfused(device, limit):
    """The fused kernel's outputs are, byte for byte, the unfused kernels'
    (routed SwiGLU backward -> bf16 dh / a' -> row and transposing quantizers),
    which the tests above pin to the oracle. dscore too: both kernels sum the
    score dot in the same order (per 128-column block, blocks in order)."""
    g = torch.Generator().manual_seed(33)
    experts, top_k, tokens, width = 6, 2, 700, 384
    ids = torch.stack([torch.randperm(experts, generator=g)[:top_k] for _ in range(tokens)]).int()
    ids[ids == 3] = 4  # an empty expert
    order, offsets, slots = O.sort_assignments(ids, experts)
    rows = tokens * top_k
    r = torch.randn(rows, width, generator=g).to(torch.bfloat16).to(device)
    h = torch.randn(rows, 2 * width, generator=g).to(torch.bfloat16).to(device)
    h[5] *= 50.0  # a row past the clamp limit
    weights = torch.rand(tokens * top_k, generator=g).to(device)
    order_d, offsets_d = order.to(device), offsets.to(device)
    dhq, dhs, dht, dhts, apt, apts, ds, padded = K.swiglu_bwd_quantize(
        r, h, weights, order_d, offsets_d, limit=limit)
    dh, ap, ds_ref = K.routed_swiglu_backward(r, h, weights, order_d, limit)
    q_ref, s_ref = K.quantize_rows(dh, gate_up=True)
    assert torch.equal(_bytes(dhq), _bytes(q_ref))
    assert torch.equal(dhs, s_ref)
    t_ref, ts_ref, _ = K.quantize_transpose(dh, offsets_d, rows, gate_up=True, padded=padded)
    a_ref, as_ref, _ = K.quantize_transpose(ap, offsets_d, rows, padded=padded)
    total = O.padded_layout(offsets)[1]
    assert torch.equal(_bytes(dht)[:, :total], _bytes(t_ref)[:, :total])
    assert torch.equal(dhts[: total // 128], ts_ref[: total // 128])
    assert torch.equal(_bytes(apt)[:, :total], _bytes(a_ref)[:, :total])
    assert torch.equal(apts[: total // 128], as_ref[: total // 128])
    assert torch.equal(ds, ds_ref)
    # Transposed outputs skipped: the row outputs are unchanged.
    dhq2, dhs2, dht2, _, apt2, _, _, _ = K.swiglu_bwd_quantize(
        r, h, weights, order_d, offsets_d, limit=limit, transposed_dh=False, transposed_ap=False)
    assert dht2 is None and apt2 is None
    assert torch.equal(_bytes(dhq2), _bytes(dhq)) and torch.equal(dhs2, dhs)
    # The bf16 form (fp8_current's backward): dh exactly as the routed SwiGLU
    # backward writes it (h's interleaved order), the same transposed
    # operands and dscore.
    blocks = K.padded_row_blocks(offsets_d, padded)
    dh3, dht3, dhts3, apt3, apts3, ds3 = K.swiglu_bwd_bf16(
        r, h, weights, order_d, offsets_d, padded=padded, row_blocks=blocks, limit=limit)
    assert torch.equal(dh3, dh)
    assert torch.equal(_bytes(dht3)[:, :total], _bytes(t_ref)[:, :total])
    assert torch.equal(dhts3[: total // 128], ts_ref[: total // 128])
    assert torch.equal(_bytes(apt3)[:, :total], _bytes(a_ref)[:, :total])
    assert torch.equal(apts3[: total // 128], as_ref[: total // 128])
    assert torch.equal(ds3, ds_ref)


def test_padded_row_blocks_table(device):
    """(first row, valid rows) of every padded 128-row block, from the oracle's
    padded layout; zeros past the last expert's blocks."""
    counts = [0, 300, 128, 1, 0, 257]
    offsets = _ragged(counts)
    starts, total = O.padded_layout(offsets)
    padded = total + 3 * 128
    blocks = K.padded_row_blocks(offsets.to(device), padded).cpu()
    want = torch.zeros(padded // 128, 2, dtype=torch.int32)
    for e, start in enumerate(starts):
        n = counts[e]
        for j in range(-(-n // 128)):
            want[start // 128 + j] = torch.tensor([int(offsets[e]) + 128 * j, min(128, n - 128 * j)])
    assert torch.equal(blocks, want)


@pytest.mark.parametrize("limit", [None, 0.9])
@pytest.mark.parametrize("inter", [256, 384])  # 2I = 512: pipelined epilogue; 768: GEMM then SwiGLU pass
def test_gemm_swiglu_fused_matches_separate_pass(device, limit, inter):
    """The up projection's fused SwiGLU output equals swiglu_quantize of its
    own h bit for bit; h equals the plain gate/up GEMM's."""
    g = torch.Generator().manual_seed(41)
    counts = [300, 0, 77, 512, 129]
    offsets = _ragged(counts)
    rows, hidden = int(offsets[-1]), 256
    x = torch.randn(rows, hidden, generator=g).to(torch.bfloat16).to(device)
    w = (torch.randn(len(counts), 2 * inter, hidden, generator=g) * 0.3).to(device)
    xq, xs = K.quantize_rows(x)
    wq, ws = K.quantize_weight_blocks(w)
    h, act, act_s = K.gemm_swiglu(xq, xs, wq, ws, offsets.to(device), limit=limit)
    h_ref = K.gemm(xq, xs, wq, ws, offsets.to(device), interleave=True)
    assert torch.equal(h, h_ref)
    q_ref, s_ref = K.swiglu_quantize(h, limit)
    assert torch.equal(_bytes(act), _bytes(q_ref))
    assert torch.equal(act_s, s_ref)


@pytest.mark.parametrize("counts,k,rank", [
    ([0, 37, 5, 0, 150, 16], 512, 16),   # empty experts, blocks spanning boundaries
    ([300, 1, 200], 1536, 32),
    ([64], 96, 48),                      # K % 128 != 0: the register-operand form
    ([64, 129, 0, 31], 384, 48),         # the LDS-staged form at each rank
    ([1000, 0, 33, 700], 1024, 64),
    ([257, 0, 40, 511, 3, 0, 90, 200], 4096, 16),   # C5's K (hidden) at its rank
    ([130, 0, 17, 250], 14336, 16),                  # C5's K (intermediate)
])
def test_rank_product_matches_fp32(device, counts, k, rank):
    g = torch.Generator().manual_seed(sum(counts) + k)
    offsets = _ragged(counts)
    rows, experts = int(offsets[-1]), len(counts)
    a = torch.randn(rows, k, generator=g).to(torch.bfloat16)
    bt = (torch.randn(experts, rank, k, generator=g) * 0.05).to(torch.bfloat16)
    out = K.rank_product(a.to(device), bt.to(device), offsets.to(device)).cpu()
    want = torch.zeros(rows, rank)
    for e in range(experts):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        want[lo:hi] = a[lo:hi].float() @ bt[e].float().t()
    # fp32 sums of exact bf16 products, one bf16 rounding of the result
    assert max_rel(out.float(), want) < 1e-2
    assert frob_rel(out.float(), want) < 4e-3


def test_rank_grad_row_weight_without_gather(device):
    """Routed rows of big (no gather) with small scaled by weight[order[j]]:
    dA2 = sum_j (score_j u2_j) a_j^T, against fp64 on the same operands."""
    g = torch.Generator().manual_seed(5)
    tokens, top_k, experts, m, rank = 250, 2, 5, 392, 16
    ids = torch.stack([torch.randperm(experts, generator=g)[:top_k] for _ in range(tokens)]).int()
    order, offsets, _ = O.sort_assignments(ids, experts)
    rows = tokens * top_k
    big = torch.randn(rows, m, generator=g).to(torch.bfloat16)
    small = (torch.randn(rows, rank, generator=g) * 0.3).to(torch.bfloat16)
    weight = torch.rand(rows, generator=g)
    out = K.rank_grad(big.to(device), small.to(device), offsets.to(device), transposed=True,
                      weight=weight.to(device), weight_index=order.to(device)).cpu()
    scaled = (small.float() * weight[order.long()][:, None]).to(torch.bfloat16)
    for e in range(experts):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        want = (big[lo:hi].double().t() @ scaled[lo:hi].double()).t()
        assert (out[e].double() - want).abs().max() <= 1e-5 * want.abs().max() + 1e-6, e


@pytest.mark.parametrize("splits", [1, 3, 7])
def test_rank_product_k_splits(device, splits):
    """K split over several blocks (fp32 partials added in split order, uneven
    chunk ranges) against fp32, and each split count repeatable bit for bit."""
    g = torch.Generator().manual_seed(90 + splits)
    offsets = _ragged([300, 0, 77, 650])
    rows, experts, k, rank = int(offsets[-1]), 4, 1152, 32
    a = torch.randn(rows, k, generator=g).to(torch.bfloat16)
    bt = (torch.randn(experts, rank, k, generator=g) * 0.05).to(torch.bfloat16)
    args = (a.to(device), bt.to(device), offsets.to(device))
    out = K.rank_product(*args, splits=splits).cpu()
    want = torch.zeros(rows, rank)
    for e in range(experts):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        want[lo:hi] = a[lo:hi].float() @ bt[e].float().t()
    assert max_rel(out.float(), want) < 1e-2
    assert frob_rel(out.float(), want) < 4e-3
    assert torch.equal(out, K.rank_product(*args, splits=splits).cpu())


@pytest.mark.parametrize("counts,m,rank,transposed,chunk", [
    ([0, 37, 5, 0, 150, 16], 512, 16, False, None),     # empty experts, short experts
    ([700, 1, 1300], 1544, 32, True, 256),              # several chunks per expert, M % 2048
    ([300, 0, 900], 3072, 48, False, 128),              # three rank passes, chunk tails
    ([2048, 1024, 4096, 0, 512, 100, 90, 80], 14336, 16, True, None),  # C5-like widths
])
def test_rank_grad_matches_fp64(device, counts, m, rank, transposed, chunk):
    """``sum_j big[j]^T small[j]`` per expert (the LoRA factor gradients)
    against an fp64 product of the same bf16 operands."""
    g = torch.Generator().manual_seed(sum(counts) + m + rank)
    offsets = _ragged(counts)
    rows = int(offsets[-1])
    big = torch.randn(rows, m, generator=g).to(torch.bfloat16)
    small = (torch.randn(rows, rank, generator=g) * 0.3).to(torch.bfloat16)
    out = K.rank_grad(big.to(device), small.to(device), offsets.to(device),
                      transposed=transposed, chunk=chunk).cpu()
    for e in range(len(counts)):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        want = big[lo:hi].double().t() @ small[lo:hi].double()
        if transposed:
            want = want.t()
        got = out[e].double()
        if hi == lo:
            assert torch.all(got == 0)
            continue
        # fp32 sums of exact bf16 products
        assert (got - want).abs().max() <= 1e-5 * want.abs().max() + 1e-6, e
    again = K.rank_grad(big.to(device), small.to(device), offsets.to(device),
                        transposed=transposed, chunk=chunk).cpu()
    assert torch.equal(out, again)  # fixed summation order


@pytest.mark.parametrize("weighted", [False, True])
@pytest.mark.parametrize("transposed", [False, True])
def test_rank_grad_gathered_token_rows(device, weighted, transposed):
    """The token-side form: row j of big is the token row big[order[j] // k],
    and small's row j is scaled by weight[order[j]] * alpha (rounded to bf16
    once), against an fp64 product of the same operands. An empty expert and
    ragged counts come from the routing."""
    g = torch.Generator().manual_seed(7 + 2 * weighted + transposed)
    tokens, top_k, experts, m, rank = 300, 2, 6, 264, 16
    ids = torch.stack([torch.randperm(experts, generator=g)[:top_k] for _ in range(tokens)]).int()
    ids[ids == 2] = 3  # expert 2 gets no rows
    order, offsets, _ = O.sort_assignments(ids, experts)
    rows = tokens * top_k
    big = torch.randn(tokens, m, generator=g).to(torch.bfloat16)
    small = (torch.randn(rows, rank, generator=g) * 0.3).to(torch.bfloat16)
    weight = torch.rand(rows, generator=g) if weighted else None
    alpha = 1.5 if weighted else 1.0
    out = K.rank_grad(big.to(device), small.to(device), offsets.to(device),
                      transposed=transposed, gather=order.to(device), gather_div=top_k,
                      weight=None if weight is None else weight.to(device),
                      weight_index=order.to(device), alpha=alpha).cpu()
    tok = order.long() // top_k
    scaled = small
    if weighted:
        scaled = (small.float() * (weight[order.long()] * alpha)[:, None]).to(torch.bfloat16)
    for e in range(experts):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        want = big[tok[lo:hi]].double().t() @ scaled[lo:hi].double()
        if transposed:
            want = want.t()
        got = out[e].double()
        if hi == lo:
            assert torch.all(got == 0)
            continue
        assert (got - want).abs().max() <= 1e-5 * want.abs().max() + 1e-6, e
