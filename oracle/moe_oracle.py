"""CPU restatement of the reference MoE path -- TEST INFRASTRUCTURE ONLY.

Every function cites the reference lines it restates (paths relative to
``src/mlops`` of als244/mlops). The checks that pin each one are listed in
``PINNED`` and implemented in ``tests/test_oracle.py``.

Conventions shared with the HIP kernels:
* routed rows ``A = T * k`` in expert-sorted order (``order``);
* 1x128 activation scales stored ``[K/128, rows]``;
* weight scales ``[E, ceil(out/128), ceil(in/128)]``;
* ``h13`` interleaved: column ``2j`` = gate ``j``, ``2j+1`` = up ``j``.
"""

from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

FP8 = torch.float8_e4m3fn
E4M3_MAX = 448.0
INV448 = float(np.float32(1.0) / np.float32(448.0))  # fp32-rounded reciprocal

# function -> how it is pinned (tests/test_oracle.py)
PINNED = {
    "route": "brute force over tiny inputs; torch.topk on distinct values; ties to the lower id;"
             " weight sums (1 or routed_scaling); group mask by hand",
    "sort_assignments": "brute-force stable counting sort; invariants slots[order[i]] = i,"
                        " ids nondecreasing along order, offsets = cumsum(bincount)",
    "routing_statistics": "closed forms on hand-built inputs (uniform logits, one-hot routes)",
    "routing_gradient": "torch autograd of the closed-form route weights / aux / probability sum",
    "quantize_blocks": "zero block stays zero; amax element maps to +-448; <= 1 e4m3 step;"
                       " torch float8 cast as the rounding library",
    "quantize_rows_1x128": "as quantize_blocks, per 1x128 group, reciprocal-multiply descale",
    "quantize_transpose_padded": "pow2 descales: power-of-two and amax/scale in (224, 448] properties",
    "grouped_gemm": "fp64 dequantized product vs a per-row dot-product loop",
    "swiglu / routed_swiglu_backward": "torch autograd of silu(min(g,L))*clamp(u,L)",
    "native_moe": "dense-masked (reference) vs sparse-gathered evaluation; autograd gradients",
    "fp8_moe_forward / fp8_moe_backward": "equal native_moe (output, both input gradients, both"
                                          " weight gradients, router gradient; two routing"
                                          " modes, a SwiGLU limit) when e4m3 rounding is the"
                                          " identity",
    "wgrad": "row-by-row outer-product sums over each expert's unpadded rows (exact under"
             " identity rounding, since the descales are powers of two)",
    "combine / unpermute_sum": "per-token fp64 loops, within one bf16 step",
    "quantize_rows_current": "128-wide rows equal the pinned quantize_rows_1x128; per-row closed"
                             " form with numpy; zero row; amax element maps to +-448",
    "quantize_weights_current": "the reference container test's bounds (row-max relative error"
                                " < 0.07 both orientations); interleaved = chunk/stack of the plain"
                                " layout; dequantized interleaved == plain",
    "rowwise_gemm": "fp64 product vs a per-row dot-product loop",
    "current_moe_forward": "equals native_moe when the quantizers are identities",
}


# ----------------------------------------------------------------- routing
def route(logits, top_k, mode, *, bias=None, n_group=1, topk_group=1, routed_scaling=1.0,
          forced_ids=None):
    """``(weights fp32 [T,k], ids int32 [T,k])`` -- kernels/moe_router.py:347-400
    (route_torch): stable descending sort, ties to the lower expert id."""
    lf = logits.float()
    if forced_ids is not None:
        ids = forced_ids.long()
    elif mode == "sigmoid_noaux_tc":
        scores = torch.sigmoid(lf)
        sel = scores + (0.0 if bias is None else bias.float())
        tokens, experts = sel.shape
        if int(topk_group) < int(n_group):
            grouped = sel.view(tokens, int(n_group), experts // int(n_group))
            grouped, _ = torch.sort(grouped, dim=-1, descending=True, stable=True)
            gscore = grouped[..., : min(2, grouped.shape[-1])].sum(-1)
            _, gids = torch.sort(gscore, dim=-1, descending=True, stable=True)
            gmask = torch.zeros(tokens, int(n_group), dtype=torch.bool, device=sel.device)
            gmask.scatter_(1, gids[:, : int(topk_group)], True)
            sel = sel.masked_fill(~gmask.repeat_interleave(experts // int(n_group), 1), -math.inf)
        _, ids = torch.sort(sel, dim=-1, descending=True, stable=True)
        ids = ids[:, : int(top_k)]
    elif mode in ("topk_then_softmax", "softmax_then_topk"):
        sel = torch.softmax(lf, -1) if mode == "softmax_then_topk" else lf
        _, ids = torch.sort(sel, dim=-1, descending=True, stable=True)
        ids = ids[:, : int(top_k)]
    else:
        raise ValueError(f"unsupported routing mode {mode!r}")
    if mode == "sigmoid_noaux_tc":
        picked = torch.sigmoid(lf).gather(1, ids)
        weights = picked / picked.sum(-1, keepdim=True) * float(routed_scaling)
    elif mode == "softmax_then_topk":
        weights = torch.softmax(lf, -1).gather(1, ids)
    else:
        weights = torch.softmax(lf.gather(1, ids), -1)
    return weights.float(), ids.to(torch.int32)


def probabilities(logits, mode):
    """Softmax (softmax modes) or normalized sigmoid -- providers/moe_common.py:38-43."""
    if mode == "sigmoid_noaux_tc":
        s = torch.sigmoid(logits.float())
        return s / s.sum(-1, keepdim=True)
    return torch.softmax(logits.float(), -1)


def routing_statistics(logits, ids, mode, lengths, experts):
    """``(aux, counts int64 [E], probability_sum [E])`` -- providers/moe_common.py:32-71."""
    rows = logits.shape[0]
    p = probabilities(logits, mode)
    prob_sum = p.sum(0)
    counts = torch.bincount(ids.reshape(-1).long(), minlength=experts)
    if mode == "sigmoid_noaux_tc":
        aux = torch.zeros((), dtype=torch.float32, device=logits.device)
        start = 0
        for length in lengths:
            stop = start + int(length)
            seg = torch.bincount(ids[start:stop].reshape(-1).long(), minlength=experts).float()
            freq = seg * experts / (ids.shape[1] * int(length))
            aux = aux + (freq * p[start:stop].mean(0)).sum()
            start = stop
    else:
        freq = counts.float() / ids.numel()
        aux = experts * (freq * (prob_sum / rows)).sum()
    return aux, counts, prob_sum


def routing_gradient(grad_aux, grad_prob_sum, grad_weights, weights, ids, logits, mode, lengths):
    """fp32 logit gradient -- providers/moe_common.py:74-124 with
    kernels/moe_router.py:403-452 (route_backward), :455-473 (batch aux),
    :476-502 (sequence aux)."""
    lf = logits.float()
    sel = ids.long()
    g = grad_weights.float()
    w = weights.float()
    tokens, experts = lf.shape
    grad = torch.zeros_like(lf)
    if mode == "sigmoid_noaux_tc":
        s_sel = torch.sigmoid(lf).gather(1, sel)
        score_sum = s_sel.sum(-1, keepdim=True)
        scaling = w.sum(-1, keepdim=True)
        dot = (g * w).sum(-1, keepdim=True)
        grad.scatter_(1, sel, ((scaling * g - dot) / score_sum) * s_sel * (1 - s_sel))
    elif mode == "topk_then_softmax":
        grad.scatter_(1, sel, w * (g - (g * w).sum(-1, keepdim=True)))
    else:
        p = torch.softmax(lf, -1)
        top = p.gather(1, sel)
        dot = (g * top).sum(-1, keepdim=True)
        grad = -p * dot
        grad.scatter_add_(1, sel, g * top)
    if grad_aux is not None:
        if mode == "sigmoid_noaux_tc":
            s = torch.sigmoid(lf)
            row_sum = s.sum(-1, keepdim=True)
            q = s / row_sum
            start = 0
            for length in lengths:
                stop = start + int(length)
                counts = torch.bincount(sel[start:stop].reshape(-1), minlength=experts).float()
                f = counts * experts / (sel.shape[1] * int(length))
                coef = grad_aux.float() / (int(length) * row_sum[start:stop])
                sg = coef * (f.unsqueeze(0) - (q[start:stop] @ f).unsqueeze(1))
                grad[start:stop] += sg * s[start:stop] * (1 - s[start:stop])
                start = stop
        else:
            counts = torch.bincount(sel.reshape(-1), minlength=experts).float()
            f = counts / sel.numel()
            p = torch.softmax(lf, -1)
            grad += grad_aux.float() * experts / tokens * p * (f.unsqueeze(0) - (p @ f).unsqueeze(1))
    if grad_prob_sum is not None:
        if mode == "sigmoid_noaux_tc":
            s = torch.sigmoid(lf)
            p = s / s.sum(-1, keepdim=True)
            scale = (1 - s) * p
        else:
            p = torch.softmax(lf, -1)
            scale = p
        gs = grad_prob_sum.float()
        grad += scale * (gs.unsqueeze(0) - (p @ gs).unsqueeze(1))
    return grad


# ------------------------------------------------------------- permutation
def sort_assignments(ids, experts):
    """``(order, offsets, slots)`` -- kernels/moe_dispatch.py:106-119."""
    flat = ids.reshape(-1).long()
    order = torch.argsort(flat, stable=True).to(torch.int32)
    counts = torch.bincount(flat, minlength=experts)
    offsets = torch.zeros(experts + 1, dtype=torch.int32)
    offsets[1:] = counts.cumsum(0).to(torch.int32)
    slots = torch.empty_like(flat, dtype=torch.int32)
    slots[order.long()] = torch.arange(flat.numel(), dtype=torch.int32)
    return order, offsets, slots.view_as(ids)


def combine(y, slots, weights, residual):
    """``bf16(residual + sum_j w * y[slot])`` in fp32 -- kernels/moe_dispatch.py:168-196."""
    gathered = y[slots.reshape(-1).long()].float().view(*slots.shape, y.shape[1])
    routed = (gathered * weights.float().unsqueeze(-1)).sum(1)
    return (residual.float() + routed).to(residual.dtype)


def unpermute_sum(dx, slots):
    """``sum_j dx[slot]`` -- kernels/moe_dispatch.py:136-165."""
    gathered = dx[slots.reshape(-1).long()].float().view(*slots.shape, dx.shape[1])
    return gathered.sum(1).to(dx.dtype)


# ------------------------------------------------------------- quantizers
def _e4m3(values):
    """Round to OCP e4m3 (torch's cast: round to nearest even)."""
    return values.to(FP8)


def quantize_blocks(weight):
    """``(data e4m3, scale fp32)`` -- kernels/block_fp8.py:84-93 (CPU branch):
    ``scale = max(amax / 448, 1e-12)`` (true division) per 128x128 block,
    zero padding, ``data = e4m3(clip(w / scale, +-448))``."""
    w = weight.float()
    experts, out, inner = w.shape
    bo, bi = -(-out // 128), -(-inner // 128)
    padded = torch.zeros(experts, bo * 128, bi * 128)
    padded[:, :out, :inner] = w
    blocks = padded.view(experts, bo, 128, bi, 128)
    scale = (blocks.abs().amax(dim=(2, 4)) / E4M3_MAX).clamp_min(1e-12)
    expanded = scale.repeat_interleave(128, 1).repeat_interleave(128, 2)[:, :out, :inner]
    data = _e4m3((w / expanded).clamp(-E4M3_MAX, E4M3_MAX))
    return data, scale


def dequantize_blocks(data, scale):
    """``data * scale`` per block -- kernels/block_fp8.py:96-99."""
    _, out, inner = data.shape
    expanded = scale.float().repeat_interleave(128, 1).repeat_interleave(128, 2)[:, :out, :inner]
    return data.float() * expanded


def quantize_rows_1x128(x):
    """``(q e4m3 [R,W], scales [W/128, R])``: the row quantizer's equations
    (kernels/quack_moe/quantize_rows.py:35-41, 210-226: ``amax * (1/448)``
    then RN division and clipping) applied per 1x128 group."""
    x = x.float()
    rows, width = x.shape
    groups = x.view(rows, width // 128, 128)
    amax = groups.abs().amax(-1)
    scales = torch.clamp_min(amax * torch.tensor(INV448, dtype=torch.float32), 1e-12)
    q = _e4m3((groups / scales.unsqueeze(-1)).clamp(-E4M3_MAX, E4M3_MAX)).view(rows, width)
    return q, scales.t().contiguous()


def gate_up_columns(width):
    """Source column of each stored column when an interleaved gate/up row is
    stored gate-first -- kernels/quack_moe/quantize_rows.py:119-130 (gate_up)."""
    half = width // 2
    logical = torch.arange(width)
    return torch.where(logical < half, 2 * logical, 2 * (logical - half) + 1)


def dequantize_rows(q, scales):
    rows, width = q.shape
    return (q.float().view(rows, width // 128, 128) * scales.t().unsqueeze(-1)).view(rows, width)


def padded_layout(offsets):
    """Per-expert 128-aligned padded row starts and the padded total."""
    counts = (offsets[1:] - offsets[:-1]).tolist()
    starts, acc = [], 0
    for c in counts:
        starts.append(acc)
        acc += -(-c // 128) * 128
    return starts, acc


def pow2_ceil(x):
    """Smallest power of two >= x, for positive normal fp32 x (exact: bit
    arithmetic on the exponent field)."""
    bits = x.float().contiguous().view(torch.int32)
    up = (bits & 0x7F800000) + 0x00800000
    return torch.where((bits & 0x007FFFFF) != 0, up, bits).view(torch.float32)


def quantize_transpose_padded(rows_bf16, offsets, padded):
    """Feature-major e4m3 ``[W, P]`` + scales ``[P/128, W]``: each expert's rows
    at its 128-aligned padded start, one descale per (feature, 128-row block).
    The descale is ``max(amax * (1/448), 1e-12)`` -- the per-feature rule of
    kernels/quack_moe/quantize_transpose.py:116-117 -- rounded up to a power of
    two (the MFMA applies power-of-two scales in hardware), then ``q =
    e4m3(clip(x / scale, +-448))`` as at :117."""
    x = rows_bf16.float()
    width = x.shape[1]
    starts, total = padded_layout(offsets)
    full = torch.zeros(padded, width)
    for e, start in enumerate(starts):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        full[start:start + hi - lo] = x[lo:hi]
    groups = full.t().contiguous().view(width, padded // 128, 128)
    amax = groups.abs().amax(-1)
    scales = pow2_ceil(torch.clamp_min(amax * torch.tensor(INV448, dtype=torch.float32), 1e-12))
    q = _e4m3((groups / scales.unsqueeze(-1)).clamp(-E4M3_MAX, E4M3_MAX)).view(width, padded)
    return q, scales.t().contiguous(), total


def quantize_rows_current(x):
    """``(q e4m3 [R, W], scales fp32 [R])``: one descale per row --
    kernels/quack_moe/quantize_rows.py:35-41, 210-226 (``amax * (1/448)`` in
    fp32, floor 1e-12, RN division, clip to +-448, e4m3 rounding)."""
    x = x.float()
    amax = x.abs().amax(-1)
    scales = torch.clamp_min(amax * torch.tensor(INV448, dtype=torch.float32), 1e-12)
    q = _e4m3((x / scales[:, None]).clamp(-E4M3_MAX, E4M3_MAX))
    return q, scales


def interleave_rows(w):
    """``[E, out, in]`` gate-then-up rows -> stored 2j = gate j, 2j + 1 = up j
    (expert_parallel/quack/parameters/fp8.py:24-27)."""
    experts, out, inner = w.shape
    return w.view(experts, 2, out // 2, inner).transpose(1, 2).reshape(w.shape)


def quantize_weights_current(w, interleaved=False):
    """``(data [E,out,in], transposed [E,in,out], scale [E,out],
    transposed_scale [E,in])``: both orientations quantized per row, rows
    gate/up-adjacent when ``interleaved`` -- kernels/quack_moe/
    quantize_transpose.py:316-339 (the GPU path: reciprocal-multiply descale,
    :116-117 and :247-255 for the transposed orientation)."""
    v = w.float()
    if interleaved:
        v = interleave_rows(v)
    experts, out, inner = v.shape
    data, scale = quantize_rows_current(v.reshape(experts * out, inner))
    cols, cscale = quantize_rows_current(v.transpose(1, 2).reshape(experts * inner, out))
    return (data.view(experts, out, inner), cols.view(experts, inner, out),
            scale.view(experts, out), cscale.view(experts, inner))


# ------------------------------------------------------------------ GEMMs
def rowwise_gemm(aq, a_scales, wq, w_scales, offsets):
    """fp64 ``(a @ w[e]^T) * a_scale[r] * w_scale[e, n]`` per expert: the
    row-scaled epilogue GEMM of the fp8_current path (kernels/quack_moe/
    fp8.py, providers/sonicmoe/fp8.py:205-247). ``wq`` is ``[E, N, K]``."""
    a = aq.double() * a_scales.double()[:, None]
    w = wq.double() * w_scales.double()[..., None]
    out = torch.zeros(a.shape[0], w.shape[1], dtype=torch.float64)
    for e in range(w.shape[0]):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        if hi > lo:
            out[lo:hi] = a[lo:hi] @ w[e].t()
    return out


def grouped_gemm(aq, a_scales, wq, w_scale, offsets, *, transposed=False, interleave=False):
    """fp64 product of the dequantized operands per expert -- the quantity
    kernels/block_fp8.py:120-236 and quack_moe/block_fp8_gemm.py:1424-1482
    compute. ``transposed``: ``wq`` is the weight ``[E,K,N]`` itself (scale
    ``[E,K/128,N/128]``) and the product is ``rows @ W`` (input gradient),
    else ``rows @ W^T`` with ``wq [E,N,K]``."""
    a = dequantize_rows(aq, a_scales).double()
    w = dequantize_blocks(wq, w_scale).double()
    rows = a.shape[0]
    n = w.shape[2] if transposed else w.shape[1]
    out = torch.zeros(rows, n, dtype=torch.float64)
    for e in range(w.shape[0]):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        if hi > lo:
            out[lo:hi] = a[lo:hi] @ (w[e] if transposed else w[e].t())
    if interleave:
        half = n // 2
        out = torch.stack((out[:, :half], out[:, half:]), dim=-1).reshape(rows, n)
    return out


def wgrad(pq, p_scales, qq, q_scales, offsets):
    """``dW[e] = sum_rows p q^T`` over expert e's padded rows (fp64, dequantized)."""
    p = dequantize_rows(pq, p_scales).double()
    q = dequantize_rows(qq, q_scales).double()
    starts, _ = padded_layout(offsets)
    experts = len(starts)
    out = torch.zeros(experts, p.shape[0], q.shape[0], dtype=torch.float64)
    for e, start in enumerate(starts):
        n = int(offsets[e + 1] - offsets[e])
        stop = start + -(-n // 128) * 128
        out[e] = p[:, start:stop] @ q[:, start:stop].t()
    return out


# ----------------------------------------------------------------- SwiGLU
def swiglu(h13, limit=None):
    """``silu(min(g, L)) * clamp(u, +-L)`` of interleaved ``h13`` in fp32 --
    kernels/quack_moe/swiglu_rows.py:32-76."""
    h = h13.float()
    g, u = h[:, 0::2], h[:, 1::2]
    if limit is not None:
        g, u = g.clamp(max=limit), u.clamp(-limit, limit)
    return F.silu(g) * u


def routed_swiglu_backward(r, h13, score, limit=None):
    """``(dscore, dh interleaved, a')`` -- kernels/quack_moe/swiglu_rows.py:101-146."""
    h = h13.float()
    rg, ru = h[:, 0::2], h[:, 1::2]
    g, u = rg, ru
    if limit is not None:
        g, u = g.clamp(max=limit), u.clamp(-limit, limit)
    sig = torch.sigmoid(g)
    silu = g * sig
    act = silu * u
    r = r.float()
    dscore = (r * act).sum(-1)
    gg = r * score.float().unsqueeze(1)
    dgate = gg * u * (sig + silu * (1 - sig))
    dup = gg * silu
    if limit is not None:
        dgate = torch.where(rg <= limit, dgate, torch.zeros_like(dgate))
        dup = torch.where((ru >= -limit) & (ru <= limit), dup, torch.zeros_like(dup))
    dh = torch.stack((dgate, dup), -1).reshape(h.shape)
    return dscore, dh, act * score.float().unsqueeze(1)


# ------------------------------------------------------------ router GEMM
def router_logits(x, router_weight):
    """fp32 logits from bf16 operands with fp32 sums -- kernels/router.py:54-70."""
    return x.to(torch.bfloat16).float() @ router_weight.to(torch.bfloat16).float().t()


# -------------------------------------------------------------- full layer
def native_moe(h2, residual, router_weight, w13, w2, *, top_k, routing_mode, router_bias=None,
               n_group=1, topk_group=1, routed_scaling=1.0, lengths=None, swiglu_limit=None,
               compute_dtype=torch.float32, lora=None):
    """The reference's native oracle -- kernels/moe_reference.py:20-109: every
    expert runs on every row, masked by its route coefficient. Differentiable
    (plain autograd). Computed at ``compute_dtype`` (fp32 by default).
    ``w13``/``w2`` are ``[E, ...]`` tensors or lists of per-expert ``[...]``
    tensors (same values; per-expert leaves avoid autograd materializing a
    full ``[E, ...]`` gradient for every expert's slice).

    ``lora = (a13, b13, a2, b2, scale)`` adds expert LoRA as
    lora/experts.py:46-50 and :160-163 compose it: each projection
    ``v @ W[e]^T`` becomes ``v @ W[e]^T + scale * (v @ A[e]^T) @ B[e]^T``."""
    shape = h2.shape
    x = h2.reshape(-1, shape[-1])
    res = residual.reshape_as(x)
    rows = x.shape[0]
    lengths = (rows,) if lengths is None else tuple(lengths)
    logits = router_logits(x, router_weight)
    weights, ids = route(logits, top_k, routing_mode, bias=router_bias, n_group=n_group,
                         topk_group=topk_group, routed_scaling=routed_scaling)
    # Route weights stay differentiable functions of the logits (route_torch
    # keeps them live); the selection itself is not differentiable.
    weights = _live_weights(logits, ids, routing_mode, routed_scaling)
    experts = router_weight.shape[0]
    aux, counts, prob_sum = _live_statistics(logits, ids, routing_mode, lengths, experts)
    width = w2[0].shape[-1]
    xc = x.to(compute_dtype)
    routed = torch.zeros(rows, shape[-1], dtype=torch.float32, device=x.device)
    for e in range(experts):
        coef = (weights * (ids == e)).sum(-1)
        h13 = xc @ w13[e].to(compute_dtype).t()
        if lora is not None:
            a13, b13, scale = lora[0][e], lora[1][e], lora[4]
            h13 = h13 + scale * (xc @ a13.to(compute_dtype).t()) @ b13.to(compute_dtype).t()
        g, u = h13[:, :width], h13[:, width:]
        if swiglu_limit is not None:
            g, u = g.clamp(max=swiglu_limit), u.clamp(-swiglu_limit, swiglu_limit)
        act = F.silu(g.float()).to(compute_dtype) * u
        y = act @ w2[e].to(compute_dtype).t()
        if lora is not None:
            a2, b2, scale = lora[2][e], lora[3][e], lora[4]
            y = y + scale * (act @ a2.to(compute_dtype).t()) @ b2.to(compute_dtype).t()
        routed = routed + coef[:, None] * y.float()
    out = (res.float() + routed).to(h2.dtype)
    return out.reshape(shape), aux, counts, prob_sum


def _live_weights(logits, ids, mode, routed_scaling):
    lf = logits.float()
    sel = ids.long()
    if mode == "sigmoid_noaux_tc":
        picked = torch.sigmoid(lf).gather(1, sel)
        return picked / picked.sum(-1, keepdim=True) * float(routed_scaling)
    if mode == "softmax_then_topk":
        return torch.softmax(lf, -1).gather(1, sel)
    return torch.softmax(lf.gather(1, sel), -1)


def _live_statistics(logits, ids, mode, lengths, experts):
    p = probabilities(logits, mode)
    counts = torch.bincount(ids.reshape(-1).long(), minlength=experts)
    prob_sum = p.sum(0)
    if mode == "sigmoid_noaux_tc":
        aux = torch.zeros((), dtype=torch.float32, device=logits.device)
        start = 0
        for length in lengths:
            stop = start + int(length)
            seg = torch.bincount(ids[start:stop].reshape(-1).long(), minlength=experts).float()
            freq = seg * experts / (ids.shape[1] * int(length))
            aux = aux + (freq * p[start:stop].mean(0)).sum()
            start = stop
    else:
        freq = counts.float() / ids.numel()
        aux = experts * (freq * (prob_sum / logits.shape[0])).sum()
    return aux, counts, prob_sum


def fp8_moe_forward(x, residual, router_weight, w13_q, w13_s, w2_q, w2_s, *, top_k, routing_mode,
                    router_bias=None, n_group=1, topk_group=1, routed_scaling=1.0, lengths=None,
                    swiglu_limit=None, logits=None):
    """The block-FP8 layer forward with the MI355X provider's quantization
    points (1x128 activations, 128x128 weights), fp64 products of dequantized
    operands, bf16 roundings where the provider stores bf16. Restates
    providers/sonicmoe/moe.py:441-515 with providers/sonicmoe/block_fp8.py:114-140.
    Returns a dict of every intermediate."""
    rows, width = x.shape
    lengths = (rows,) if lengths is None else tuple(lengths)
    experts = router_weight.shape[0]
    if logits is None:
        logits = router_logits(x, router_weight)
    weights, ids = route(logits, top_k, routing_mode, bias=router_bias, n_group=n_group,
                         topk_group=topk_group, routed_scaling=routed_scaling)
    order, offsets, slots = sort_assignments(ids, experts)
    xr = x[order.long() // top_k]
    xq, xs = quantize_rows_1x128(xr)
    h13 = grouped_gemm(xq, xs, w13_q, w13_s, offsets, interleave=True).to(torch.bfloat16)
    act = swiglu(h13, swiglu_limit)
    aq, as_ = quantize_rows_1x128(act)
    y = grouped_gemm(aq, as_, w2_q, w2_s, offsets).to(torch.bfloat16)
    out = combine(y, slots, weights, residual)
    aux, counts, prob_sum = routing_statistics(logits, ids, routing_mode, lengths, experts)
    return dict(out=out, aux=aux, counts=counts, prob_sum=prob_sum, logits=logits,
                weights=weights, ids=ids, order=order, offsets=offsets, slots=slots, xq=xq, xs=xs,
                h13=h13, aq=aq, as_=as_, y=y)


def current_moe_forward(x, residual, router_weight, w13, w2, *, top_k, routing_mode,
                        router_bias=None, n_group=1, topk_group=1, routed_scaling=1.0,
                        lengths=None, swiglu_limit=None, logits=None):
    """The fp8_current layer forward at the MI355X provider's quantization
    points: routed rows quantized per row, the up product against the
    gate/up-adjacent rows of ``w13`` (``(data, transposed, scale,
    transposed_scale)`` as quantize_weights_current gives with interleaved),
    bf16 ``h13`` (interleaved), SwiGLU of it quantized per row, the down
    product, combine. Restates providers/sonicmoe/moe.py:441-515 with
    sonicmoe/fp8.py:205-264 (the activation from the stored pre-activation, as
    project_down_from_preactivation does)."""
    rows, width = x.shape
    lengths = (rows,) if lengths is None else tuple(lengths)
    experts = router_weight.shape[0]
    if logits is None:
        logits = router_logits(x, router_weight)
    weights, ids = route(logits, top_k, routing_mode, bias=router_bias, n_group=n_group,
                         topk_group=topk_group, routed_scaling=routed_scaling)
    order, offsets, slots = sort_assignments(ids, experts)
    xq, xs = quantize_rows_current(x[order.long() // top_k])
    h13 = rowwise_gemm(xq, xs, w13[0], w13[2], offsets).to(torch.bfloat16)
    aq, as_ = quantize_rows_current(swiglu(h13, swiglu_limit))
    y = rowwise_gemm(aq, as_, w2[0], w2[2], offsets).to(torch.bfloat16)
    out = combine(y, slots, weights, residual)
    aux, counts, prob_sum = routing_statistics(logits, ids, routing_mode, lengths, experts)
    return dict(out=out, aux=aux, counts=counts, prob_sum=prob_sum, logits=logits,
                weights=weights, ids=ids, order=order, offsets=offsets, slots=slots, xq=xq, xs=xs,
                h13=h13, aq=aq, as_=as_, y=y)


def fp8_moe_backward(fwd, x, grad_out, router_weight, w13_q, w13_s, w2_q, w2_s, *, top_k,
                     routing_mode, lengths=None, swiglu_limit=None, grad_aux=None,
                     grad_prob_sum=None):
    """The block-FP8 layer backward at the provider's quantization points:
    providers/sonicmoe/moe.py:268-438 and :517-620 with
    providers/sonicmoe/block_fp8.py:143-196 (dgrad / dSwiGLU), the wgrad
    operands quantized per (feature, 128-row block) of each expert."""
    rows, width = x.shape
    lengths = (rows,) if lengths is None else tuple(lengths)
    order, offsets, slots = fwd["order"], fwd["offsets"], fwd["slots"]
    tok = order.long() // top_k
    dyr = grad_out[tok]
    dyq, dys = quantize_rows_1x128(dyr)
    r = grouped_gemm(dyq, dys, w2_q, w2_s, offsets, transposed=True).to(torch.bfloat16)
    score = fwd["weights"].reshape(-1)[order.long()]
    dscore, dh, a_prime = routed_swiglu_backward(r, fwd["h13"], score, swiglu_limit)
    dh = dh.to(torch.bfloat16)
    a_prime = a_prime.to(torch.bfloat16)
    _, padded = padded_layout(offsets)
    padded = max(padded, 128)
    dyt, dyts, _ = quantize_transpose_padded(dyr, offsets, padded)
    apt, apts, _ = quantize_transpose_padded(a_prime, offsets, padded)
    dw2 = wgrad(dyt, dyts, apt, apts, offsets)
    cols = gate_up_columns(dh.shape[1])
    dh_planar = dh[:, cols]
    dhq, dhs = quantize_rows_1x128(dh_planar)
    dx = grouped_gemm(dhq, dhs, w13_q, w13_s, offsets, transposed=True).to(torch.bfloat16)
    dht, dhts, _ = quantize_transpose_padded(dh_planar, offsets, padded)
    xt, xts, _ = quantize_transpose_padded(x[tok], offsets, padded)
    dw13 = wgrad(dht, dhts, xt, xts, offsets)
    grad_x = unpermute_sum(dx, slots)
    grad_w = dscore[slots.reshape(-1).long()].view(rows, top_k)
    grad_logits = routing_gradient(grad_aux, grad_prob_sum, grad_w, fwd["weights"], fwd["ids"],
                                   fwd["logits"], routing_mode, lengths)
    xb = x.to(torch.bfloat16).float()
    grad_router = grad_logits.t() @ xb
    grad_x = (grad_x.float() + grad_logits.to(torch.bfloat16).float()
              @ router_weight.to(torch.bfloat16).float()).to(torch.bfloat16)
    return dict(grad_x=grad_x, grad_router=grad_router, dw13=dw13, dw2=dw2, r=r, dh=dh,
                a_prime=a_prime, dscore=dscore, dx=dx, grad_logits=grad_logits)


__all__ = [name for name in dir() if not name.startswith("_")]
