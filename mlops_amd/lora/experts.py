"""Expert LoRA on the MI355X block-FP8 MoE path.

``expert_lora`` (reference: ``src/mlops/lora/experts.py:53-167``) is the
routed MoE layer with a rank-r correction on both projections of every
expert, ``W -> W + scale * B[e] @ A[e]``:

    h13 = x @ W13[e]^T + scale * (x @ A13[e]^T) @ B13[e]^T
    y   = a @ W2[e]^T  + scale * (a @ A2[e]^T) @ B2[e]^T,   a = SwiGLU(h13)

The base weights are block-FP8 (``BlockFP8Weight`` containers, or plain
masters quantized per call with ``compute_precision="fp8_block"``) or
per-row FP8 (``RowFP8Weight``, or ``compute_precision="fp8_current"``), as
the reference's SonicMoE LoRA serves both (``providers/sonicmoe/lora.py
:36-40``), and run on the MI355X grouped GEMMs. Each low-rank term
``z @ F^T`` starts the GEMM's fp32 accumulators
(``mi355x_gemm_fp8_block_lora`` / ``mi355x_gemm_fp8_rowwise_lora``: a
rank-16-at-a-time bf16 MFMA per output tile; the row-scaled form divides it
by the descales its epilogue applies), where the reference's SonicMoE composition passes it
as the GEMM's C input (``providers/sonicmoe/lora.py:1-45``): no LoRA term is
materialized as ``[rows, N]`` or added by a separate pass. The scale is
folded into the small ``B`` factors; ranks are padded with zero columns to a
multiple of 16.

Rank projections of token rows (``x @ A13^T`` forward, ``dy @ B2`` backward)
are formed once per token for all experts, as one dense ``[T, E*r]`` GEMM
(hipBLASLt through torch), and gathered to the routed rows; those of routed
rows (``a @ A2^T``, ``dh @ B13``) run on ``mi355x_rank_product``. The four
factor gradients are reductions over each expert's routed rows on
``mi355x_rank_grad`` (token rows gathered for ``dB2`` and ``dA13``), bf16
operands with fp32 sums, with no host synchronization; they come back at the
factors' dtype.
"""

from __future__ import annotations

import torch

from .. import kernels, router
from ..dispatch.context import weight_gradient_dtype
from ..providers.mi355x import moe as provider
from ..providers.mi355x import moe_current
from ..routing import current_route_weight_precision, next_override
from ..weight_formats import is_row_fp8

IMPLEMENTATIONS = ("auto", "mi355x")


def interleaved_rows(b: torch.Tensor) -> torch.Tensor:
    """``[E, 2I, r]`` gate rows then up rows -> gate/up rows alternating
    (reference ``providers/sonicmoe/lora.py:81-84``)."""
    experts, packed, rank = b.shape
    return b.view(experts, 2, packed // 2, rank).transpose(1, 2).reshape(b.shape)


def gate_up_rows(b: torch.Tensor) -> torch.Tensor:
    """Inverse of :func:`interleaved_rows`."""
    experts, packed, rank = b.shape
    return b.view(experts, packed // 2, 2, rank).transpose(1, 2).reshape(b.shape)


def _padded(t: torch.Tensor, rank: int) -> torch.Tensor:
    """``t [..., r]`` with zero columns up to ``rank``, contiguous."""
    extra = rank - t.shape[-1]
    return torch.nn.functional.pad(t, (0, extra)).contiguous() if extra else t.contiguous()


def _padded_rank_rows(t: torch.Tensor, rank: int) -> torch.Tensor:
    """``t [E, r, n]`` with zero rows up to ``rank``, contiguous."""
    extra = rank - t.shape[1]
    return torch.nn.functional.pad(t, (0, 0, 0, extra)).contiguous() if extra else t.contiguous()


def _scaled_bf16(t: torch.Tensor, scale: float) -> torch.Tensor:
    """``bf16(t * scale)`` with one rounding of the fp32 product (a bf16 ``t``
    is multiplied in fp32 by torch and rounded once, in one kernel)."""
    if t.dtype == torch.bfloat16:
        return torch.mul(t, scale)
    return (t.float() * scale).to(torch.bfloat16)


def _rank16(r: int) -> int:
    return -(-r // 16) * 16


def _row_rank(rows: torch.Tensor, factors_t: torch.Tensor, offsets) -> torch.Tensor:
    """``rows[r] @ factors_t[e]^T`` for each expert's rows, bf16 ``[rows, R]``
    (R a multiple of 16): the thin product kernel, 64 rank columns per call."""
    rank = factors_t.shape[1]
    if rank <= 64:
        return kernels.rank_product(rows, factors_t, offsets)
    return torch.cat([kernels.rank_product(rows, factors_t[:, c:c + 64].contiguous(), offsets)
                      for c in range(0, rank, 64)], dim=1)


def _factor_grad(big: torch.Tensor, small: torch.Tensor, offsets, rank: int, *,
                 transposed: bool, **gather) -> torch.Tensor:
    """Per expert ``sum_j big[j]^T small[j]`` over its rows, fp32, cut to the
    true ``rank``: ``[E, M, rank]``, or ``[E, rank, M]`` when ``transposed``.
    bf16 operands with fp32 sums (``mi355x_rank_grad``, no host sync).
    ``gather`` options (token rows of ``big``, a per-row weight on ``small``)
    pass through to :func:`kernels.rank_grad`."""
    padded = _padded(small, _rank16(rank))
    parts = [kernels.rank_grad(big, padded[:, c:c + 64].contiguous(), offsets,
                               transposed=transposed, **gather)
             for c in range(0, padded.shape[1], 64)]
    out = parts[0] if len(parts) == 1 else torch.cat(parts, dim=1 if transposed else 2)
    return (out[:, :rank] if transposed else out[..., :rank]).contiguous()


def _token_projection(x_tok: torch.Tensor, factors_flat: torch.Tensor, experts: int,
                      tokens_of_row: torch.Tensor, experts_of_row: torch.Tensor) -> torch.Tensor:
    """Per routed row j: ``x_tok[token_j] @ F[e_j]`` with ``factors_flat``
    ``[D, E*r]`` holding every expert's ``F[e]`` side by side: one dense GEMM
    over the tokens, then the gather."""
    projected = x_tok @ factors_flat
    rank = factors_flat.shape[1] // experts
    return projected.view(x_tok.shape[0], experts, rank)[tokens_of_row, experts_of_row]


class _ExpertLoRA(torch.autograd.Function):
    @staticmethod
    def forward(ctx, hidden, residual, router_weight, w13, w2, a13, b13, a2, b2, opts):
        ctx.set_materialize_grads(False)
        top_k, mode, scale, limit = opts["top_k"], opts["routing_mode"], opts["scale"], opts["limit"]
        width = hidden.shape[-1]
        tokens = hidden.numel() // width
        experts = router_weight.shape[0]
        current = is_row_fp8(w13)
        if current:  # rows (gate/up-adjacent for w13), transpose, per-row descales
            w13_data, _, w13_scale, _ = w13.components()
            w2_data, _, w2_scale, _ = w2.components()
        else:
            w13_data, w13_scale = w13.components()
            w2_data, w2_scale = w2.components()
        inter = w2_data.shape[2]
        with torch.no_grad():
            x = hidden.reshape(tokens, width).contiguous()
            base = residual.reshape(tokens, width).contiguous()
            logits = router.router_logits(x, router_weight)
            forced = next_override(tokens, experts, top_k, x.device)
            bias = opts["router_bias"]
            weights, ids = kernels.router_topk(
                logits, top_k, mode, bias=bias, n_group=opts["n_group"],
                topk_group=opts["topk_group"], routed_scaling=opts["routed_scaling"],
                forced_ids=forced,
            )
            counts, offsets, order, slots = kernels.permute_plan(ids, experts)
            order_l = order.long()
            rows_token = order_l // top_k
            rows_expert = ids.reshape(-1).long()[order_l]
            # Factors at the activations' dtype, the scale folded into B.
            a13b = a13.detach().to(torch.bfloat16)
            b13s = _scaled_bf16(b13.detach(), scale)
            b13b = interleaved_rows(b13s)
            a2b = a2.detach().to(torch.bfloat16)
            b2b = _scaled_bf16(b2.detach(), scale)
            rank13, rank2 = a13b.shape[1], a2b.shape[1]
            r13, r2 = _rank16(rank13), _rank16(rank2)
            # Up projection: z13 = x @ A13^T per routed row; z13 (s B13)^T
            # starts the GEMM's accumulators (B13 in its gate-first row order,
            # the order of the weight rows the GEMM reads).
            z13 = _token_projection(x, a13b.reshape(experts * rank13, width).t(), experts,
                                    rows_token, rows_expert)
            if current:
                # The per-row w13 is stored gate/up-adjacent: B13 in that order.
                xq, xs = kernels.permute_quantize_current(x, slots)
                h13 = kernels.gemm_rowwise(xq, xs, w13_data, w13_scale, offsets,
                                           lora=(_padded(z13, r13), _padded(b13b, r13)))
                aq, as_, act = kernels.swiglu_quantize_rows_current(h13, limit, activation=True)
            else:
                xq, xs = kernels.permute_quantize(x, slots)
                h13 = kernels.gemm(xq, xs, w13_data, w13_scale, offsets, interleave=True,
                                   lora=(_padded(z13, r13), _padded(b13s, r13)))
                aq, as_, act = kernels.swiglu_quantize(h13, limit, activation=True)
            # Down projection: z2 = a @ A2^T per routed row (the thin product
            # streams a once; rank padded to 16).
            z2p = _row_rank(act, _padded_rank_rows(a2b, r2), offsets)
            if current:
                y = kernels.gemm_rowwise(aq, as_, w2_data, w2_scale, offsets,
                                         lora=(z2p, _padded(b2b, r2)))
            else:
                y = kernels.gemm(aq, as_, w2_data, w2_scale, offsets,
                                 lora=(z2p, _padded(b2b, r2)))
            output = kernels.combine(y, slots, weights, base)
            aux, probability_sum, _, _ = kernels.router_stats(logits, ids, top_k, mode,
                                                              opts["lengths"])
        ctx.opts = opts
        ctx.w13, ctx.w2 = w13, w2
        ctx.factor_dtypes = (a13.dtype, b13.dtype, a2.dtype, b2.dtype)
        # The bf16 activation (A * I * 2 bytes) is kept only for dA2.
        if not ctx.needs_input_grad[7]:
            act = act.new_empty(0)
        ctx.save_for_backward(hidden, router_weight, logits, weights, ids, order, offsets, slots,
                              h13, act, z13, z2p, rows_token, rows_expert, a13b, b13b, a2b, b2b)
        ctx.mark_non_differentiable(counts)
        return output.reshape(hidden.shape), aux, counts, probability_sum

    @staticmethod
    def backward(ctx, grad_output, grad_aux, _grad_counts, grad_probability_sum):
        (hidden, router_weight, logits, weights, ids, order, offsets, slots, h13, act, z13, z2p,
         rows_token, rows_expert, a13b, b13b, a2b, b2b) = ctx.saved_tensors
        opts = ctx.opts
        top_k, mode, scale, limit = opts["top_k"], opts["routing_mode"], opts["scale"], opts["limit"]
        need = ctx.needs_input_grad
        width = hidden.shape[-1]
        tokens = hidden.numel() // width
        experts = router_weight.shape[0]
        assignments = order.numel()
        current = is_row_fp8(ctx.w13)
        if current:
            _, w13_t, _, w13_ts = ctx.w13.components()
            w2_data, w2_t, _, w2_ts = ctx.w2.components()
        else:
            w13_data, w13_scale = ctx.w13.components()
            w2_data, w2_scale = ctx.w2.components()
        inter = w2_data.shape[2]
        rank13, rank2 = a13b.shape[1], a2b.shape[1]
        grad_dtype = weight_gradient_dtype()
        with torch.no_grad():
            x = hidden.reshape(tokens, width).contiguous()
            if grad_output is None:
                dy = torch.zeros((tokens, width), dtype=torch.bfloat16, device=x.device)
            else:
                dy = grad_output.reshape(tokens, width).contiguous().to(torch.bfloat16)
            # Row gradient of the activation, unscaled by the route weight:
            # r = dy_j @ W2[e] + (dy_j @ (s B2[e])) @ A2[e].
            u2 = _token_projection(dy, b2b.permute(1, 0, 2).reshape(width, experts * rank2),
                                   experts, rows_token, rows_expert)
            r2 = _rank16(rank2)
            lora_r = (_padded(u2, r2), _padded(a2b.transpose(1, 2), r2))
            if current:
                dyq, dys = kernels.permute_quantize_current(dy, slots)
                r = kernels.gemm_rowwise(dyq, dys, w2_t, w2_ts, offsets, lora=lora_r)
            else:
                dyq, dys = kernels.permute_quantize(dy, slots)
                w2_t = provider.transposed_data(ctx.w2)
                r = kernels.gemm(dyq, dys, w2_t, w2_scale, offsets, transposed_scale=True,
                                 lora=lora_r)
            # a' = score * a is only an operand of the base W2's gradient; the
            # factor gradient dA2 takes the forward's bf16 a with the score on
            # the thin u2 instead.
            want_ap = bool(need[4])
            if current:
                dh, a_prime, dscore = kernels.routed_swiglu_backward(
                    r, h13, weights.reshape(-1), order, limit, a_prime=want_ap)
            else:
                # dh row-quantized for the input-gradient GEMM in the same pass
                dh, a_prime, dscore, dhq, dhs = kernels.routed_swiglu_backward_rows(
                    r, h13, weights.reshape(-1), order, limit, a_prime=want_ap)
            del r
            # Input gradient: dx_j = dh_j @ W13[e] + (dh_j @ (s B13[e])) @ A13[e].
            r13 = _rank16(rank13)
            u13p = _row_rank(dh, _padded(b13b, r13).transpose(1, 2).contiguous(), offsets)
            lora_x = (u13p, _padded(a13b.transpose(1, 2), r13))
            if current:
                # dh's interleaved columns are the K order of w13's transpose.
                dhq, dhs = kernels.quantize_rows_current(dh)
                dx = kernels.gemm_rowwise(dhq, dhs, w13_t, w13_ts, offsets, lora=lora_x)
            else:
                w13_t = provider.transposed_data(ctx.w13)
                dx = kernels.gemm(dhq, dhs, w13_t, w13_scale, offsets, transposed_scale=True,
                                  lora=lora_x)
            del dhq, dhs
            grad_hidden = kernels.unpermute_sum(dx, slots)
            del dx
            # Factor gradients (fp32 sums), scale applied once.
            grads = [None, None, None, None]
            # Token rows of the routed rows: big[order[j] // k] in the reductions.
            token_rows = dict(gather=order, gather_div=top_k)
            if need[8]:    # B2: s * sum_j dy_{t(j)} (score_j z2_j)^T
                grads[3] = _factor_grad(dy, z2p, offsets, rank2, transposed=False,
                                        weight=weights.reshape(-1), weight_index=order,
                                        alpha=scale, **token_rows)
            if need[7]:    # A2: sum_j (score_j u2_j) a_j^T  (= sum_j u2_j a'_j^T)
                grads[2] = _factor_grad(act, u2, offsets, rank2, transposed=True,
                                        weight=weights.reshape(-1), weight_index=order)
            if need[6]:    # B13: s * sum_j dh_j z13_j^T (rows back to gate then up)
                g = _factor_grad(dh, z13, offsets, rank13, transposed=False)
                grads[1] = gate_up_rows(g.mul_(scale))
            if need[5]:    # A13: sum_j u13_j x_{t(j)}^T
                grads[0] = _factor_grad(x, u13p, offsets, rank13, transposed=True, **token_rows)
            grads = [None if g is None else g.to(dtype)
                     for g, dtype in zip(grads, ctx.factor_dtypes)]
            # Base weight gradients, when the base is trained.
            grad_w13 = grad_w2 = None
            if need[3] or need[4]:
                direct = grad_dtype if grad_dtype in (torch.bfloat16, torch.float32) else torch.float32
                padded = kernels.wgrad_padded_rows(assignments, experts)
                blocks = kernels.padded_row_blocks(offsets, padded)
                common = dict(padded=padded, row_blocks=blocks)
                if need[4]:
                    dy_t, dy_ts, _ = kernels.quantize_transpose(
                        dy, offsets, assignments, gather=order, gather_div=top_k, **common)
                    ap_t, ap_ts, _ = kernels.quantize_transpose(a_prime, offsets, assignments,
                                                                **common)
                    grad_w2 = kernels.wgrad(dy_t, dy_ts, ap_t, ap_ts, offsets, out_dtype=direct,
                                            rows=assignments)
                if need[3]:
                    dh_t, dh_ts, _ = kernels.quantize_transpose(dh, offsets, assignments,
                                                                gate_up=True, **common)
                    x_t, x_ts, _ = kernels.quantize_transpose(
                        x, offsets, assignments, gather=order, gather_div=top_k, **common)
                    grad_w13 = kernels.wgrad(dh_t, dh_ts, x_t, x_ts, offsets, out_dtype=direct,
                                             rows=assignments)
                logical = torch.bfloat16 if grad_dtype is None else grad_dtype
                grad_w13 = None if grad_w13 is None else grad_w13.to(logical)
                grad_w2 = None if grad_w2 is None else grad_w2.to(logical)
            router_dtype = router_weight.dtype if grad_dtype is None else grad_dtype
            grad_router = provider.routing_backward(
                grad_hidden, x, router_weight, logits, weights, ids, dscore, slots, offsets,
                grad_aux, grad_probability_sum, top_k=top_k, routing_mode=mode,
                lengths=opts["lengths"], router_dtype=router_dtype, need_router=bool(need[2]),
            )
        # d residual is the output cotangent itself (no copy).
        grad_residual = grad_output if need[1] else None
        return (grad_hidden.reshape(hidden.shape).to(hidden.dtype) if need[0] else None,
                grad_residual, grad_router if need[2] else None, grad_w13, grad_w2,
                *grads, None)


def expert_lora(
    hidden, residual, router_weight, gate_up, down, a13, b13, a2, b2, *, top_k, routing_mode,
    scale, router_bias=None, n_group=1, topk_group=1, routed_scaling=1.0, lengths=None,
    swiglu_limit=None, implementation="auto", compute_precision=None,
):
    """Routed MoE with per-expert LoRA factors: ``(output, aux, counts,
    probability_sum)`` as ``mlops.lora.experts.expert_lora`` returns them.

    Weights ``gate_up [E, 2I, D]`` (gate rows then up rows) and ``down
    [E, D, I]``, factors ``a13 [E, r, D]``, ``b13 [E, 2I, r]``, ``a2 [E, r, I]``,
    ``b2 [E, D, r]`` (any float dtype, computed in bf16), ``router_weight
    [E, D]``. Routing options and ``swiglu_limit`` are `mlops.moe`'s.
    ``implementation`` is ``"auto"`` or ``"mi355x"`` (this build has no other
    composition); ``compute_precision`` is ``None`` for FP8 containers
    (block or per-row), or ``"fp8_block"`` / ``"fp8_current"`` (plain masters
    quantized per call). Gradients reach the
    factors, the router, the hidden and residual rows, and base weights that
    require them (plain masters; straight through the per-call quantizer).
    """
    if implementation not in IMPLEMENTATIONS:
        raise ValueError(f"unknown expert LoRA implementation {implementation!r}; this build "
                         f"serves {IMPLEMENTATIONS}")
    if swiglu_limit is not None:
        swiglu_limit = float(swiglu_limit)
        if not swiglu_limit > 0:
            raise ValueError("swiglu_limit must be positive")
    rows = hidden.numel() // hidden.shape[-1]
    lengths = (rows,) if lengths is None else tuple(int(x) for x in lengths)
    rules = moe_current if (compute_precision == "fp8_current" or (
        compute_precision is None and any(is_row_fp8(w) for w in (gate_up, down)))
    ) else provider
    support = rules.supports(
        hidden, residual, router_weight, gate_up, down, surface="semantic", top_k=top_k,
        routing_mode=routing_mode, router_bias=router_bias, n_group=n_group,
        topk_group=topk_group, routed_scaling=routed_scaling, lengths=lengths,
        compute_precision=compute_precision, swiglu_limit=swiglu_limit,
    )
    if not support:
        raise ValueError(f"the MI355X expert LoRA path does not apply here: {support.reason}")
    experts, inter, width = router_weight.shape[0], down.shape[2], hidden.shape[-1]
    rank = a13.shape[1]
    expected = {"a13": (experts, rank, width), "b13": (experts, 2 * inter, rank),
                "a2": (experts, a2.shape[1], inter), "b2": (experts, width, a2.shape[1])}
    for name, factor in zip(expected, (a13, b13, a2, b2)):
        if tuple(factor.shape) != expected[name]:
            raise ValueError(f"LoRA factor {name} must have shape {expected[name]}, "
                             f"got {tuple(factor.shape)}")
        if not factor.is_floating_point() or factor.device != hidden.device:
            raise ValueError(f"LoRA factor {name} must be a floating tensor on {hidden.device}")
    w13, w2 = rules._containers(gate_up, down)
    bias = None if router_bias is None or router_bias.numel() == 0 else router_bias
    opts = dict(top_k=int(top_k), routing_mode=str(routing_mode), scale=float(scale),
                limit=swiglu_limit, router_bias=bias, n_group=int(n_group),
                topk_group=int(topk_group), routed_scaling=float(routed_scaling),
                lengths=lengths, weight_precision=current_route_weight_precision())
    return _ExpertLoRA.apply(hidden, residual, router_weight, w13, w2, a13, b13, a2, b2, opts)


__all__ = ["expert_lora", "gate_up_rows", "interleaved_rows"]
