"""The routed block-FP8 MoE as two opaque regions on the MI355X kernels.

Same contract as the reference's composed implementations
(``src/mlops/providers/sonicmoe/moe_composed.py:1-850``,
``src/mlops/providers/builtin/moe_composed.py:1-898``). The routing and
up-projection region ("prepare") ends at the saved pre-activation ``h13``.
The activation, down-projection and combine region ("finish") starts from it.
So AOTAutograd can rematerialize the first region without replaying the
second. The two regions exchange ``h13`` (bf16 ``[A, 2I]``, gate/up
interleaved) and ``route_weights`` forward, and their cotangents backward.

The kernels are those of ``mi355x.moe.block_fp8``. Where the fused backward
quantizes ``dh`` straight from registers, the finish region here writes it as
bf16 (it crosses the region boundary). The prepare region then quantizes it
with the row and transposing quantizers. Those produce, byte for byte, what
the fused pass does, so every output and gradient equals the fused
operator's.

It serves both FP8 precisions, as the reference's composed form does:
block-FP8 weights run the kernels of ``mi355x.moe.block_fp8``, and
``fp8_current`` weights (per-row scales, `RowFP8Weight`) those of
``mi355x.moe.fp8_current``. Either way the results equal that fused
operator's.

The fused operators stay the default (``PRIORITY`` below theirs); this one is
selected by its implementation ID.
"""

from __future__ import annotations

import torch

from ... import kernels, router
from ...block_fp8 import BlockFP8Weight
from ...dispatch import logical_costs as logical
from ...dispatch.context import weight_gradient_dtype
from ...dispatch.costs import flop_formula
from ...dispatch.registry import Implementation, SupportResult, register_implementation
from ...routing import current_route_weight_precision, next_override
from ...row_fp8 import RowFP8Weight
from ...weight_formats import (block_parts, is_row_fp8, register_container_class,
                               route_containers, row_parts)
from . import moe as fused
from . import moe_current as current

IMPLEMENTATION_ID = "mi355x.moe.composed"
PRIORITY = 115  # below mi355x.moe.block_fp8 (120), which is faster


def _is_current(compute_precision, w13, w2) -> bool:
    return compute_precision == "fp8_current" or (
        compute_precision is None and any(is_row_fp8(w) for w in (w13, w2)))


def _supports(h2, residual, router_weight, w13_experts, w2_experts, *, surface, **kwargs):
    """The fused operator's rules at the requested precision (fp8_block, or
    fp8_current, as the reference's composed form serves both)."""
    if surface == "explicit":
        return SupportResult.no("trace-visible MoE composition is a semantic-only implementation")
    rules = current if _is_current(kwargs.get("compute_precision"), w13_experts, w2_experts) else fused
    return rules.supports(h2, residual, router_weight, w13_experts, w2_experts, surface=surface,
                          **kwargs)


class _Weight(tuple):
    """A weight's operands: ``(data, scale[, data_t])`` for 128x128 blocks, or
    ``(data, transposed, scale, transposed_scale)`` per row (``current``)."""

    current = False


def _weight(data, components):
    """The operands from the unwrapped data and its components: one or two
    (the block scale, then optionally the transposed data) for block-FP8,
    three (transposed data, scale, transposed scale) for fp8_current."""
    if len(components) in (1, 2):
        return _Weight((data, *components))
    if len(components) == 3:
        weight = _Weight((data, *components))
        weight.current = True
        return weight
    raise ValueError("a composed region takes its weight's scale (and optionally its transposed "
                     "data), or the three per-row components, as components")


def _rows(x, slots, weight):
    """The routed copies of token rows quantized for ``weight``'s GEMMs."""
    return (kernels.permute_quantize_current(x, slots) if getattr(weight, "current", False)
            else kernels.permute_quantize(x, slots))


def _forward_gemm(aq, as_, weight, offsets, *, interleave=False):
    if getattr(weight, "current", False):
        return kernels.gemm_rowwise(aq, as_, weight[0], weight[2], offsets)
    return kernels.gemm(aq, as_, weight[0], weight[1], offsets, interleave=interleave)


def _input_gradient_gemm(aq, as_, weight, offsets):
    """``rows @ W`` through the weight's transposed copy (per-row FP8), or, for
    block FP8, as :func:`fused.input_gradient_gemm` chooses."""
    if getattr(weight, "current", False):
        return kernels.gemm_rowwise(aq, as_, weight[1], weight[3], offsets)
    return fused.input_gradient_gemm(aq, as_, weight, offsets)


def _grad_dtypes(weight_grad_dtype, router_weight=None):
    """(expert gradient dtype, dtype the wgrad kernel writes, router gradient dtype)."""
    router_dtype = None
    if router_weight is not None:
        router_dtype = router_weight.dtype if weight_grad_dtype is None else weight_grad_dtype
    expert = torch.bfloat16 if weight_grad_dtype is None else weight_grad_dtype
    direct = expert if expert in (torch.bfloat16, torch.float32) else torch.float32
    return expert, direct, router_dtype


# --------------------------------------------------------------------------
# The two regions on plain tensors (weights as (data, scale[, data_t])).
def prepare_forward(h2, router_weight, w13, *, top_k, routing_mode, router_bias=None,
                    n_group=1, topk_group=1, routed_scaling=1.0, lengths=None):
    """``(aux, counts, probability_sum, logits, route_weights, route_ids, order,
    offsets, slots, h13)`` (reference ``builtin/moe_composed.py:58-117``)."""
    width = h2.shape[-1]
    rows = h2.numel() // width
    lengths = fused._normalized((rows,) if lengths is None else lengths, rows)
    experts = router_weight.shape[0]
    with torch.no_grad():
        x = h2.reshape(rows, width).contiguous()
        logits = router.router_logits(x, router_weight)
        forced = next_override(rows, experts, top_k, x.device)
        bias = None if router_bias is None or router_bias.numel() == 0 else router_bias
        weights, ids = kernels.router_topk(
            logits, int(top_k), routing_mode, bias=bias, n_group=int(n_group),
            topk_group=int(topk_group), routed_scaling=float(routed_scaling), forced_ids=forced,
        )
        counts, offsets, order, slots = kernels.permute_plan(ids, experts)
        # Block-FP8 w13 is stored gate rows then up rows and the GEMM
        # interleaves its output; an fp8_current w13 is stored interleaved.
        if getattr(w13, "current", False):
            xq, xs = _rows(x, slots, w13)
            h13 = _forward_gemm(xq, xs, w13, offsets, interleave=True)
        else:
            h13 = fused.routed_rows_gemm(x, slots, order, int(top_k), w13, offsets,
                                         interleave=True)
        aux, probability_sum, _, _ = kernels.router_stats(logits, ids, int(top_k), routing_mode,
                                                          lengths)
    return aux, counts, probability_sum, logits, weights, ids, order, offsets, slots, h13


def finish_forward(h13, w2, route_weights, offsets, slots, residual, *, swiglu_limit=None):
    """``residual + combine(down(swiglu(h13)))`` (reference ``builtin/moe_composed.py:190-208``)."""
    width = residual.shape[-1]
    with torch.no_grad():
        base = residual.reshape(-1, width).contiguous()
        if getattr(w2, "current", False):
            aq, as_ = kernels.swiglu_quantize_rows_current(h13, swiglu_limit)
        else:
            aq, as_ = kernels.swiglu_quantize(h13, swiglu_limit)
        y = _forward_gemm(aq, as_, w2, offsets)
        return kernels.combine(y, slots, route_weights, base).reshape(residual.shape)


def finish_backward(grad_output, h13, w2, route_weights, order, offsets, slots, *, top_k,
                    weight_grad_dtype=None, need_w2=True, swiglu_limit=None, grad_h13_out=None):
    """``(grad_h13, grad_w2, grad_route_weights, grad_residual)`` (reference
    ``builtin/moe_composed.py:211-251``). ``grad_h13`` is bf16 in ``h13``'s
    interleaved layout. It is written into ``grad_h13_out`` when given, which
    may be ``h13`` itself: each lane of the SwiGLU backward reads its h values
    before it writes their gradients."""
    expert_dtype, direct, _ = _grad_dtypes(weight_grad_dtype)
    width = grad_output.shape[-1]
    assignments = order.numel()
    experts = offsets.numel() - 1
    with torch.no_grad():
        dy = grad_output.reshape(-1, width).contiguous()
        if dy.dtype != torch.bfloat16:
            dy = dy.to(torch.bfloat16)
        if getattr(w2, "current", False):
            dyq, dys = _rows(dy, slots, w2)
            r = _input_gradient_gemm(dyq, dys, w2, offsets)
        else:
            r = fused.routed_rows_gemm(dy, slots, order, int(top_k), w2, offsets,
                                       input_gradient=True)
        grad_h13, a_prime, dscore = kernels.routed_swiglu_backward(
            r, h13, route_weights.reshape(-1), order, swiglu_limit, dh_out=grad_h13_out)
        grad_route_weights = dscore[slots.reshape(-1).long()].view(route_weights.shape)
        if grad_route_weights.dtype != route_weights.dtype:
            grad_route_weights = grad_route_weights.to(route_weights.dtype)
        if need_w2:
            padded = kernels.wgrad_padded_rows(assignments, experts)
            blocks = kernels.padded_row_blocks(offsets, padded)
            dy_t, dy_ts, _ = kernels.quantize_transpose(
                dy, offsets, assignments, gather=order, gather_div=int(top_k), padded=padded,
                row_blocks=blocks)
            ap_t, ap_ts, _ = kernels.quantize_transpose(
                a_prime, offsets, assignments, padded=padded, row_blocks=blocks)
            grad_w2 = fused._grad_at(
                kernels.wgrad(dy_t, dy_ts, ap_t, ap_ts, offsets, out_dtype=direct,
                              rows=assignments), expert_dtype)
        else:
            grad_w2 = fused.skipped_gradient(h13, expert_dtype)
    return grad_h13, grad_w2, grad_route_weights, grad_output.clone()


def prepare_backward(grad_aux, grad_probability_sum, grad_route_weights, grad_h13, h2,
                     router_weight, w13, logits, route_weights, route_ids, order, offsets, slots,
                     *, top_k, routing_mode, lengths, weight_grad_dtype=None, need_router=True,
                     need_w13=True):
    """``(grad_h2, grad_router, grad_w13)`` (reference ``builtin/moe_composed.py:120-187``)."""
    expert_dtype, direct, router_dtype = _grad_dtypes(weight_grad_dtype, router_weight)
    width = h2.shape[-1]
    rows = h2.numel() // width
    lengths = fused._normalized(lengths, rows)
    assignments = order.numel()
    experts = offsets.numel() - 1
    with torch.no_grad():
        x = h2.reshape(rows, width).contiguous()
        if grad_h13.dtype != torch.bfloat16:
            grad_h13 = grad_h13.to(torch.bfloat16)
        grad_h13 = grad_h13.contiguous()
        if getattr(w13, "current", False):
            # The interleaved K order of the transposed w13 copy is h13's.
            dhq, dhs = kernels.quantize_rows_current(grad_h13)
        else:
            dhq, dhs = kernels.quantize_rows(grad_h13, gate_up=True)
        dx = _input_gradient_gemm(dhq, dhs, w13, offsets)
        if need_w13:
            padded = kernels.wgrad_padded_rows(assignments, experts)
            blocks = kernels.padded_row_blocks(offsets, padded)
            dh_t, dh_ts, _ = kernels.quantize_transpose(
                grad_h13, offsets, assignments, gate_up=True, padded=padded, row_blocks=blocks)
            x_t, x_ts, _ = kernels.quantize_transpose(
                x, offsets, assignments, gather=order, gather_div=int(top_k), padded=padded,
                row_blocks=blocks)
            grad_w13 = fused._grad_at(
                kernels.wgrad(dh_t, dh_ts, x_t, x_ts, offsets, out_dtype=direct,
                              rows=assignments), expert_dtype)
        else:
            grad_w13 = fused.skipped_gradient(h2, expert_dtype)
        grad_h2 = kernels.unpermute_sum(dx, slots)
        # The score cotangent per sorted row, as the fused backward computes it.
        dscore = torch.empty(assignments, dtype=torch.float32, device=h2.device)
        dscore[slots.reshape(-1).long()] = grad_route_weights.reshape(-1).float()
        grad_router = fused.routing_backward(
            grad_h2, x, router_weight, logits, route_weights, route_ids, dscore, slots, offsets,
            grad_aux, grad_probability_sum, top_k=top_k, routing_mode=routing_mode,
            lengths=lengths, router_dtype=router_dtype, need_router=need_router,
        )
    return grad_h2.reshape(h2.shape).to(h2.dtype), grad_router, grad_w13


# --------------------------------------------------------------------------
# Operators. Weights travel as their e4m3 data plus a components list (the
# scale, then the transposed data when the per-call quantizer made it).
@torch.library.custom_op("mlops_mi355x::moe_mi355x_prepare_fwd", mutates_args=())
def _prepare_op(
    h2: torch.Tensor, router_weight: torch.Tensor, w13_experts: torch.Tensor,
    router_bias: torch.Tensor, top_k: int, routing_mode: str, n_group: int, topk_group: int,
    routed_scaling: float, lengths: list[int], weight_precision: str,
    weight_grad_dtype: torch.dtype | None, weight_components: list[torch.Tensor],
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor,
           torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    del weight_precision, weight_grad_dtype
    return prepare_forward(
        h2, router_weight, _weight(w13_experts, weight_components), top_k=top_k,
        routing_mode=routing_mode, router_bias=router_bias, n_group=n_group,
        topk_group=topk_group, routed_scaling=routed_scaling, lengths=lengths,
    )


@_prepare_op.register_fake
def _prepare_fake(h2, router_weight, w13_experts, router_bias, top_k, routing_mode, n_group,
                  topk_group, routed_scaling, lengths, weight_precision, weight_grad_dtype,
                  weight_components):
    rows = h2.numel() // h2.shape[-1]
    experts = router_weight.shape[0]
    assignments = rows * int(top_k)
    device = h2.device
    return (
        torch.empty((), dtype=torch.float32, device=device),
        torch.empty(experts, dtype=torch.int64, device=device),
        torch.empty(experts, dtype=torch.float32, device=device),
        torch.empty((rows, experts), dtype=torch.float32, device=device),
        torch.empty((rows, int(top_k)), dtype=torch.float32, device=device),
        torch.empty((rows, int(top_k)), dtype=torch.int32, device=device),
        torch.empty(assignments, dtype=torch.int32, device=device),
        torch.empty(experts + 1, dtype=torch.int32, device=device),
        torch.empty((rows, int(top_k)), dtype=torch.int32, device=device),
        torch.empty((assignments, w13_experts.shape[1]), dtype=h2.dtype, device=device),
    )


@torch.library.custom_op("mlops_mi355x::moe_mi355x_prepare_bwd", mutates_args=())
def _prepare_backward_op(
    grad_aux: torch.Tensor, grad_probability_sum: torch.Tensor,
    grad_route_weights: torch.Tensor, grad_h13: torch.Tensor, h2: torch.Tensor,
    router_weight: torch.Tensor, w13_experts: torch.Tensor, logits: torch.Tensor,
    route_weights: torch.Tensor, route_ids: torch.Tensor, order: torch.Tensor,
    offsets: torch.Tensor, slots: torch.Tensor, top_k: int, routing_mode: str,
    lengths: list[int], weight_grad_dtype: torch.dtype | None,
    weight_components: list[torch.Tensor], need_router: bool, need_w13: bool,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    return prepare_backward(
        grad_aux, grad_probability_sum, grad_route_weights, grad_h13, h2, router_weight,
        _weight(w13_experts, weight_components), logits, route_weights, route_ids, order,
        offsets, slots, top_k=top_k, routing_mode=routing_mode, lengths=lengths,
        weight_grad_dtype=weight_grad_dtype, need_router=need_router, need_w13=need_w13,
    )


@_prepare_backward_op.register_fake
def _prepare_backward_fake(grad_aux, grad_probability_sum, grad_route_weights, grad_h13, h2,
                           router_weight, w13_experts, logits, route_weights, route_ids, order,
                           offsets, slots, top_k, routing_mode, lengths, weight_grad_dtype,
                           weight_components, need_router, need_w13):
    expert_dtype, _, router_dtype = _grad_dtypes(weight_grad_dtype, router_weight)
    return (
        torch.empty_like(h2),
        torch.empty(router_weight.shape, dtype=router_dtype, device=h2.device)
        if need_router else fused.skipped_gradient(router_weight, router_dtype),
        torch.empty(w13_experts.shape, dtype=expert_dtype, device=h2.device)
        if need_w13 else fused.skipped_gradient(h2, expert_dtype),
    )


@torch.library.custom_op("mlops_mi355x::moe_mi355x_finish_fwd", mutates_args=())
def _finish_op(
    h13: torch.Tensor, w2_experts: torch.Tensor, route_weights: torch.Tensor,
    order: torch.Tensor, offsets: torch.Tensor, slots: torch.Tensor, residual: torch.Tensor,
    top_k: int, weight_grad_dtype: torch.dtype | None, swiglu_limit: float | None,
    weight_components: list[torch.Tensor],
) -> torch.Tensor:
    del order, top_k, weight_grad_dtype
    return finish_forward(h13, _weight(w2_experts, weight_components), route_weights, offsets,
                          slots, residual, swiglu_limit=swiglu_limit)


@_finish_op.register_fake
def _finish_fake(h13, w2_experts, route_weights, order, offsets, slots, residual, top_k,
                 weight_grad_dtype, swiglu_limit, weight_components):
    return torch.empty_like(residual)


@torch.library.custom_op("mlops_mi355x::moe_mi355x_finish_bwd", mutates_args=())
def _finish_backward_op(
    grad_output: torch.Tensor, h13: torch.Tensor, w2_experts: torch.Tensor,
    route_weights: torch.Tensor, order: torch.Tensor, offsets: torch.Tensor,
    slots: torch.Tensor, top_k: int, weight_grad_dtype: torch.dtype | None,
    swiglu_limit: float | None, weight_components: list[torch.Tensor], need_w2: bool,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    return finish_backward(
        grad_output, h13, _weight(w2_experts, weight_components), route_weights, order, offsets,
        slots, top_k=top_k, weight_grad_dtype=weight_grad_dtype, need_w2=need_w2,
        swiglu_limit=swiglu_limit,
    )


def _finish_backward_outputs(grad_output, h13, w2_experts, route_weights, weight_grad_dtype,
                             need_w2):
    expert_dtype, _, _ = _grad_dtypes(weight_grad_dtype)
    return (
        torch.empty(w2_experts.shape, dtype=expert_dtype, device=h13.device)
        if need_w2 else fused.skipped_gradient(h13, expert_dtype),
        torch.empty_like(route_weights),
        torch.empty_like(grad_output),
    )


@_finish_backward_op.register_fake
def _finish_backward_fake(grad_output, h13, w2_experts, route_weights, order, offsets, slots,
                          top_k, weight_grad_dtype, swiglu_limit, weight_components, need_w2):
    return (torch.empty_like(h13), *_finish_backward_outputs(
        grad_output, h13, w2_experts, route_weights, weight_grad_dtype, need_w2))


@torch.library.custom_op("mlops_mi355x::moe_mi355x_finish_bwd_donate_h13",
                         mutates_args=("h13",))
def _finish_backward_donate_h13_op(
    grad_output: torch.Tensor, h13: torch.Tensor, w2_experts: torch.Tensor,
    route_weights: torch.Tensor, order: torch.Tensor, offsets: torch.Tensor,
    slots: torch.Tensor, top_k: int, weight_grad_dtype: torch.dtype | None,
    swiglu_limit: float | None, weight_components: list[torch.Tensor], need_w2: bool,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """The finish VJP writing ``grad_h13`` over a dead ``h13`` (reference
    ``builtin/moe_composed.py:671-713``): for a caller that has proven ``h13``
    has no later reader. Returns the other three results; ``h13`` then holds
    ``grad_h13``. The functional operator above stays the autograd one."""
    _, grad_w2, grad_route_weights, grad_residual = finish_backward(
        grad_output, h13, _weight(w2_experts, weight_components), route_weights, order, offsets,
        slots, top_k=top_k, weight_grad_dtype=weight_grad_dtype, need_w2=need_w2,
        swiglu_limit=swiglu_limit, grad_h13_out=h13,
    )
    return grad_w2, grad_route_weights, grad_residual


@_finish_backward_donate_h13_op.register_fake
def _finish_backward_donate_h13_fake(grad_output, h13, w2_experts, route_weights, order,
                                     offsets, slots, top_k, weight_grad_dtype, swiglu_limit,
                                     weight_components, need_w2):
    return _finish_backward_outputs(grad_output, h13, w2_experts, route_weights,
                                    weight_grad_dtype, need_w2)


@flop_formula(_prepare_op)
def _prepare_flops(h2, router_weight, w13_experts, router_bias, top_k, *_rest, out_val=None,
                   **_kwargs):
    rows = h2.numel() // h2.shape[-1]
    return logical.moe_prepare_flops(rows, h2.shape[-1], router_weight.shape[0],
                                     rows * int(top_k), w13_experts.shape[1], forward=True)


@flop_formula(_prepare_backward_op)
def _prepare_backward_flops(grad_aux, grad_probability_sum, grad_route_weights, grad_h13, h2,
                            router_weight, w13_experts, *_rest, out_val=None, **_kwargs):
    rows = h2.numel() // h2.shape[-1]
    return logical.moe_prepare_flops(rows, h2.shape[-1], router_weight.shape[0],
                                     grad_h13.shape[0], w13_experts.shape[1], forward=False)


@flop_formula(_finish_op)
def _finish_flops(h13, w2_experts, *_rest, out_val=None, **_kwargs):
    return logical.moe_finish_flops(h13.shape[0], w2_experts.shape[2], w2_experts.shape[1],
                                    forward=True)


@flop_formula(_finish_backward_op)
def _finish_backward_flops(grad_output, h13, w2_experts, *_rest, out_val=None, **_kwargs):
    return logical.moe_finish_flops(h13.shape[0], w2_experts.shape[2], w2_experts.shape[1],
                                    forward=False)


def _container_rule(cls, func, types, args, kwargs):
    """Unwraps the one container argument to its data, appending its
    scale and, for the backward operators and wherever the per-call quantizer
    carried it, its transposed data to the ``weight_components`` argument."""
    del cls, types
    if kwargs:
        raise ValueError("use positional operator arguments")
    args = list(args)
    slot = [a.name for a in func._schema.arguments].index("weight_components")
    components = list(args[slot])
    backward = func in (torch.ops.mlops_mi355x.moe_mi355x_prepare_bwd.default,
                        torch.ops.mlops_mi355x.moe_mi355x_finish_bwd.default,
                        torch.ops.mlops_mi355x.moe_mi355x_finish_bwd_donate_h13.default)
    for index, value in enumerate(args):
        block, row = block_parts(value), row_parts(value)
        if block is not None:
            args[index] = block[0]
            components.append(block[1])
            transposed = (fused.available_transposed(value) if backward
                          else getattr(value, "_transposed", None))
            if transposed is not None:
                components.append(transposed)
        elif row is not None:
            args[index] = row[0]
            components.extend(row[1:])
    args[slot] = components
    return func(*args)


OPERATORS = (_prepare_op, _prepare_backward_op, _finish_op, _finish_backward_op,
             _finish_backward_donate_h13_op)
for _cls in (BlockFP8Weight, RowFP8Weight):
    register_container_class(OPERATORS, _container_rule, _cls)


def _prepare_context(ctx, inputs, output):
    (h2, router_weight, w13, _bias, top_k, routing_mode, _n_group, _topk_group, _scaling,
     lengths, _precision, weight_grad_dtype, components) = inputs
    (_aux, counts, _psum, logits, route_weights, route_ids, order, offsets, slots, _h13) = output
    ctx.save_for_backward(h2, router_weight, w13, logits, route_weights, route_ids, order,
                          offsets, slots, *components)
    ctx.top_k = int(top_k)
    ctx.routing_mode = routing_mode
    ctx.lengths = list(lengths)
    ctx.weight_grad_dtype = weight_grad_dtype
    ctx.set_materialize_grads(False)
    ctx.mark_non_differentiable(counts, logits, route_ids, order, offsets, slots)


def _prepare_autograd_backward(ctx, grad_aux, _g_counts, grad_probability_sum, _g_logits,
                               grad_route_weights, _g_ids, _g_order, _g_offsets, _g_slots,
                               grad_h13):
    saved = ctx.saved_tensors
    residuals, components = saved[:9], list(saved[9:])
    h2, router_weight, w13 = residuals[:3]
    route_weights, order = residuals[4], residuals[6]
    device = h2.device
    if grad_aux is None:
        grad_aux = torch.zeros((), dtype=torch.float32, device=device)
    if grad_probability_sum is None:
        grad_probability_sum = torch.zeros(router_weight.shape[0], dtype=torch.float32,
                                           device=device)
    if grad_route_weights is None:
        grad_route_weights = torch.zeros_like(route_weights)
    if grad_h13 is None:
        grad_h13 = torch.zeros((order.numel(), w13.shape[1]), dtype=h2.dtype, device=device)
    needs = ctx.needs_input_grad
    grad_h2, grad_router, grad_w13 = _prepare_backward_op(
        grad_aux, grad_probability_sum, grad_route_weights.contiguous(), grad_h13.contiguous(),
        *residuals, ctx.top_k, ctx.routing_mode, ctx.lengths, ctx.weight_grad_dtype, components,
        bool(needs[1]), bool(needs[2]),
    )
    return (grad_h2, grad_router if needs[1] else None, grad_w13 if needs[2] else None,
            *([None] * 9), [None] * len(components))


_prepare_op.register_autograd(_prepare_autograd_backward, setup_context=_prepare_context)


def _finish_context(ctx, inputs, output):
    del output
    (h13, w2, route_weights, order, offsets, slots, _residual, top_k, weight_grad_dtype,
     swiglu_limit, components) = inputs
    ctx.save_for_backward(h13, w2, route_weights, order, offsets, slots, *components)
    ctx.top_k = int(top_k)
    ctx.weight_grad_dtype = weight_grad_dtype
    ctx.swiglu_limit = swiglu_limit


def _finish_autograd_backward(ctx, grad_output):
    saved = ctx.saved_tensors
    residuals, components = saved[:6], list(saved[6:])
    needs = ctx.needs_input_grad
    grad_h13, grad_w2, grad_route_weights, grad_residual = _finish_backward_op(
        grad_output.contiguous(), *residuals, ctx.top_k, ctx.weight_grad_dtype,
        ctx.swiglu_limit, components, bool(needs[1]),
    )
    return (grad_h13, grad_w2 if needs[1] else None, grad_route_weights, None, None, None,
            grad_residual, None, None, None, [None] * len(components))


_finish_op.register_autograd(_finish_autograd_backward, setup_context=_finish_context)


def apply(
    h2, residual, router_weight, w13_experts, w2_experts, *, top_k, routing_mode,
    router_bias=None, n_group=1, topk_group=1, routed_scaling=1.0, lengths=None,
    shared_w13=None, shared_w2=None, shared_gate_weight=None, shared_mode="add",
    compute_precision=None, swiglu_limit=None,
):
    """``(out, aux, counts, probability_sum)`` through the two regions (reference
    ``sonicmoe/moe_composed.py:751-834``)."""
    rules = current if _is_current(compute_precision, w13_experts, w2_experts) else fused
    _, refusal = rules._precision(compute_precision, w13_experts, w2_experts)
    if refusal is not None:
        raise ValueError(refusal)
    w13, w2 = rules._containers(w13_experts, w2_experts)
    route_containers(OPERATORS, _container_rule, w13, w2)
    rows = h2.numel() // h2.shape[-1]
    normalized = (rows,) if lengths is None else tuple(int(x) for x in lengths)
    bias = (torch.empty(0, dtype=torch.float32, device=h2.device) if router_bias is None
            else router_bias)
    base = fused._shared_base(h2, residual, shared_w13, shared_w2, shared_gate_weight,
                              shared_mode, swiglu_limit)
    grad_dtype = weight_gradient_dtype()
    limit = None if swiglu_limit is None else float(swiglu_limit)
    (aux, counts, probability_sum, _logits, route_weights, _ids, order, offsets, slots,
     h13) = _prepare_op(
        h2, router_weight, w13, bias, int(top_k), str(routing_mode), int(n_group),
        int(topk_group), float(routed_scaling), list(normalized),
        current_route_weight_precision(), grad_dtype, [],
    )
    output = _finish_op(h13, w2, route_weights, order, offsets, slots, base, int(top_k),
                        grad_dtype, limit, [])
    return output, aux, counts, probability_sum


IMPLEMENTATION = register_implementation(
    Implementation(
        operation="moe",
        implementation_id=IMPLEMENTATION_ID,
        provider="mi355x",
        priority=PRIORITY,
        deterministic=True,
        supports=_supports,
        apply=apply,
    )
)

__all__ = [
    "IMPLEMENTATION",
    "apply",
    "finish_backward",
    "finish_forward",
    "prepare_backward",
    "prepare_forward",
]
