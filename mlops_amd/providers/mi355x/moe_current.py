"""``mi355x.moe.fp8_current``: the routed MoE at ``compute_precision="fp8_current"``.

The reference serves this precision on its SonicMoE provider
(``src/mlops/providers/sonicmoe/fp8.py:1-458``, ``sonicmoe/moe.py:169-431``).
Expert weights are `RowFP8Weight` containers (the reference's
``QuackFP8Weight``), or bf16/fp32 masters quantized per call. Every operand
of the expert GEMMs carries one descale per row:

* forward: each token's row quantized once (from top_k 4 read by the GEMM
  through the routed rows' tokens, ``mi355x_gemm_fp8_rowwise_gathered``;
  below, written to its routed slots, ``mi355x_permute_quantize_current_fp8``);
  the up GEMM against the
  gate/up-adjacent rows of ``w13`` writes ``h13`` interleaved; SwiGLU and
  its per-row quantization in one pass; the down GEMM; combine;
* backward: the gathered cotangent quantized per row, then ``r = dy @ W2``
  through the transposed copy; the routed SwiGLU backward (``dh`` interleaved,
  ``a'``, the score gradient); ``dh`` quantized per row, then ``dx = dh @ W13``
  through the transposed copy, whose K order is the same interleaving;
* the GEMMs are ``mi355x_gemm_fp8_rowwise``: the K loop accumulates in the
  MFMA, and the epilogue applies ``(acc * row descale) * column descale``
  once. The block-scaled form instead folds scales at every 128-deep K step;
* weight gradients, as in the block-FP8 operator, come from the
  feature-major e4m3 transposes and the e4m3 weight-gradient GEMM. The
  reference computes them in bf16 here (sonicmoe/moe.py:346-358, 408-419).
  ``dW13`` comes back in nn.Linear (gate-then-up) row order.

Where the reference's fused up-projection epilogue activates the fp32
product, this path activates the stored bf16 ``h13``, as the reference's
composed form does (``fp8.project_down_from_preactivation``).
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
from ...weight_formats import (is_block_fp8, is_row_fp8, register_container_class,
                               route_containers, row_interleaved, row_parts)
from . import moe as fused

IMPLEMENTATION_ID = "mi355x.moe.fp8_current"
PRIORITY = 120
GEMM_ALIGN = 256  # every N of the four row-scaled GEMMs (2I, H, I, H)


def _precision(compute_precision, w13, w2):
    """``"fp8_current"`` when this implementation serves the request, else a refusal."""
    weights = (w13, w2)
    if any(is_block_fp8(w) for w in weights):
        return None, "block-FP8 (BlockFP8Weight) weights compute at fp8_block"
    if compute_precision == "fp8_current":
        return "fp8_current", None
    if compute_precision is None and any(is_row_fp8(w) for w in weights):
        return "fp8_current", None
    return None, f"compute_precision={compute_precision!r} is not fp8_current"


def supports(h2, residual, router_weight, w13_experts, w2_experts, *, surface, top_k,
             routing_mode, compute_precision=None, **kwargs) -> SupportResult:
    """Metadata-only checks: the block-FP8 operator's shape and routing rules,
    this precision's containers, and widths the row-scaled GEMM tiles."""
    _, refusal = _precision(compute_precision, w13_experts, w2_experts)
    if refusal is not None:
        return SupportResult.no(refusal)
    if is_row_fp8(w13_experts) and not row_interleaved(w13_experts):
        return SupportResult.no(
            "an FP8 w13 must be quantized with interleaved=True (gate/up rows adjacent)")
    del surface
    common = fused.check_shapes(
        h2, residual, router_weight, w13_experts, w2_experts, top_k=top_k,
        routing_mode=routing_mode, **{k: kwargs[k] for k in (
            "router_bias", "n_group", "topk_group", "lengths", "shared_w13", "shared_w2")
            if k in kwargs})
    if not common:
        return common
    if h2.shape[-1] % GEMM_ALIGN or w2_experts.shape[2] % GEMM_ALIGN:
        return SupportResult.no(
            f"fp8_current on the MI355X needs model and expert widths that are multiples of "
            f"{GEMM_ALIGN}")
    return SupportResult.yes()


# --------------------------------------------------------------------------
# The routed math on plain tensors; a weight is (data, transposed, scale,
# transposed_scale).
def forward_routed(h2, residual, router_weight, w13, w2, *, top_k, routing_mode,
                   router_bias=None, n_group=1, topk_group=1, routed_scaling=1.0, lengths=None,
                   swiglu_limit=None):
    """``(output, aux, counts, probability_sum, logits, route_weights, route_ids,
    order, offsets, slots, h13)``, ``h13`` interleaved (sonicmoe/moe.py:441-514)."""
    width = h2.shape[-1]
    rows = h2.numel() // width
    lengths = fused._normalized((rows,) if lengths is None else lengths, rows)
    experts = router_weight.shape[0]
    with torch.no_grad():
        x = h2.reshape(rows, width).contiguous()
        base = residual.reshape(rows, width).contiguous()
        logits = router.router_logits(x, router_weight)
        forced = next_override(rows, experts, top_k, x.device)
        bias = None if router_bias is None or router_bias.numel() == 0 else router_bias
        weights, ids = kernels.router_topk(
            logits, int(top_k), routing_mode, bias=bias, n_group=int(n_group),
            topk_group=int(topk_group), routed_scaling=float(routed_scaling), forced_ids=forced,
        )
        counts, offsets, order, slots = kernels.permute_plan(ids, experts)
        h13 = _routed_rows_gemm(x, slots, order, int(top_k), w13[0], w13[2], offsets)
        aq, as_ = kernels.swiglu_quantize_rows_current(h13, swiglu_limit)
        y = kernels.gemm_rowwise(aq, as_, w2[0], w2[2], offsets)
        output = kernels.combine(y, slots, weights, base)
        aux, probability_sum, _, _ = kernels.router_stats(logits, ids, int(top_k), routing_mode,
                                                          lengths)
    return (output.reshape(h2.shape), aux, counts, probability_sum, logits, weights, ids, order,
            offsets, slots, h13)


def _routed_rows_gemm(x, slots, order, top_k, data, scale, offsets):
    """The row-scaled GEMM on the routed rows of token rows ``x``: from
    ``GATHER_MIN_TOP_K`` routed rows per token, on the token rows quantized
    once (``mi355x_gemm_fp8_rowwise_gathered``), else on the permuted copy.
    Bitwise the same either way."""
    if top_k >= fused.GATHER_MIN_TOP_K and data.shape[1] % 256 == 0:
        tq, ts = kernels.quantize_rows_current(x)
        # Routed row r reads token order[r] // top_k, divided in the kernel.
        return kernels.gemm_rowwise_gathered(tq, ts, order, data, scale, offsets,
                                             rows_div=top_k)
    xq, xs = kernels.permute_quantize_current(x, slots)
    return kernels.gemm_rowwise(xq, xs, data, scale, offsets)


def backward_routed(grad_output, grad_aux, grad_probability_sum, h2, router_weight, w13, w2,
                    logits, route_weights, route_ids, order, offsets, slots, h13, *, top_k,
                    routing_mode, lengths, weight_grad_dtype=None, swiglu_limit=None,
                    need_router=True, need_w13=True, need_w2=True, need_residual=True):
    """VJPs ``(h2, residual, router_weight, w13, w2)`` (sonicmoe/moe.py:517-620);
    the expert weights' at ``weight_grad_dtype`` (bf16 when None) in nn.Linear
    row order, the router's at ``weight_grad_dtype`` (its own dtype when None)."""
    width = h2.shape[-1]
    rows = h2.numel() // width
    lengths = fused._normalized(lengths, rows)
    experts = router_weight.shape[0]
    assignments = order.numel()
    router_dtype = router_weight.dtype if weight_grad_dtype is None else weight_grad_dtype
    expert_dtype = torch.bfloat16 if weight_grad_dtype is None else weight_grad_dtype
    direct = expert_dtype if expert_dtype in (torch.bfloat16, torch.float32) else torch.float32
    with torch.no_grad():
        x = h2.reshape(rows, width).contiguous()
        dy = grad_output.reshape(rows, width).contiguous()
        if dy.dtype != torch.bfloat16:
            dy = dy.to(torch.bfloat16)
        r = _routed_rows_gemm(dy, slots, order, int(top_k), w2[1], w2[3], offsets)
        if need_w2 or need_w13:
            # One pass for bf16 dh and the transposed dh and a' of the weight
            # gradients (equal to the SwiGLU backward then quantize_transpose).
            padded = kernels.wgrad_padded_rows(assignments, experts)
            blocks = kernels.padded_row_blocks(offsets, padded)
            dh, dh_t, dh_ts, ap_t, ap_ts, dscore = kernels.swiglu_bwd_bf16(
                r, h13, route_weights.reshape(-1), order, offsets, padded=padded,
                row_blocks=blocks, limit=swiglu_limit, transposed_dh=need_w13,
                transposed_ap=need_w2)
        else:
            dh, _, dscore = kernels.routed_swiglu_backward(
                r, h13, route_weights.reshape(-1), order, swiglu_limit)
        if need_w2:
            dy_t, dy_ts, _ = kernels.quantize_transpose(
                dy, offsets, assignments, gather=order, gather_div=int(top_k), padded=padded,
                row_blocks=blocks)
            grad_w2 = fused._grad_at(
                kernels.wgrad(dy_t, dy_ts, ap_t, ap_ts, offsets, out_dtype=direct,
                              rows=assignments), expert_dtype)
        else:
            grad_w2 = fused.skipped_gradient(h2, expert_dtype)
        dhq, dhs = kernels.quantize_rows_current(dh)
        dx = kernels.gemm_rowwise(dhq, dhs, w13[1], w13[3], offsets)
        if need_w13:
            x_t, x_ts, _ = kernels.quantize_transpose(
                x, offsets, assignments, gather=order, gather_div=int(top_k), padded=padded,
                row_blocks=blocks)
            grad_w13 = fused._grad_at(
                kernels.wgrad(dh_t, dh_ts, x_t, x_ts, offsets, out_dtype=direct,
                              rows=assignments), expert_dtype)
        else:
            grad_w13 = fused.skipped_gradient(h2, expert_dtype)
        grad_h2 = kernels.unpermute_sum(dx, slots)
        grad_router = fused.routing_backward(
            grad_h2, x, router_weight, logits, route_weights, route_ids, dscore, slots, offsets,
            grad_aux, grad_probability_sum, top_k=top_k, routing_mode=routing_mode,
            lengths=lengths, router_dtype=router_dtype, need_router=need_router,
        )
    grad_residual = grad_output.clone() if need_residual else grad_output.new_empty(0)
    return (grad_h2.reshape(h2.shape).to(h2.dtype), grad_residual, grad_router, grad_w13, grad_w2)


def _split(w13, w2, components):
    """Each weight's data with its three further components, in weight order."""
    if len(components) != 6:
        raise ValueError("the fp8_current operators take three further components per weight "
                         "(transposed, scale, transposed_scale)")
    return (w13, *components[:3]), (w2, *components[3:])


# --------------------------------------------------------------------------
@torch.library.custom_op("mlops_mi355x::moe_mi355x_fp8_current_fwd", mutates_args=())
def _forward_op(
    h2: torch.Tensor, residual: torch.Tensor, router_weight: torch.Tensor,
    w13_experts: torch.Tensor, w2_experts: torch.Tensor, router_bias: torch.Tensor,
    top_k: int, routing_mode: str, n_group: int, topk_group: int, routed_scaling: float,
    lengths: list[int], weight_precision: str, weight_grad_dtype: torch.dtype | None,
    swiglu_limit: float | None, weight_components: list[torch.Tensor],
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor,
           torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    del weight_precision, weight_grad_dtype
    w13, w2 = _split(w13_experts, w2_experts, weight_components)
    return forward_routed(
        h2, residual, router_weight, w13, w2, top_k=top_k, routing_mode=routing_mode,
        router_bias=router_bias, n_group=n_group, topk_group=topk_group,
        routed_scaling=routed_scaling, lengths=lengths, swiglu_limit=swiglu_limit,
    )


@_forward_op.register_fake
def _forward_fake(h2, residual, router_weight, w13_experts, w2_experts, router_bias, top_k,
                  routing_mode, n_group, topk_group, routed_scaling, lengths, weight_precision,
                  weight_grad_dtype, swiglu_limit, weight_components):
    return fused._forward_fake(h2, residual, router_weight, w13_experts, w2_experts, router_bias,
                               top_k, routing_mode, n_group, topk_group, routed_scaling, lengths,
                               weight_precision, weight_grad_dtype, swiglu_limit,
                               weight_components)


@torch.library.custom_op("mlops_mi355x::moe_mi355x_fp8_current_bwd", mutates_args=())
def _backward_op(
    grad_output: torch.Tensor, grad_aux: torch.Tensor, grad_probability_sum: torch.Tensor,
    h2: torch.Tensor, router_weight: torch.Tensor, w13_experts: torch.Tensor,
    w2_experts: torch.Tensor, logits: torch.Tensor, route_weights: torch.Tensor,
    route_ids: torch.Tensor, order: torch.Tensor, offsets: torch.Tensor, slots: torch.Tensor,
    h13: torch.Tensor, top_k: int, routing_mode: str, lengths: list[int],
    weight_grad_dtype: torch.dtype | None, swiglu_limit: float | None, need_router: bool,
    need_w13: bool, need_w2: bool, need_residual: bool,
    weight_components: list[torch.Tensor],
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    w13, w2 = _split(w13_experts, w2_experts, weight_components)
    return backward_routed(
        grad_output, grad_aux, grad_probability_sum, h2, router_weight, w13, w2, logits,
        route_weights, route_ids, order, offsets, slots, h13, top_k=top_k,
        routing_mode=routing_mode, lengths=lengths, weight_grad_dtype=weight_grad_dtype,
        swiglu_limit=swiglu_limit, need_router=need_router, need_w13=need_w13, need_w2=need_w2,
        need_residual=need_residual,
    )


@_backward_op.register_fake
def _backward_fake(grad_output, grad_aux, grad_probability_sum, h2, router_weight, w13_experts,
                   w2_experts, logits, route_weights, route_ids, order, offsets, slots, h13,
                   top_k, routing_mode, lengths, weight_grad_dtype, swiglu_limit, need_router,
                   need_w13, need_w2, need_residual, weight_components):
    return fused._backward_fake(grad_output, grad_aux, grad_probability_sum, h2, router_weight,
                                w13_experts, w2_experts, logits, route_weights, route_ids, order,
                                offsets, slots, h13, top_k, routing_mode, lengths,
                                weight_grad_dtype, swiglu_limit, need_router, need_w13, need_w2,
                                need_residual, weight_components)


@flop_formula(_forward_op)
def _forward_flops(h2, residual, router_weight, w13_experts, w2_experts, router_bias, top_k,
                   *_rest, out_val=None, **_kwargs):
    return logical.moe_flops(h2, router_weight, w13_experts, w2_experts, top_k, forward=True)


@flop_formula(_backward_op)
def _backward_flops(grad_output, grad_aux, grad_probability_sum, h2, router_weight, w13_experts,
                    w2_experts, logits, route_weights, route_ids, order, offsets, slots, h13,
                    top_k, *_rest, out_val=None, **_kwargs):
    return logical.moe_flops(h2, router_weight, w13_experts, w2_experts, top_k, forward=False)


def _container_rule(cls, func, types, args, kwargs):
    """Each row-FP8 container argument becomes its e4m3 rows; its transposed copy
    and the two descale vectors fill ``weight_components``, in weight order
    (reference ``sonicmoe/fp8.py:223-256``)."""
    del cls, types
    if kwargs:
        raise ValueError("use positional operator arguments")
    args = list(args)
    slot = [a.name for a in func._schema.arguments].index("weight_components")
    components = list(args[slot])
    for index, value in enumerate(args):
        parts = row_parts(value)
        if parts is not None:
            args[index] = parts[0]
            components.extend(parts[1:])
    args[slot] = components
    return func(*args)


OPERATORS = (_forward_op, _backward_op)
register_container_class(OPERATORS, _container_rule, RowFP8Weight)


def _setup_context(ctx, inputs, output):
    fused._setup_context(ctx, inputs, output)


def _autograd_backward(ctx, grad_output, grad_aux, _g_counts, grad_probability_sum, *_unused):
    saved = ctx.saved_tensors
    h2, router_weight = saved[:2]
    components = list(saved[11:])
    # An absent cotangent travels as an empty tensor (no fill kernel); the
    # router backward then treats it as zero.
    if grad_aux is None:
        grad_aux = torch.empty(0, dtype=torch.float32, device=h2.device)
    if grad_probability_sum is None:
        grad_probability_sum = torch.empty(0, dtype=torch.float32, device=h2.device)
    if grad_output is None:
        grad_output = torch.zeros_like(h2)
    needs = ctx.needs_input_grad
    grads = _backward_op(
        grad_output.contiguous(), grad_aux, grad_probability_sum, *saved[:11], ctx.top_k,
        ctx.routing_mode, ctx.lengths, ctx.weight_grad_dtype, ctx.swiglu_limit, bool(needs[2]),
        bool(needs[3]), bool(needs[4]), False, components,
    )
    grad_h2, _, grad_router, grad_w13, grad_w2 = grads
    # d residual is the incoming cotangent itself; the operator returns an
    # empty placeholder here rather than a copy (a custom operator's outputs
    # may not alias its inputs).
    grad_residual = grad_output if needs[1] else None
    return (grad_h2, grad_residual, grad_router if needs[2] else None,
            grad_w13 if needs[3] else None, grad_w2 if needs[4] else None, *([None] * 10),
            [None] * ctx.n_components)


_forward_op.register_autograd(_autograd_backward, setup_context=_setup_context)


def _containers(w13, w2):
    """Plain weights quantized per call (straight through, w13 gate/up-adjacent);
    containers as they are."""
    weights = (w13 if is_row_fp8(w13) else RowFP8Weight.quantize(w13, interleaved=True),
               w2 if is_row_fp8(w2) else RowFP8Weight.quantize(w2))
    route_containers(OPERATORS, _container_rule, *weights)
    return weights


def apply(
    h2, residual, router_weight, w13_experts, w2_experts, *, top_k, routing_mode,
    router_bias=None, n_group=1, topk_group=1, routed_scaling=1.0, lengths=None,
    shared_w13=None, shared_w2=None, shared_gate_weight=None, shared_mode="add",
    compute_precision=None, swiglu_limit=None,
):
    """``(out, aux, counts, probability_sum)`` with autograd through the op pair."""
    _, refusal = _precision(compute_precision, w13_experts, w2_experts)
    if refusal is not None:
        raise ValueError(refusal)
    w13, w2 = _containers(w13_experts, w2_experts)
    rows = h2.numel() // h2.shape[-1]
    normalized = (rows,) if lengths is None else tuple(int(x) for x in lengths)
    bias = (torch.empty(0, dtype=torch.float32, device=h2.device) if router_bias is None
            else router_bias)
    base = fused._shared_base(h2, residual, shared_w13, shared_w2, shared_gate_weight,
                              shared_mode, swiglu_limit)
    outputs = _forward_op(
        h2, base, router_weight, w13, w2, bias, int(top_k), str(routing_mode), int(n_group),
        int(topk_group), float(routed_scaling), list(normalized),
        current_route_weight_precision(), weight_gradient_dtype(),
        None if swiglu_limit is None else float(swiglu_limit), [],
    )
    return outputs[:4]


def _weight(weight, interleaved):
    parts = row_parts(weight)
    if parts is not None:
        return parts
    return kernels.quantize_weights_current(weight.detach(), interleaved=interleaved)


def forward(
    h2, residual, router_weight, w13_experts, w2_experts, *, top_k, routing_mode,
    router_bias=None, n_group=1, topk_group=1, routed_scaling=1.0, lengths=None,
    weight_precision="float32", swiglu_implementation=None, swiglu_limit=None,
):
    """Explicit surface: the 11-tuple of the fused operator, ``h13`` interleaved."""
    del weight_precision, swiglu_implementation
    return forward_routed(
        h2, residual, router_weight, _weight(w13_experts, True), _weight(w2_experts, False),
        top_k=top_k, routing_mode=routing_mode, router_bias=router_bias, n_group=n_group,
        topk_group=topk_group, routed_scaling=routed_scaling, lengths=lengths,
        swiglu_limit=swiglu_limit,
    )


def backward(
    grad_output, grad_aux, grad_probability_sum, h2, router_weight, w13_experts, w2_experts,
    logits, route_weights, route_ids, order, offsets, slots, h13, *, top_k, routing_mode,
    lengths, swiglu_implementation=None, swiglu_limit=None, weight_grad_dtype=None,
):
    """Explicit surface: ``(d_h2, d_residual, d_router, d_w13, d_w2)``."""
    del swiglu_implementation
    grad_dtype = weight_gradient_dtype() if weight_grad_dtype is None else weight_grad_dtype
    return backward_routed(
        grad_output, grad_aux, grad_probability_sum, h2, router_weight,
        _weight(w13_experts, True), _weight(w2_experts, False), logits, route_weights,
        route_ids, order, offsets, slots, h13, top_k=top_k, routing_mode=routing_mode,
        lengths=lengths, weight_grad_dtype=grad_dtype, swiglu_limit=swiglu_limit,
    )


IMPLEMENTATION = register_implementation(
    Implementation(
        operation="moe",
        implementation_id=IMPLEMENTATION_ID,
        provider="mi355x",
        priority=PRIORITY,
        deterministic=True,
        supports=supports,
        apply=apply,
        forward=forward,
        backward=backward,
        estimate=fused.estimate,
    )
)

__all__ = ["IMPLEMENTATION", "apply", "backward", "backward_routed", "forward",
           "forward_routed", "supports"]
