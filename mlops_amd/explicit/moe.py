"""Explicit (manual VJP) routed-MoE entry points, as ``mlops.explicit.moe``
(``src/mlops/explicit/moe.py:12-119``): ``forward`` returns the output, the
auxiliary statistics and the residuals ``(output, aux, counts,
probability_sum, logits, route_weights, route_ids, order, offsets, slots,
h13)``; ``backward`` returns ``(d_h2, d_residual, d_router, d_w13, d_w2)``.
Both run under ``no_grad`` and never write ``.grad``.
"""

from __future__ import annotations

from collections.abc import Sequence

import torch

from ..dispatch import resolve_implementation


def forward(
    h2, residual, router_weight, w13_experts, w2_experts, *, top_k: int, routing_mode: str,
    router_bias=None, n_group: int = 1, topk_group: int = 1, routed_scaling: float = 1.0,
    lengths: Sequence[int] | None = None, weight_precision: str = "float32",
    swiglu_implementation: str = "builtin.packed_swiglu.triton",
):
    implementation = resolve_implementation(
        "moe", h2, residual, router_weight, w13_experts, w2_experts, surface="explicit",
        top_k=int(top_k), routing_mode=str(routing_mode), router_bias=router_bias,
        n_group=int(n_group), topk_group=int(topk_group), routed_scaling=float(routed_scaling),
        lengths=lengths,
    )
    with torch.no_grad():
        return implementation.forward(
            h2, residual, router_weight, w13_experts, w2_experts, top_k=int(top_k),
            routing_mode=str(routing_mode), router_bias=router_bias, n_group=int(n_group),
            topk_group=int(topk_group), routed_scaling=float(routed_scaling), lengths=lengths,
            weight_precision=str(weight_precision),
            swiglu_implementation=str(swiglu_implementation),
        )


def backward(
    grad_output, grad_aux, grad_probability_sum, h2, router_weight, w13_experts, w2_experts,
    logits, route_weights, route_ids, order, offsets, slots, h13, *, top_k: int,
    routing_mode: str, lengths: Sequence[int],
    swiglu_implementation: str = "builtin.packed_swiglu.triton",
):
    implementation = resolve_implementation(
        "moe", h2, h2, router_weight, w13_experts, w2_experts, surface="explicit",
        top_k=int(top_k), routing_mode=str(routing_mode), lengths=lengths,
    )
    with torch.no_grad():
        return implementation.backward(
            grad_output, grad_aux, grad_probability_sum, h2, router_weight, w13_experts,
            w2_experts, logits, route_weights, route_ids, order, offsets, slots, h13,
            top_k=int(top_k), routing_mode=str(routing_mode), lengths=lengths,
            swiglu_implementation=str(swiglu_implementation),
        )


__all__ = ["backward", "forward"]
