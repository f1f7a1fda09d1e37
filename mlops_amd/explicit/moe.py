"""``mlops_amd.explicit.moe``: the routed MoE as an explicit forward and a
manual VJP, for callers that drive the backward themselves.

The signatures and result tuples are the reference's explicit surface
(``src/mlops/explicit/moe.py:12-119``), which callers depend on:

* ``forward`` -> ``(output, aux, counts, probability_sum, logits,
  route_weights, route_ids, order, offsets, slots, h13)``;
* ``backward`` -> ``(d_h2, d_residual, d_router, d_w13, d_w2)``.

Both pick the implementation for the call on the explicit surface and run it
under ``no_grad``; neither writes ``.grad``. The residuals a forward returns
are that implementation's own (``h13`` here is the interleaved gate/up
pre-activation) and go back, unchanged, into its backward.
"""

from __future__ import annotations

from collections.abc import Sequence

import torch

from ..dispatch import resolve_implementation


def _explicit(weights, routing: dict):
    """The implementation serving ``(h2, residual, router, w13, w2)`` on the
    explicit surface with ``routing`` (the options every such call states)."""
    return resolve_implementation("moe", *weights, surface="explicit", **routing)


def forward(
    h2, residual, router_weight, w13_experts, w2_experts, *, top_k: int, routing_mode: str,
    router_bias=None, n_group: int = 1, topk_group: int = 1, routed_scaling: float = 1.0,
    lengths: Sequence[int] | None = None, weight_precision: str = "float32",
    swiglu_implementation: str = "builtin.packed_swiglu.triton",
):
    """Output, auxiliary statistics and the residuals of the explicit VJP."""
    routing = dict(top_k=int(top_k), routing_mode=str(routing_mode), router_bias=router_bias,
                   n_group=int(n_group), topk_group=int(topk_group),
                   routed_scaling=float(routed_scaling), lengths=lengths)
    operands = (h2, residual, router_weight, w13_experts, w2_experts)
    implementation = _explicit(operands, routing)
    with torch.no_grad():
        return implementation.forward(*operands, **routing,
                                      weight_precision=str(weight_precision),
                                      swiglu_implementation=str(swiglu_implementation))


def backward(
    grad_output, grad_aux, grad_probability_sum, h2, router_weight, w13_experts, w2_experts,
    logits, route_weights, route_ids, order, offsets, slots, h13, *, top_k: int,
    routing_mode: str, lengths: Sequence[int],
    swiglu_implementation: str = "builtin.packed_swiglu.triton",
):
    """Gradients for ``(h2, residual, router_weight, w13, w2)`` from the
    forward's residuals and the three cotangents."""
    routing = dict(top_k=int(top_k), routing_mode=str(routing_mode), lengths=lengths)
    # The residual only enters the output additively, so h2 stands in for it
    # when the implementation is chosen (same shape, dtype and device).
    implementation = _explicit((h2, h2, router_weight, w13_experts, w2_experts), routing)
    residuals = (logits, route_weights, route_ids, order, offsets, slots, h13)
    with torch.no_grad():
        return implementation.backward(grad_output, grad_aux, grad_probability_sum, h2,
                                       router_weight, w13_experts, w2_experts, *residuals,
                                       **routing,
                                       swiglu_implementation=str(swiglu_implementation))


__all__ = ["backward", "forward"]
