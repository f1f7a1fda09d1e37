"""Canonical logical FLOP counts of the routed MoE.

Convention of the reference (``src/mlops/dispatch/logical_costs.py:401-494``):
a multiply-add is two FLOPs and each of the ``rows * top_k`` assignments is
charged as one row of every expert product, whatever the routing. Router:
``2*T*D*E`` for the logits plus ``3*T*E`` for the routing arithmetic; up
projection ``2*A*D*2F``; activation ``5*A*F``; down ``2*A*F*D``; combine
``2*A*D``. The backward doubles the GEMMs (input and weight gradients).
"""

from __future__ import annotations


def _rows(h2) -> int:
    return h2.numel() // h2.shape[-1]


def _elements(*tensors) -> int:
    return sum(t.numel() * t.element_size() for t in tensors if t is not None)


def _forward(entrypoint) -> bool:
    if entrypoint not in ("forward", "backward"):
        raise ValueError("entrypoint must be 'forward' or 'backward'")
    return entrypoint == "forward"


def moe_prepare_flops(rows, width, experts, assignments, packed, *, forward):
    router = 2 * rows * width * experts + 3 * rows * experts
    up = 2 * assignments * width * packed
    if forward:
        return router + up
    return 2 * router - 3 * rows * experts + 2 * up


def moe_finish_flops(assignments, expert_width, width, *, forward):
    activation = 5 * assignments * expert_width
    down = 2 * assignments * expert_width * width
    combine = 2 * assignments * width
    if forward:
        return activation + down + combine
    return 2 * activation + 2 * down + combine


def moe_flops(h2, router_weight, w13_experts, w2_experts, top_k, *, forward) -> int:
    rows = _rows(h2)
    width = h2.shape[-1]
    experts = router_weight.shape[0]
    assignments = rows * int(top_k)
    return moe_prepare_flops(
        rows, width, experts, assignments, w13_experts.shape[1], forward=forward
    ) + moe_finish_flops(assignments, w2_experts.shape[2], width, forward=forward)


def moe(h2, residual, router_weight, w13_experts, w2_experts, *, top_k,
        entrypoint="forward", **_kwargs):
    from .costs import CostHints

    forward = _forward(entrypoint)
    flops = moe_flops(h2, router_weight, w13_experts, w2_experts, top_k, forward=forward)
    weights = _elements(router_weight, w13_experts, w2_experts)
    if forward:
        return CostHints(
            logical_flops=flops,
            logical_bytes_accessed=_elements(h2, residual) + weights + _elements(h2),
            notes=("minimum traffic: activations and every expert read once, output written",),
        )
    h13 = _rows(h2) * int(top_k) * w13_experts.shape[1] * h2.element_size()
    return CostHints(
        logical_flops=flops,
        logical_bytes_accessed=4 * _elements(h2) + 2 * weights + h13,
        notes=("backward reads dy, h2, the weights and h13; writes every gradient",),
    )


ESTIMATORS = {"moe": moe}

__all__ = ["ESTIMATORS", "moe", "moe_finish_flops", "moe_flops", "moe_prepare_flops"]
