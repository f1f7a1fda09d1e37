"""Model-facing routed-MoE façade: ``mlops_amd.moe(...)``.

Same signature, validation and result as the reference's ``mlops.moe``
(``src/mlops/moe.py:40-136``): validates the arguments, resolves an
implementation through the registry for this exact invocation (the MI355X
block-FP8 provider on gfx950) and returns ``(out, aux, counts,
probability_sum)``.
"""

from __future__ import annotations

from .dispatch import resolve_implementation


def moe(
    h2,
    residual,
    router_weight,
    w13_experts,
    w2_experts,
    *,
    top_k,
    routing_mode,
    router_bias=None,
    n_group=1,
    topk_group=1,
    routed_scaling=1.0,
    lengths=None,
    shared_w13=None,
    shared_w2=None,
    shared_gate_weight=None,
    shared_mode="add",
    compute_precision=None,
    swiglu_limit=None,
):
    """Routed output, auxiliary loss, expert counts and probability sum.

    Weights are in nn.Linear orientation: ``router_weight [E, D]``,
    ``w13_experts [E, 2F, D]`` (gate rows then up rows), ``w2_experts [E, D, F]``;
    expert weights may be `BlockFP8Weight` containers. ``compute_precision``
    ``"fp8_block"`` (the containers' default) computes the expert GEMMs in e4m3
    with 1x128 activation and 128x128 weight scales. ``swiglu_limit`` clamps the
    gate at the limit and the up projection to ``[-limit, limit]``.
    """
    rows = h2.numel() // h2.shape[-1]
    if compute_precision not in (None, "bf16", "fp8_current", "fp8_block"):
        raise ValueError(f"unsupported compute precision {compute_precision!r}")
    if swiglu_limit is not None:
        swiglu_limit = float(swiglu_limit)
        if not swiglu_limit > 0:
            raise ValueError("swiglu_limit must be positive")
    lengths = (rows,) if lengths is None else tuple(int(x) for x in lengths)
    if (shared_w13 is None) != (shared_w2 is None):
        raise ValueError("shared_w13 and shared_w2 must be supplied together")
    if shared_mode not in ("add", "sigmoid"):
        raise ValueError(f"unsupported shared expert mode {shared_mode!r}")
    if shared_mode == "sigmoid" and shared_gate_weight is None:
        raise ValueError("sigmoid shared expert requires shared_gate_weight")
    options = dict(
        top_k=int(top_k),
        routing_mode=routing_mode,
        router_bias=router_bias,
        n_group=int(n_group),
        topk_group=int(topk_group),
        routed_scaling=float(routed_scaling),
        lengths=lengths,
        shared_w13=shared_w13,
        shared_w2=shared_w2,
        shared_gate_weight=shared_gate_weight,
        shared_mode=shared_mode,
        compute_precision=compute_precision,
        swiglu_limit=swiglu_limit,
    )
    implementation = resolve_implementation(
        "moe", h2, residual, router_weight, w13_experts, w2_experts, surface="semantic", **options
    )
    return implementation.apply(h2, residual, router_weight, w13_experts, w2_experts, **options)


__all__ = ["moe"]
