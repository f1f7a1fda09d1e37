"""``mlops_amd.moe(...)``: the model-facing routed mixture-of-experts call.

It takes the reference façade's arguments and returns its 4-tuple
``(out, aux, counts, probability_sum)`` (``src/mlops/moe.py:40-136``). The
call is checked here, then the registry picks the implementation for this
exact invocation -- on gfx950 one of the MI355X providers -- and runs its
autograd entry point.
"""

from __future__ import annotations

from .dispatch import resolve_implementation

PRECISIONS = (None, "bf16", "fp8_current", "fp8_block")
SHARED_MODES = ("add", "sigmoid")


def _checked_limit(swiglu_limit):
    if swiglu_limit is None:
        return None
    limit = float(swiglu_limit)
    if not limit > 0:  # also refuses NaN
        raise ValueError(f"swiglu_limit must be positive, got {swiglu_limit!r}")
    return limit


def _check_shared(shared_w13, shared_w2, shared_gate_weight, shared_mode):
    if (shared_w13 is None) is not (shared_w2 is None):
        raise ValueError("a shared expert needs shared_w13 and shared_w2 together")
    if shared_mode not in SHARED_MODES:
        raise ValueError(f"shared_mode is one of {SHARED_MODES}, not {shared_mode!r}")
    if shared_mode == "sigmoid" and shared_gate_weight is None:
        raise ValueError("shared_mode='sigmoid' gates the shared expert with "
                         "shared_gate_weight, which is missing")


def moe(h2, residual, router_weight, w13_experts, w2_experts, *, top_k, routing_mode,
        router_bias=None, n_group=1, topk_group=1, routed_scaling=1.0, lengths=None,
        shared_w13=None, shared_w2=None, shared_gate_weight=None, shared_mode="add",
        compute_precision=None, swiglu_limit=None):
    """Routed output, auxiliary loss, per-expert counts and probability sum.

    Weights are nn.Linear-oriented: ``router_weight [E, D]``, ``w13_experts
    [E, 2F, D]`` (gate rows, then up rows) and ``w2_experts [E, D, F]``; the
    expert weights may be FP8 containers. ``compute_precision`` selects the
    precision of the expert products: ``"fp8_block"`` (e4m3 with 1x128
    activation and 128x128 weight scales; the default for block-FP8
    containers), ``"fp8_current"`` (one scale per row; the default for row-FP8
    containers) or ``"bf16"``. ``swiglu_limit`` caps the gate at the limit and
    clips the up projection to ``[-limit, limit]`` before ``silu(gate) * up``.
    ``lengths`` splits the rows into sequences for the per-sequence auxiliary
    statistics of ``sigmoid_noaux_tc`` routing.
    """
    if compute_precision not in PRECISIONS:
        raise ValueError(f"compute precision {compute_precision!r} is not one of {PRECISIONS}")
    _check_shared(shared_w13, shared_w2, shared_gate_weight, shared_mode)
    rows = h2.numel() // h2.shape[-1]
    options = {
        "top_k": int(top_k),
        "routing_mode": routing_mode,
        "router_bias": router_bias,
        "n_group": int(n_group),
        "topk_group": int(topk_group),
        "routed_scaling": float(routed_scaling),
        "lengths": (rows,) if lengths is None else tuple(int(n) for n in lengths),
        "shared_w13": shared_w13,
        "shared_w2": shared_w2,
        "shared_gate_weight": shared_gate_weight,
        "shared_mode": shared_mode,
        "compute_precision": compute_precision,
        "swiglu_limit": _checked_limit(swiglu_limit),
    }
    operands = (h2, residual, router_weight, w13_experts, w2_experts)
    chosen = resolve_implementation("moe", *operands, surface="semantic", **options)
    return chosen.apply(*operands, **options)


__all__ = ["moe"]
