"""FLOP formulas for custom operators and advisory cost estimates.

``flop_formula`` registers a shape-only FLOP count with
``torch.utils.flop_counter`` so ``FlopCounterMode`` prices the provider's
opaque operators (reference: ``src/mlops/dispatch/costs.py:142-175``).
``estimate_implementation`` merges the operation's canonical estimate with the
selected implementation's own hints (``costs.py:81-120``).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch.utils.flop_counter import flop_registry
from torch.utils.flop_counter import register_flop_formula as _register

from .context import use_implementation
from .registry import implementations_for
from .resolution import explain_implementation


@dataclass(frozen=True)
class CostHints:
    """Advisory work/traffic figures; ``None`` means unknown, never zero."""

    logical_flops: int | None = None
    logical_bytes_accessed: int | None = None
    implementation_flops: int | None = None
    implementation_bytes_accessed: int | None = None
    workspace_bytes: int | None = None
    notes: tuple[str, ...] = ()

    @property
    def has_roofline_estimate(self) -> bool:
        return (
            self.implementation_flops is not None
            and self.implementation_bytes_accessed is not None
        )

    def merged(self, other: "CostHints") -> "CostHints":
        fields = (
            "logical_flops",
            "logical_bytes_accessed",
            "implementation_flops",
            "implementation_bytes_accessed",
            "workspace_bytes",
        )
        values = {
            name: getattr(self, name) if getattr(other, name) is None else getattr(other, name)
            for name in fields
        }
        return CostHints(**values, notes=self.notes + other.notes)


def _packet(operator):
    if isinstance(operator, torch._ops.OpOverloadPacket):
        return operator
    if isinstance(operator, torch._ops.OpOverload):
        return operator.overloadpacket
    overload = getattr(operator, "_opoverload", None)
    if isinstance(overload, torch._ops.OpOverload):
        return overload.overloadpacket
    raise TypeError(
        "flop_formula takes a registered custom operator or its torch.ops packet, "
        f"not {type(operator).__name__}"
    )


def flop_formula(*operators):
    """Decorator: register the function as the FLOP count of ``operators``.

    The function receives the operator's arguments plus ``out_val`` and must
    read shapes only (it also runs under fake tensors)."""
    packets = tuple(_packet(op) for op in operators)
    if not packets:
        raise ValueError("flop_formula requires at least one operator")

    def register(formula):
        for packet in packets:
            _register(packet, get_raw=True)(formula)
        return formula

    return register


def has_flop_formula(operator) -> bool:
    return _packet(operator) in flop_registry


def estimate_implementation(
    operation: str,
    *args,
    implementation_id: str | None = None,
    surface: str = "semantic",
    entrypoint: str = "forward",
    **kwargs,
) -> CostHints:
    """Canonical estimate merged with the implementation's own, from metadata."""
    if entrypoint not in ("forward", "backward"):
        raise ValueError("entrypoint must be 'forward' or 'backward'")
    if implementation_id is None:
        explanation = explain_implementation(operation, *args, surface=surface, **kwargs)
    else:
        with use_implementation(operation, implementation_id):
            explanation = explain_implementation(operation, *args, surface=surface, **kwargs)
    if explanation.selected is None:
        reasons = "; ".join(
            f"{name}: {result.reason}" for name, result in sorted(explanation.candidates.items())
        )
        raise RuntimeError(f"cannot estimate unsupported {operation!r}: {reasons}")
    from . import logical_costs

    implementation = implementations_for(operation)[explanation.selected]
    canonical_fn = logical_costs.ESTIMATORS.get(str(operation))
    canonical = (
        CostHints(notes=("canonical operation estimate is undefined",))
        if canonical_fn is None
        else canonical_fn(*args, entrypoint=entrypoint, **kwargs)
    )
    own = (
        CostHints(notes=(f"{implementation.implementation_id} provides no physical estimate",))
        if implementation.estimate is None
        else implementation.estimate(*args, entrypoint=entrypoint, **kwargs)
    )
    return canonical.merged(own)


__all__ = ["CostHints", "estimate_implementation", "flop_formula", "has_flop_formula"]
