"""FLOP formulas for opaque custom operators, and advisory cost estimates.

* `flop_formula(op, ...)` registers a shape-only function with
  ``torch.utils.flop_counter`` so that ``FlopCounterMode`` can price the
  provider's custom operators (which it cannot see into); the reference
  exposes the same decorator (``src/mlops/dispatch/costs.py``).
* `estimate_implementation` returns the operation's logical cost (from
  `logical_costs`) overlaid with the selected implementation's own figures.
  Every figure is advisory: ``None`` means "unknown", never zero.
"""

from __future__ import annotations

from dataclasses import dataclass, fields

import torch
from torch.utils.flop_counter import flop_registry, register_flop_formula

from .context import use_implementation
from .registry import implementations_for
from .resolution import explain_implementation

_FIGURES = ("logical_flops", "logical_bytes_accessed", "implementation_flops",
            "implementation_bytes_accessed", "workspace_bytes")


@dataclass(frozen=True)
class CostHints:
    """Work and traffic figures of one call (``None``: unknown)."""

    logical_flops: int | None = None
    logical_bytes_accessed: int | None = None
    implementation_flops: int | None = None
    implementation_bytes_accessed: int | None = None
    workspace_bytes: int | None = None
    notes: tuple[str, ...] = ()

    @property
    def has_roofline_estimate(self) -> bool:
        """Whether both implementation figures a roofline needs are known."""
        return None not in (self.implementation_flops, self.implementation_bytes_accessed)

    def merged(self, other: "CostHints") -> "CostHints":
        """``other``'s known figures over this one's; notes of both."""
        values = {}
        for item in fields(self):
            mine, theirs = getattr(self, item.name), getattr(other, item.name)
            if item.name == "notes":
                values["notes"] = tuple(mine) + tuple(theirs)
            else:
                values[item.name] = mine if theirs is None else theirs
        return CostHints(**values)


def _overload_packet(operator):
    """The ``torch.ops`` packet of a custom operator, its overload, or the
    function object ``torch.library.custom_op`` returns."""
    if isinstance(operator, torch._ops.OpOverloadPacket):
        return operator
    for candidate in (operator, getattr(operator, "_opoverload", None)):
        packet = getattr(candidate, "overloadpacket", None)
        if isinstance(packet, torch._ops.OpOverloadPacket):
            return packet
    raise TypeError(f"{operator!r} is not a registered custom operator; flop formulas attach "
                    "to operators from torch.library.custom_op or torch.ops")


def flop_formula(*operators):
    """Decorator registering a FLOP count for ``operators``. The function
    gets the operator's arguments and ``out_val``, and must only read shapes:
    it also runs on fake tensors."""
    if not operators:
        raise ValueError("flop_formula needs at least one operator")
    packets = [_overload_packet(op) for op in operators]

    def register(formula):
        for packet in packets:
            register_flop_formula(packet, get_raw=True)(formula)
        return formula

    return register


def has_flop_formula(operator) -> bool:
    return _overload_packet(operator) in flop_registry


def estimate_implementation(operation: str, *args, implementation_id: str | None = None,
                            surface: str = "semantic", entrypoint: str = "forward",
                            **kwargs) -> CostHints:
    """Logical cost of the call, overlaid with the implementation's own
    estimate (the selected one, or ``implementation_id``'s). Reads metadata
    only; raises when no implementation supports the call."""
    if entrypoint not in ("forward", "backward"):
        raise ValueError(f"entrypoint is 'forward' or 'backward', not {entrypoint!r}")
    if implementation_id is None:
        explanation = explain_implementation(operation, *args, surface=surface, **kwargs)
    else:
        with use_implementation(operation, implementation_id):
            explanation = explain_implementation(operation, *args, surface=surface, **kwargs)
    if explanation.selected is None:
        refusals = "; ".join(f"{key}: {verdict.reason}"
                             for key, verdict in sorted(explanation.candidates.items()))
        raise RuntimeError(f"no estimate: no implementation of {operation!r} supports this "
                           f"call ({refusals})")
    from . import logical_costs

    record = implementations_for(operation)[explanation.selected]
    logical = logical_costs.ESTIMATORS.get(str(operation))
    hints = (logical(*args, entrypoint=entrypoint, **kwargs) if logical is not None
             else CostHints(notes=(f"no logical cost model for {operation!r}",)))
    if record.estimate is None:
        return hints.merged(CostHints(notes=(f"{record.implementation_id} gives no estimate "
                                             "of its own",)))
    return hints.merged(record.estimate(*args, entrypoint=entrypoint, **kwargs))


__all__ = ["CostHints", "estimate_implementation", "flop_formula", "has_flop_formula"]
