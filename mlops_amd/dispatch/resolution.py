"""Support filtering and priority selection.

Selection rule as in the reference (``src/mlops/dispatch/resolution.py:53-112``):
every implementation's ``supports`` is asked; a forced choice wins if it is
supported; otherwise the highest priority wins, ties broken by the smaller ID;
the explicit surface only considers implementations with forward/backward.
"""

from __future__ import annotations

from collections.abc import Mapping
from dataclasses import dataclass
from types import MappingProxyType

from .context import implementation_override, record_dispatch
from .registry import (
    Implementation,
    SupportResult,
    frozen_implementation,
    implementations_for,
)


@dataclass(frozen=True)
class ImplementationExplanation:
    operation: str
    surface: str
    selected: str | None
    forced: str | None
    candidates: Mapping[str, SupportResult]


def _ask(implementation: Implementation, *args, surface: str, **kwargs) -> SupportResult:
    if surface not in ("semantic", "explicit"):
        return SupportResult.no(f"unknown surface {surface!r}")
    if surface == "explicit" and implementation.forward is None:
        return SupportResult.no("implementation does not expose explicit forward/backward")
    try:
        answer = implementation.supports(*args, surface=surface, **kwargs)
    except Exception as error:  # a provider's refusal must not break resolution
        return SupportResult.no(f"support check failed: {type(error).__name__}: {error}")
    if isinstance(answer, SupportResult):
        return answer
    if isinstance(answer, bool):
        return SupportResult(answer, "supported" if answer else "rejected")
    raise TypeError(
        f"{implementation.implementation_id}.supports returned {type(answer).__name__}"
    )


def explain_implementation(
    operation: str, *args, surface: str = "semantic", **kwargs
) -> ImplementationExplanation:
    table = implementations_for(operation)
    answers = {
        name: _ask(impl, *args, surface=surface, **kwargs) for name, impl in table.items()
    }
    forced = implementation_override(operation)
    if forced is not None:
        selected = forced if answers[forced].supported else None
    else:
        ranked = sorted(
            (impl for name, impl in table.items() if answers[name].supported),
            key=lambda impl: (-impl.priority, impl.implementation_id),
        )
        selected = ranked[0].implementation_id if ranked else None
    return ImplementationExplanation(
        operation=str(operation),
        surface=str(surface),
        selected=selected,
        forced=forced,
        candidates=MappingProxyType(answers),
    )


def resolve_implementation(
    operation: str, *args, surface: str = "semantic", **kwargs
) -> Implementation:
    """The selected implementation, or ``RuntimeError`` listing every refusal."""
    explanation = explain_implementation(operation, *args, surface=surface, **kwargs)
    if explanation.selected is None:
        reasons = "; ".join(
            f"{name}: {result.reason}"
            for name, result in sorted(explanation.candidates.items())
        )
        head = (
            f"forced implementation {explanation.forced!r} is unsupported"
            if explanation.forced is not None
            else "no supported implementation"
        )
        raise RuntimeError(
            f"{head} for {explanation.operation!r} on {surface!r} surface; {reasons}"
        )
    implementation = frozen_implementation(explanation.operation, explanation.selected)
    record_dispatch(explanation.operation, implementation.implementation_id)
    return implementation


__all__ = ["ImplementationExplanation", "explain_implementation", "resolve_implementation"]
