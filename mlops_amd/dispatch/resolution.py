"""Choosing an implementation for one call.

Every registered implementation of the operation is asked whether it
supports the call (metadata only). The selection rule is the reference's
(``src/mlops/dispatch/resolution.py``): a forced ID is taken if, and only if,
it supports the call; otherwise the supporting implementation with the
highest priority, ties going to the lexicographically smaller ID. The
explicit surface only considers records with a forward/backward pair.
"""

from __future__ import annotations

from collections.abc import Mapping
from dataclasses import dataclass
from types import MappingProxyType

from .context import implementation_override, record_dispatch
from .registry import Implementation, SupportResult, frozen_implementation, implementations_for

SURFACES = ("semantic", "explicit")


@dataclass(frozen=True)
class ImplementationExplanation:
    """Every candidate's answer and the choice made from them."""

    operation: str
    surface: str
    selected: str | None
    forced: str | None
    candidates: Mapping[str, SupportResult]


def _as_result(implementation: Implementation, answer) -> SupportResult:
    if isinstance(answer, SupportResult):
        return answer
    if isinstance(answer, bool):
        return SupportResult.yes() if answer else SupportResult.no("declined")
    raise TypeError(f"supports() of {implementation.implementation_id} must return a "
                    f"SupportResult or bool, not {type(answer).__name__}")


def _verdict(implementation: Implementation, surface: str, args, kwargs) -> SupportResult:
    if surface not in SURFACES:
        return SupportResult.no(f"surface {surface!r} is not one of {SURFACES}")
    if surface == "explicit" and not implementation.explicit:
        return SupportResult.no("no explicit forward/backward pair")
    try:
        answer = implementation.supports(*args, surface=surface, **kwargs)
    except Exception as error:  # one provider's failure must not end resolution
        return SupportResult.no(f"support check raised {type(error).__name__}: {error}")
    return _as_result(implementation, answer)


def _preference(implementation: Implementation):
    """Sort key: higher priority first, then the smaller ID."""
    return -implementation.priority, implementation.implementation_id


def explain_implementation(operation: str, *args, surface: str = "semantic",
                           **kwargs) -> ImplementationExplanation:
    """The candidates' answers and the selection, without dispatching."""
    table = implementations_for(operation)
    verdicts = {key: _verdict(record, surface, args, kwargs) for key, record in table.items()}
    forced = implementation_override(operation)
    if forced is not None:
        selected = forced if verdicts[forced].supported else None
    else:
        accepted = [table[key] for key, verdict in verdicts.items() if verdict.supported]
        selected = min(accepted, key=_preference).implementation_id if accepted else None
    return ImplementationExplanation(str(operation), str(surface), selected, forced,
                                     MappingProxyType(verdicts))


def resolve_implementation(operation: str, *args, surface: str = "semantic",
                           **kwargs) -> Implementation:
    """The implementation to run; RuntimeError with every refusal otherwise."""
    explanation = explain_implementation(operation, *args, surface=surface, **kwargs)
    if explanation.selected is None:
        refusals = "; ".join(f"{key}: {verdict.reason}"
                             for key, verdict in sorted(explanation.candidates.items()))
        what = ("no supported implementation" if explanation.forced is None
                else f"the forced implementation {explanation.forced!r} does not support it")
        raise RuntimeError(f"{what} for {explanation.operation!r} ({surface} surface): "
                           f"{refusals}")
    record_dispatch(explanation.operation, explanation.selected)
    return frozen_implementation(explanation.operation, explanation.selected)


def implementation_pairs(operations) -> Mapping[str, Mapping[str, Mapping[str, str]]]:
    """For each operation, the two forcing maps a verifier compares: the
    implementation resolution prefers (``"default"``) and the preferred
    ``native_torch`` provider record (``"native_torch"``), each as
    ``{operation: implementation ID}`` ready for ``use_implementations``.
    Support is not consulted (the pair is fixed by the catalog alone); an
    operation with no native_torch record raises ValueError (reference
    ``src/mlops/dispatch/resolution.py:113-140``)."""
    pairs = {}
    for operation in map(str, operations):
        ranked = sorted(implementations_for(operation).values(), key=_preference)
        natives = [record for record in ranked if record.provider == "native_torch"]
        if not natives:
            raise ValueError(f"{operation!r} has no native_torch implementation to pair with")
        pairs[operation] = MappingProxyType({
            "default": MappingProxyType({operation: ranked[0].implementation_id}),
            "native_torch": MappingProxyType({operation: natives[0].implementation_id}),
        })
    return MappingProxyType(pairs)


__all__ = ["ImplementationExplanation", "explain_implementation", "implementation_pairs",
           "resolve_implementation"]
