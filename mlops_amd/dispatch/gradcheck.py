"""Checking one registered implementation's backward against finite
differences, without letting resolution pick another implementation.

Reference surface: ``src/mlops/dispatch/gradcheck.py`` (`GradcheckResult`
:15, `GradcheckCase` :25, `gradcheck_implementation` :34,
`gradcheck_implementations` :106). Each check first asks the named
implementation whether it takes the inputs (on the semantic surface, with the
ID forced); one that declines is reported ``skipped`` with its reason, never
replaced. Inputs are the operation's usual differentiable arguments in
float64, which ``torch.autograd.gradcheck`` needs; the MI355X MoE
implementations compute in fp8/bf16 and therefore report ``skipped``.
"""

from __future__ import annotations

from collections.abc import Iterable, Mapping, Sequence
from dataclasses import dataclass

import torch

from .context import use_implementation
from .registry import implementations_for
from .resolution import explain_implementation

STATUSES = ("passed", "failed", "skipped")


@dataclass(frozen=True)
class GradcheckResult:
    """The outcome for one (operation, implementation ID)."""

    operation: str
    implementation_id: str
    status: str  # one of STATUSES
    reason: str


@dataclass(frozen=True)
class GradcheckCase:
    """Inputs for one operation and the IDs to check (None: every ID)."""

    operation: str
    inputs: tuple[torch.Tensor, ...]
    kwargs: Mapping[str, object] | None = None
    implementation_ids: tuple[str, ...] | None = None


def _declined(operation: str, implementation_id: str, inputs, kwargs) -> str | None:
    """The implementation's refusal of these inputs, or None if it takes them."""
    with use_implementation(operation, implementation_id):
        answer = explain_implementation(operation, *inputs, surface="semantic", **kwargs)
    if answer.selected == implementation_id:
        return None
    return answer.candidates[implementation_id].reason


def gradcheck_implementation(operation: str, implementation_id: str,
                             inputs: Sequence[torch.Tensor], *,
                             kwargs: Mapping[str, object] | None = None, eps: float = 1e-6,
                             atol: float = 1e-5, rtol: float = 1e-3,
                             raise_exception: bool = False) -> GradcheckResult:
    """``torch.autograd.gradcheck`` of exactly ``implementation_id``'s apply.

    An unknown ID raises ValueError. A gradcheck error is reported as
    ``failed`` with the error text unless ``raise_exception`` is set.
    """
    operation, implementation_id = str(operation), str(implementation_id)
    table = implementations_for(operation)
    record = table.get(implementation_id)
    if record is None:
        raise ValueError(f"{operation!r} has no implementation {implementation_id!r} "
                         f"(registered: {', '.join(sorted(table))})")
    extra = dict(kwargs or {})
    refusal = _declined(operation, implementation_id, inputs, extra)
    if refusal is not None:
        return GradcheckResult(operation, implementation_id, "skipped", refusal)
    try:
        ok = torch.autograd.gradcheck(lambda *args: record.apply(*args, **extra), tuple(inputs),
                                      eps=float(eps), atol=float(atol), rtol=float(rtol),
                                      raise_exception=bool(raise_exception))
    except Exception as error:
        if raise_exception:
            raise
        return GradcheckResult(operation, implementation_id, "failed",
                               f"{type(error).__name__}: {error}")
    if ok:
        return GradcheckResult(operation, implementation_id, "passed",
                               "analytic and numerical Jacobians agree")
    return GradcheckResult(operation, implementation_id, "failed",
                           "analytic and numerical Jacobians differ")


def gradcheck_implementations(cases: Iterable[GradcheckCase], *, eps: float = 1e-6,
                              atol: float = 1e-5, rtol: float = 1e-3,
                              raise_exception: bool = False) -> tuple[GradcheckResult, ...]:
    """Every case against its listed IDs, or all of the operation's IDs in
    sorted order when it lists none."""
    out: list[GradcheckResult] = []
    for case in cases:
        ids = case.implementation_ids
        if ids is None:
            ids = tuple(sorted(implementations_for(case.operation)))
        out.extend(gradcheck_implementation(case.operation, implementation_id, case.inputs,
                                            kwargs=case.kwargs, eps=eps, atol=atol, rtol=rtol,
                                            raise_exception=raise_exception)
                   for implementation_id in ids)
    return tuple(out)


__all__ = ["GradcheckCase", "GradcheckResult", "gradcheck_implementation",
           "gradcheck_implementations"]
