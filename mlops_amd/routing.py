"""Context-local routing controls of the reference router
(``src/mlops/kernels/moe_router.py:22-100``):

* ``route_weight_precision("float32" | "input")`` -- the dtype of the route
  weights. Logits are fp32, so both choices give fp32 weights here.
* ``routing_override(decisions)`` -- force successive router calls to use
  caller-supplied top-k expert ids (a diagnostic for separating near-tie
  flips from kernel error); weights stay live functions of the logits. The
  context raises if fewer decisions were consumed than supplied.
"""

from __future__ import annotations

from contextlib import contextmanager
from contextvars import ContextVar
from dataclasses import dataclass

import torch

_WEIGHT_PRECISION: ContextVar[str] = ContextVar("mlops_amd_route_weight_precision", default="float32")


@dataclass
class _Overrides:
    decisions: tuple
    consumed: int = 0


_OVERRIDES: ContextVar[_Overrides | None] = ContextVar("mlops_amd_routing_overrides", default=None)


def current_route_weight_precision() -> str:
    return _WEIGHT_PRECISION.get()


@contextmanager
def route_weight_precision(name: str):
    if name not in ("float32", "input"):
        raise ValueError(f"unsupported route-weight precision {name!r}")
    token = _WEIGHT_PRECISION.set(name)
    try:
        yield
    finally:
        _WEIGHT_PRECISION.reset(token)


@contextmanager
def routing_override(decisions):
    state = _Overrides(tuple(d.detach() for d in decisions))
    token = _OVERRIDES.set(state)
    try:
        yield
        if state.consumed != len(state.decisions):
            raise RuntimeError(
                f"routing override supplied {len(state.decisions)} decisions "
                f"but consumed {state.consumed}"
            )
    finally:
        _OVERRIDES.reset(token)


def next_override(tokens: int, experts: int, top_k: int, device) -> torch.Tensor | None:
    """The next forced decision, validated, as int32 on ``device``; None if no
    override is active."""
    state = _OVERRIDES.get()
    if state is None:
        return None
    if state.consumed >= len(state.decisions):
        raise RuntimeError("routing override exhausted before model forward ended")
    ids = state.decisions[state.consumed]
    state.consumed += 1
    if tuple(ids.shape) != (tokens, int(top_k)):
        raise ValueError(
            f"routing override {state.consumed - 1} has shape {tuple(ids.shape)}; "
            f"expected {(tokens, int(top_k))}"
        )
    ids = ids.long()
    if bool(((ids < 0) | (ids >= experts)).any()):
        raise ValueError("routing override contains an out-of-range expert id")
    ordered = torch.sort(ids, dim=-1).values
    if bool((ordered[:, 1:] == ordered[:, :-1]).any()):
        raise ValueError("routing override contains duplicate experts in one row")
    return ids.to(device=device, dtype=torch.int32)


__all__ = [
    "current_route_weight_precision",
    "next_override",
    "route_weight_precision",
    "routing_override",
]
