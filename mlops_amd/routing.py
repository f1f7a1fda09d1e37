"""Routing controls that belong to the calling context, as the reference's
router offers them (``src/mlops/kernels/moe_router.py:22-100``).

* ``route_weight_precision("float32" | "input")`` sets the dtype of the route
  weights. Logits are fp32 on this path, so both give fp32 weights.
* ``routing_override(decisions)`` makes successive router calls use the
  caller's top-k expert ids, one ``[tokens, k]`` tensor per call, instead of
  selecting them; the weights are still computed from the logits. It is a
  diagnostic (e.g. to tell near-tie flips from kernel error), and leaving the
  block with decisions unused is an error.
"""

from __future__ import annotations

from contextlib import contextmanager
from contextvars import ContextVar

import torch

PRECISIONS = ("float32", "input")
_precision: ContextVar[str] = ContextVar("mlops_amd_route_weight_precision", default="float32")


def current_route_weight_precision() -> str:
    return _precision.get()


@contextmanager
def route_weight_precision(name: str):
    if name not in PRECISIONS:
        raise ValueError(f"route-weight precision is one of {PRECISIONS}, not {name!r}")
    token = _precision.set(name)
    try:
        yield
    finally:
        _precision.reset(token)


class _ForcedRoutes:
    """The decisions of one `routing_override` block, handed out in order."""

    def __init__(self, decisions):
        self.pending = [d.detach() for d in decisions]
        self.total = len(self.pending)
        self.used = 0

    def take(self) -> torch.Tensor:
        if self.used == self.total:
            raise RuntimeError(f"routing override ran out: all {self.total} forced "
                               "decisions were used before the forward finished")
        decision = self.pending[self.used]
        self.used += 1
        return decision


_forced: ContextVar[_ForcedRoutes | None] = ContextVar("mlops_amd_forced_routes", default=None)


@contextmanager
def routing_override(decisions):
    routes = _ForcedRoutes(decisions)
    token = _forced.set(routes)
    try:
        yield
        if routes.used != routes.total:
            raise RuntimeError(f"routing override: {routes.total} decisions given, "
                               f"consumed {routes.used}")
    finally:
        _forced.reset(token)


def next_override(tokens: int, experts: int, top_k: int, device) -> torch.Tensor | None:
    """The next forced ``[tokens, k]`` decision as int32 on ``device`` after
    checking it (shape, id range, no expert twice in a row); None when no
    override is active."""
    routes = _forced.get()
    if routes is None:
        return None
    index = routes.used
    ids = routes.take().long()
    want = (int(tokens), int(top_k))
    if tuple(ids.shape) != want:
        raise ValueError(f"forced routing decision {index} has shape {tuple(ids.shape)}, "
                         f"the router expects {want}")
    if ids.numel() and (int(ids.min()) < 0 or int(ids.max()) >= experts):
        raise ValueError(f"forced routing decision {index} names an expert outside "
                         f"[0, {experts})")
    ranked = ids.sort(dim=-1).values
    if bool((ranked[:, 1:] == ranked[:, :-1]).any()):
        raise ValueError(f"forced routing decision {index} picks a duplicate expert for a token")
    return ids.to(device=device, dtype=torch.int32)


__all__ = [
    "current_route_weight_precision",
    "next_override",
    "route_weight_precision",
    "routing_override",
]
