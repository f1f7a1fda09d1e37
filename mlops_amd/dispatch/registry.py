"""Implementation records and the process-local catalog of the ``moe`` operation.

Mirrors the reference's registry contract (``src/mlops/dispatch/registry.py:12-69``):
an implementation is an immutable record keyed by an exact ID, its forward and
backward come as a pair or not at all, and registering an ID twice is an error.
"""

from __future__ import annotations

from collections.abc import Callable, Mapping
from dataclasses import dataclass
from types import MappingProxyType


@dataclass(frozen=True)
class SupportResult:
    """Whether an implementation accepts one concrete invocation, and why not."""

    supported: bool
    reason: str = ""

    @classmethod
    def yes(cls) -> "SupportResult":
        return cls(True, "supported")

    @classmethod
    def no(cls, reason: str) -> "SupportResult":
        return cls(False, str(reason))

    def __bool__(self) -> bool:
        return self.supported


@dataclass(frozen=True)
class Implementation:
    """One stateless implementation of one semantic operation.

    ``supports`` inspects metadata only; ``apply`` is the autograd-visible
    entry; ``forward``/``backward`` form the explicit (manual VJP) surface.
    """

    operation: str
    implementation_id: str
    provider: str
    priority: int
    deterministic: bool
    supports: Callable
    apply: Callable
    forward: Callable | None = None
    backward: Callable | None = None
    estimate: Callable | None = None

    def __post_init__(self) -> None:
        if not (self.operation and self.implementation_id and self.provider):
            raise ValueError("operation, implementation_id and provider must be non-empty")
        if (self.forward is None) is not (self.backward is None):
            raise ValueError(
                f"{self.implementation_id}: explicit forward and backward come together"
            )


_CATALOG: dict[str, dict[str, Implementation]] = {}


def register_implementation(implementation: Implementation) -> Implementation:
    """Add ``implementation`` to the catalog and return it; IDs are unique."""
    table = _CATALOG.setdefault(str(implementation.operation), {})
    key = str(implementation.implementation_id)
    if key in table:
        raise ValueError(
            f"duplicate implementation ID {key!r} for {implementation.operation!r}"
        )
    table[key] = implementation
    return implementation


def _ensure_loaded() -> None:
    from ..providers import ensure_implementations_registered

    ensure_implementations_registered()


def implementation_registry() -> Mapping[str, Mapping[str, Implementation]]:
    """A read-only snapshot of every registered implementation."""
    _ensure_loaded()
    return MappingProxyType(
        {op: MappingProxyType(dict(table)) for op, table in sorted(_CATALOG.items())}
    )


def implementations_for(operation: str) -> Mapping[str, Implementation]:
    """The implementations of one exact operation name."""
    _ensure_loaded()
    try:
        return MappingProxyType(_CATALOG[str(operation)])
    except KeyError as error:
        raise ValueError(f"unknown semantic operation {operation!r}") from error


def frozen_implementation(operation: str, implementation_id: str) -> Implementation:
    """The record registered under ``implementation_id``."""
    _ensure_loaded()
    return _CATALOG[str(operation)][str(implementation_id)]


__all__ = [
    "Implementation",
    "SupportResult",
    "frozen_implementation",
    "implementation_registry",
    "implementations_for",
    "register_implementation",
]
