"""The catalog of implementations, keyed by operation and exact ID.

The records are the plugin contract of the reference registry
(``src/mlops/dispatch/registry.py``): an `Implementation` names one
operation, one unique ID, its provider, a priority and whether it is
deterministic; it carries a metadata-only ``supports`` check, the autograd
entry ``apply`` and, optionally, the explicit ``forward``/``backward`` pair
and a cost ``estimate``. Here the catalog is a small class of nested dicts;
reads go through read-only views, and providers are imported on first read
so that every built-in implementation is present.
"""

from __future__ import annotations

from collections.abc import Callable, Mapping
from dataclasses import dataclass
from types import MappingProxyType


@dataclass(frozen=True)
class SupportResult:
    """One implementation's answer for one concrete call: accepted, or why not."""

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
    """A stateless implementation of one semantic operation (see module doc)."""

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
        missing = [name for name in ("operation", "implementation_id", "provider")
                   if not getattr(self, name)]
        if missing:
            raise ValueError(f"an implementation record needs a non-empty {', '.join(missing)}")
        if (self.forward is None) != (self.backward is None):
            raise ValueError(f"{self.implementation_id} gives only one of forward/backward; "
                             "the explicit surface needs them together")

    @property
    def explicit(self) -> bool:
        """Whether the record exposes the explicit forward/backward pair."""
        return self.forward is not None


class _Catalog:
    def __init__(self) -> None:
        self.tables: dict[str, dict[str, Implementation]] = {}
        self._providers_loaded = False

    def add(self, record: Implementation) -> Implementation:
        table = self.tables.setdefault(str(record.operation), {})
        key = str(record.implementation_id)
        if key in table:
            raise ValueError(f"implementation {key!r} of {record.operation!r} is already "
                             "registered (duplicate IDs are not allowed)")
        table[key] = record
        return record

    def load_providers(self) -> None:
        if not self._providers_loaded:
            self._providers_loaded = True
            from ..providers import ensure_implementations_registered

            ensure_implementations_registered()

    def table(self, operation: str) -> dict[str, Implementation]:
        self.load_providers()
        found = self.tables.get(str(operation))
        if found is None:
            raise ValueError(f"no operation named {operation!r} is registered "
                             f"(known: {', '.join(sorted(self.tables))})")
        return found


_catalog = _Catalog()


def register_implementation(implementation: Implementation) -> Implementation:
    """Add a record to the catalog (its ID must be new) and return it."""
    return _catalog.add(implementation)


def implementation_registry() -> Mapping[str, Mapping[str, Implementation]]:
    """Read-only view of every operation's implementations."""
    _catalog.load_providers()
    return MappingProxyType({operation: MappingProxyType(dict(table))
                             for operation, table in sorted(_catalog.tables.items())})


def implementations_for(operation: str) -> Mapping[str, Implementation]:
    """Read-only view of one operation's implementations, by ID."""
    return MappingProxyType(_catalog.table(operation))


def frozen_implementation(operation: str, implementation_id: str) -> Implementation:
    """The record registered under an exact ID."""
    return _catalog.table(operation)[str(implementation_id)]


__all__ = [
    "Implementation",
    "SupportResult",
    "frozen_implementation",
    "implementation_registry",
    "implementations_for",
    "register_implementation",
]
