"""Dispatch settings that belong to the calling context.

Four settings travel with the caller (thread / asyncio task), each readable
anywhere below it and restorable on exit:

* forced implementations, ``operation -> implementation ID`` (checked against
  the catalog when set; also read from ``MLOPS_IMPLEMENTATIONS="op=id,..."``);
* the dtype weight gradients are returned at (``None``: each weight's own);
* whether bitwise-repeatable kernels were requested;
* an optional trace that counts which implementation each resolution chose.

The function names and their meaning are the reference's control surface
(``src/mlops/dispatch/context.py``); here all four live in one immutable
record in a single context variable, and every scoped helper swaps that
record for the duration of its block.
"""

from __future__ import annotations

import os
import re
from contextlib import contextmanager
from contextvars import ContextVar
from dataclasses import dataclass, field, replace
from types import MappingProxyType
from typing import Mapping

import torch

ENVIRONMENT_OVERRIDES = "MLOPS_IMPLEMENTATIONS"
_PAIR = re.compile(r"^\s*([^\s=,]+)\s*=\s*([^\s=,]+)\s*$")


@dataclass(frozen=True)
class _Settings:
    forced: Mapping[str, str] = field(default_factory=lambda: MappingProxyType({}))
    gradient_dtype: torch.dtype | None = None
    deterministic: bool = False
    trace: dict | None = None


_SETTINGS: ContextVar[_Settings] = ContextVar("mlops_amd_dispatch_settings",
                                              default=_Settings())


@contextmanager
def _scoped(**changes):
    token = _SETTINGS.set(replace(_SETTINGS.get(), **changes))
    try:
        yield
    finally:
        _SETTINGS.reset(token)


def _update(**changes) -> None:
    _SETTINGS.set(replace(_SETTINGS.get(), **changes))


# ------------------------------------------------------------- forced choices
def implementation_override(operation: str) -> str | None:
    """The implementation ID forced for ``operation`` here, or None."""
    return _SETTINGS.get().forced.get(str(operation))


def _validated(choices: Mapping[str, str]) -> dict[str, str]:
    from .registry import implementations_for

    checked = {}
    for operation, wanted in choices.items():
        operation, wanted = str(operation), str(wanted)
        available = implementations_for(operation)
        if wanted not in available:
            raise ValueError(f"unknown implementation {wanted!r} for operation {operation!r} "
                             f"(registered: {', '.join(sorted(available))})")
        checked[operation] = wanted
    return checked


def _forced_with(choices: Mapping[str, str]) -> Mapping[str, str]:
    return MappingProxyType({**_SETTINGS.get().forced, **choices})


@contextmanager
def use_implementations(overrides: Mapping[str, str]):
    """Force the given implementation IDs inside the block; choices made by
    enclosing blocks for other operations still hold."""
    chosen = _validated(overrides)
    with _scoped(forced=_forced_with(chosen)):
        yield MappingProxyType(chosen)


@contextmanager
def use_implementation(operation: str, implementation_id: str):
    """Force one operation's implementation inside the block."""
    with use_implementations({operation: implementation_id}) as chosen:
        yield chosen[str(operation)]


def set_implementations(overrides: Mapping[str, str]) -> None:
    """Force implementation IDs for the rest of the calling context."""
    _update(forced=_forced_with(_validated(overrides)))


def apply_environment_overrides() -> Mapping[str, str]:
    """Force what ``MLOPS_IMPLEMENTATIONS`` lists (``op=id`` pairs separated by
    commas) and return it; an empty or unset variable forces nothing."""
    text = os.environ.get(ENVIRONMENT_OVERRIDES, "")
    if not text.strip():
        return MappingProxyType({})
    pairs = {}
    for item in text.split(","):
        match = _PAIR.match(item)
        if match is None:
            raise ValueError(f"cannot read {item!r} in {ENVIRONMENT_OVERRIDES}: each entry "
                             "must be operation=implementation_id")
        pairs[match.group(1)] = match.group(2)
    set_implementations(pairs)
    return MappingProxyType(pairs)


# -------------------------------------------------------------- determinism
def deterministic_required() -> bool:
    return _SETTINGS.get().deterministic


@contextmanager
def deterministic_kernels(enabled: bool = True):
    """Request bitwise-repeatable kernels inside the block. The MI355X MoE
    kernels fix every reduction order and use no float atomics, so they are
    repeatable whether or not this is set."""
    with _scoped(deterministic=bool(enabled)):
        yield bool(enabled)


def set_deterministic_kernels(enabled: bool = True) -> None:
    _update(deterministic=bool(enabled))


# ----------------------------------------------------- weight-gradient dtype
def _gradient_dtype(dtype):
    if dtype is None or (isinstance(dtype, torch.dtype) and dtype.is_floating_point):
        return dtype
    raise ValueError(f"a weight-gradient dtype must be a floating torch dtype or None, "
                     f"not {dtype!r}")


def weight_gradient_dtype() -> torch.dtype | None:
    """The dtype weight gradients come back at; None means each weight's own."""
    return _SETTINGS.get().gradient_dtype


@contextmanager
def weight_gradients_at(dtype: torch.dtype | None):
    """Return weight gradients at ``dtype`` inside the block (the sums
    themselves stay fp32)."""
    with _scoped(gradient_dtype=_gradient_dtype(dtype)):
        yield dtype


def set_weight_gradient_dtype(dtype: torch.dtype | None) -> None:
    _update(gradient_dtype=_gradient_dtype(dtype))


# ------------------------------------------------------------------ tracing
@contextmanager
def capture_dispatch():
    """Count, per operation, the implementations resolved inside the block."""
    trace: dict[str, dict[str, int]] = {}
    with _scoped(trace=trace):
        yield trace


def record_dispatch(operation: str, implementation_id: str) -> None:
    trace = _SETTINGS.get().trace
    if trace is None or torch.compiler.is_compiling():
        return
    per_operation = trace.setdefault(str(operation), {})
    key = str(implementation_id)
    per_operation[key] = per_operation.get(key, 0) + 1


def dispatch_manifest(trace: Mapping[str, Mapping[str, int]]) -> Mapping[str, str]:
    """``{operation: implementation_id}`` from a capture in which every
    operation resolved to exactly one implementation."""
    manifest = {}
    for operation, counts in trace.items():
        chosen = sorted(name for name, count in counts.items() if count)
        if len(chosen) != 1:
            raise ValueError(f"{operation!r} resolved to {chosen} in this capture; a manifest "
                             "pins one implementation per operation")
        manifest[str(operation)] = chosen[0]
    return MappingProxyType(manifest)


__all__ = [
    "ENVIRONMENT_OVERRIDES",
    "apply_environment_overrides",
    "capture_dispatch",
    "deterministic_kernels",
    "deterministic_required",
    "dispatch_manifest",
    "implementation_override",
    "record_dispatch",
    "set_deterministic_kernels",
    "set_implementations",
    "set_weight_gradient_dtype",
    "use_implementation",
    "use_implementations",
    "weight_gradient_dtype",
    "weight_gradients_at",
]
