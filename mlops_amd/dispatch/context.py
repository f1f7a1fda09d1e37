"""Context-local dispatch choices: forced implementations, the weight-gradient
dtype, determinism requests and dispatch capture.

Follows the reference's control surface (``src/mlops/dispatch/context.py:20-240``):
``use_implementation(s)``/``set_implementations``, the ``MLOPS_IMPLEMENTATIONS``
environment variable, ``weight_gradients_at``/``set_weight_gradient_dtype``,
``deterministic_kernels`` and ``capture_dispatch``/``dispatch_manifest``.
"""

from __future__ import annotations

import os
from contextlib import contextmanager
from contextvars import ContextVar
from types import MappingProxyType
from typing import Mapping

import torch

_FORCED: ContextVar[Mapping[str, str]] = ContextVar(
    "mlops_amd_forced_implementations", default=MappingProxyType({})
)
_TRACE: ContextVar[dict | None] = ContextVar("mlops_amd_dispatch_trace", default=None)
_DETERMINISTIC: ContextVar[bool] = ContextVar("mlops_amd_deterministic", default=False)
_GRAD_DTYPE: ContextVar[torch.dtype | None] = ContextVar(
    "mlops_amd_weight_gradient_dtype", default=None
)

ENVIRONMENT_OVERRIDES = "MLOPS_IMPLEMENTATIONS"


def implementation_override(operation: str) -> str | None:
    """The implementation forced for ``operation`` in this context, if any."""
    return _FORCED.get().get(str(operation))


def _checked(overrides: Mapping[str, str]) -> dict[str, str]:
    from .registry import implementations_for

    result = {}
    for operation, implementation_id in overrides.items():
        known = implementations_for(str(operation))
        if str(implementation_id) not in known:
            raise ValueError(
                f"unknown implementation {implementation_id!r} for {operation!r}; "
                f"choose one of {sorted(known)}"
            )
        result[str(operation)] = str(implementation_id)
    return result


def _with(extra: Mapping[str, str]) -> Mapping[str, str]:
    merged = dict(_FORCED.get())
    merged.update(extra)
    return MappingProxyType(merged)


@contextmanager
def use_implementations(overrides: Mapping[str, str]):
    """Force exact implementations inside the block (outer choices inherited)."""
    chosen = _checked(overrides)
    token = _FORCED.set(_with(chosen))
    try:
        yield MappingProxyType(chosen)
    finally:
        _FORCED.reset(token)


@contextmanager
def use_implementation(operation: str, implementation_id: str):
    """Force one implementation for one operation inside the block."""
    with use_implementations({operation: implementation_id}) as chosen:
        yield chosen[str(operation)]


def set_implementations(overrides: Mapping[str, str]) -> None:
    """Force exact implementations from here on in the calling context."""
    _FORCED.set(_with(_checked(overrides)))


def apply_environment_overrides() -> Mapping[str, str]:
    """Apply ``MLOPS_IMPLEMENTATIONS="op=id,op=id"``; returns what was applied."""
    text = os.environ.get(ENVIRONMENT_OVERRIDES, "").strip()
    if not text:
        return MappingProxyType({})
    parsed: dict[str, str] = {}
    for item in text.split(","):
        operation, sep, implementation_id = item.partition("=")
        if not sep or not operation.strip() or not implementation_id.strip():
            raise ValueError(
                f"{ENVIRONMENT_OVERRIDES} expects comma-separated "
                f"operation=implementation_id pairs, got {item!r}"
            )
        parsed[operation.strip()] = implementation_id.strip()
    set_implementations(parsed)
    return MappingProxyType(parsed)


def deterministic_required() -> bool:
    return _DETERMINISTIC.get()


@contextmanager
def deterministic_kernels(enabled: bool = True):
    """Ask for bitwise-repeatable kernels. Every kernel of the MI355X MoE
    provider is ordered (no float atomics), so it honours this unconditionally."""
    token = _DETERMINISTIC.set(bool(enabled))
    try:
        yield bool(enabled)
    finally:
        _DETERMINISTIC.reset(token)


def set_deterministic_kernels(enabled: bool = True) -> None:
    _DETERMINISTIC.set(bool(enabled))


def _floating(dtype):
    if dtype is not None and (not isinstance(dtype, torch.dtype) or not dtype.is_floating_point):
        raise ValueError(f"weight gradients need a floating dtype or None; got {dtype!r}")
    return dtype


def weight_gradient_dtype() -> torch.dtype | None:
    """The dtype weight gradients are returned at; ``None`` = each weight's own."""
    return _GRAD_DTYPE.get()


@contextmanager
def weight_gradients_at(dtype: torch.dtype | None):
    """Return weight gradients at ``dtype`` inside the block (sums stay fp32)."""
    token = _GRAD_DTYPE.set(_floating(dtype))
    try:
        yield dtype
    finally:
        _GRAD_DTYPE.reset(token)


def set_weight_gradient_dtype(dtype: torch.dtype | None) -> None:
    _GRAD_DTYPE.set(_floating(dtype))


@contextmanager
def capture_dispatch():
    """Record which implementation each resolution picked inside the block."""
    trace: dict[str, dict[str, int]] = {}
    token = _TRACE.set(trace)
    try:
        yield trace
    finally:
        _TRACE.reset(token)


def record_dispatch(operation: str, implementation_id: str) -> None:
    if torch.compiler.is_compiling():
        return
    trace = _TRACE.get()
    if trace is None:
        return
    counts = trace.setdefault(str(operation), {})
    counts[str(implementation_id)] = counts.get(str(implementation_id), 0) + 1


def dispatch_manifest(trace: Mapping[str, Mapping[str, int]]) -> Mapping[str, str]:
    """Turn an unambiguous capture into ``{operation: implementation_id}``."""
    manifest = {}
    for operation, counts in trace.items():
        used = [name for name, count in counts.items() if count]
        if len(used) != 1:
            raise ValueError(
                f"operation {operation!r} exercised {sorted(used)}; "
                "a frozen manifest requires exactly one implementation"
            )
        manifest[str(operation)] = used[0]
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
