"""Explicit catalog of the modules that register implementations.

As in the reference (``src/mlops/providers/__init__.py:11-76``) discovery is an
explicit import list, loaded once on first use of the registry.
"""

from __future__ import annotations

from importlib import import_module

_CATALOG = (
    "mlops_amd.providers.mi355x.moe",
    "mlops_amd.providers.mi355x.moe_composed",
    "mlops_amd.providers.mi355x.moe_current",
)
_REGISTERED = False


def ensure_implementations_registered() -> None:
    global _REGISTERED
    if _REGISTERED:
        return
    _REGISTERED = True
    try:
        for name in _CATALOG:
            import_module(name)
    except Exception:
        _REGISTERED = False
        raise


__all__ = ["ensure_implementations_registered"]
