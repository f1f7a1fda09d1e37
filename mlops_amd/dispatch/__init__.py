"""Dispatch: exact-ID implementation registry, selection and context controls."""

from .context import (
    capture_dispatch,
    deterministic_kernels,
    deterministic_required,
    dispatch_manifest,
    set_deterministic_kernels,
    set_implementations,
    set_weight_gradient_dtype,
    use_implementation,
    use_implementations,
    weight_gradient_dtype,
    weight_gradients_at,
)
from .costs import CostHints, estimate_implementation, flop_formula, has_flop_formula
from .registry import (
    Implementation,
    SupportResult,
    implementation_registry,
    register_implementation,
)
from .resolution import explain_implementation, resolve_implementation

__all__ = [
    "CostHints",
    "Implementation",
    "SupportResult",
    "capture_dispatch",
    "deterministic_kernels",
    "deterministic_required",
    "dispatch_manifest",
    "estimate_implementation",
    "explain_implementation",
    "flop_formula",
    "has_flop_formula",
    "implementation_registry",
    "register_implementation",
    "resolve_implementation",
    "set_deterministic_kernels",
    "set_implementations",
    "set_weight_gradient_dtype",
    "use_implementation",
    "use_implementations",
    "weight_gradient_dtype",
    "weight_gradients_at",
]
