"""Implementation dispatch for the MoE operation: the catalog of records
(`registry`), the choice for one call (`resolution`), context-local settings
(`context`), cost figures (`costs`, `logical_costs`) and a finite-difference
check of one implementation's backward (`gradcheck`). The names exported
here are the subset of the reference's ``mlops.dispatch`` API the MoE path
uses."""

from . import context, costs, gradcheck, registry, resolution
from .context import *  # noqa: F401,F403
from .costs import *  # noqa: F401,F403
from .gradcheck import *  # noqa: F401,F403
from .registry import *  # noqa: F401,F403
from .resolution import *  # noqa: F401,F403

_INTERNAL = {"ENVIRONMENT_OVERRIDES", "implementation_override", "record_dispatch",
             "frozen_implementation", "implementations_for", "apply_environment_overrides"}
__all__ = sorted({name for module in (context, costs, gradcheck, registry, resolution)
                  for name in module.__all__} - _INTERNAL)
