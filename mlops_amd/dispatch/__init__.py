"""Implementation dispatch for the MoE operation: the catalog of records
(`registry`), the choice for one call (`resolution`), context-local settings
(`context`) and cost figures (`costs`, `logical_costs`). The names exported
here are the subset of the reference's ``mlops.dispatch`` API the MoE path
uses."""

from . import context, costs, registry, resolution
from .context import *  # noqa: F401,F403
from .costs import *  # noqa: F401,F403
from .registry import *  # noqa: F401,F403
from .resolution import *  # noqa: F401,F403

_INTERNAL = {"ENVIRONMENT_OVERRIDES", "implementation_override", "record_dispatch",
             "frozen_implementation", "implementations_for", "apply_environment_overrides"}
__all__ = sorted({name for module in (context, costs, registry, resolution)
                  for name in module.__all__} - _INTERNAL)
