"""mlops_amd -- the block-FP8 MoE expert path of mlops, MI355X-native.

Public surface (mirrors the reference package's MoE surface):

* ``mlops_amd.moe(...)`` -- the routed MoE operation;
* ``mlops_amd.explicit.moe.forward/backward`` -- the manual VJP surface;
* ``mlops_amd.dispatch`` -- implementation registry and context controls;
* ``mlops_amd.BlockFP8Weight`` -- 128x128 block-scaled e4m3 expert weights;
* ``mlops_amd.routing`` -- route-weight precision and routing overrides.

The one implementation, ``mi355x.moe.block_fp8``, runs hand-written HIP
kernels for gfx950 from ``libmlops_mi355x.so`` (``include/mlops_mi355x.h``).
"""

from . import dispatch, explicit, routing
from .block_fp8 import BlockFP8Weight
from .dispatch.context import apply_environment_overrides
from .moe import moe

apply_environment_overrides()

__all__ = ["BlockFP8Weight", "dispatch", "explicit", "moe", "routing"]
