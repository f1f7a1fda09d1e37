"""mlops_amd -- the block-FP8 MoE expert path of mlops, MI355X-native.

Public surface (mirrors the reference package's MoE surface):

* ``mlops_amd.moe(...)`` -- the routed MoE operation;
* ``mlops_amd.explicit.moe.forward/backward`` -- the manual VJP surface;
* ``mlops_amd.dispatch`` -- implementation registry and context controls;
* ``mlops_amd.BlockFP8Weight`` -- 128x128 block-scaled e4m3 expert weights;
* ``mlops_amd.RowFP8Weight`` (also ``QuackFP8Weight``) -- per-row scaled e4m3
  expert weights in both orientations (``compute_precision="fp8_current"``);
* ``mlops_amd.routing`` -- route-weight precision and routing overrides;
* ``mlops_amd.checkpoint`` -- block-FP8 safetensors into `BlockFP8Weight`.

The implementations (``mi355x.moe.block_fp8``, its two-region form
``mi355x.moe.composed``, and ``mi355x.moe.fp8_current``) run hand-written HIP
kernels for gfx950 from ``libmlops_mi355x.so`` (``include/mlops_mi355x.h``).
"""

from . import checkpoint, dispatch, explicit, routing
from .block_fp8 import BlockFP8Weight
from .row_fp8 import QuackFP8Weight, RowFP8Weight
from .dispatch.context import apply_environment_overrides
from .moe import moe

apply_environment_overrides()

__all__ = ["BlockFP8Weight", "QuackFP8Weight", "RowFP8Weight", "checkpoint", "dispatch",
           "explicit", "moe", "routing"]
