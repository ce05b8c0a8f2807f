"""placemoe_amd - one GPU's share of the PlaceMoE expert layer on AMD MI355X (gfx950).

Import order registers the ``"hip"`` ``moe_experts`` kernel with the registry.
The HIP library is loaded on first use; without it every op raises.
"""

from . import kernel_registry, dispatch, placement  # noqa: F401
from .dispatch import OpSlot, veomni_moe_experts_forward  # noqa: F401
from .experts import expert_layer  # noqa: F401
from .fused_moe import (  # noqa: F401
    apply_veomni_fused_moe_patch,
    fused_moe_forward,
    hip_fused_moe_forward,
    set_router_weight_point,
)
from .kernel_registry import KERNEL_REGISTRY, HardwareRequirement, KernelSpec  # noqa: F401
from .placement import PLACEMENTS, LayerPlacement, LayerPlan, PlaceMoETopology, mirrored_r2_plan  # noqa: F401
from .replica import OverlappedReplicaSync, fold_replica_gradients, sync_redundant_gradients  # noqa: F401
from .statistics import ProfileStatistics, RouteStatisticsRecorder, profile_route_statistics  # noqa: F401

__version__ = "0.1.0"
