"""The fused-MoE op boundary, HIP backend.

Mirrors the reference's public op and plugin API in
veomni/ops/kernels/moe/__init__.py:

* ``fused_moe_forward`` (:30-65) - asserts bf16/fp16, resolves ``layer_key``,
  forwards to the bound backend pointer ``_fused_moe_forward``;
* ``apply_veomni_fused_moe_patch`` (:68-114) - binds the pointer by name; this
  module answers ``"hip"`` and raises ``ValueError`` for anything else;
* ``_make_moe_experts_adapter`` (:123-158) - adapts the OpSlot call
  ``(self, hidden_states, top_k_index, top_k_weights)`` to the raw signature;
* ``KernelSpec(name="hip", op_name="moe_experts", variant="standard")`` -
  registered with a gfx950 hardware gate (config value
  ``moe_implementation="fused_hip"``).

``hip_fused_moe_forward`` is the raw backend (the role of
``group_gemm_fused_moe_forward``, veomni/ops/kernels/moe/group_gemm.py:634-961):
with a registered ``LayerPlacement`` for ``layer_key`` it applies the
source-aware ``M`` table, otherwise every logical expert is its own slot.

Where the router weights enter follows the reference's two branches
(group_gemm.py:655, :937-961): a layer with a registered placement (PlaceMoE
runs under expert parallelism) gets the EP arithmetic, weights applied in the
combine; a layer without one gets the non-EP arithmetic, weights applied to
the fc2 input.  ``set_router_weight_point`` fixes either for every layer.
"""

from __future__ import annotations

import torch

from .experts import expert_layer
from .kernel_registry import KERNEL_REGISTRY, HardwareRequirement, KernelSpec
from .placement import PLACEMENTS

_fused_moe_forward = None

# "auto" (by placement, as above), "combine" (EP arithmetic) or "fc2_input"
# (non-EP arithmetic).
_ROUTER_WEIGHT_POINTS = ("auto", "combine", "fc2_input")
_ROUTER_WEIGHT_POINT = "auto"


def set_router_weight_point(point: str) -> str:
    """Where the hip backend applies the router weights: ``"combine"`` (the
    EP branch's ``rank_dedup_combine``), ``"fc2_input"`` (the non-EP branch's
    ``fc1_activation * scattered_gate_weight``) or ``"auto"`` (the default:
    ``"combine"`` for layers with a registered placement, else
    ``"fc2_input"``).  Returns the previous setting."""
    global _ROUTER_WEIGHT_POINT
    if point not in _ROUTER_WEIGHT_POINTS:
        raise ValueError(f"router weight point must be one of {_ROUTER_WEIGHT_POINTS}, got {point!r}")
    prev, _ROUTER_WEIGHT_POINT = _ROUTER_WEIGHT_POINT, point
    return prev


def fused_moe_forward(
    num_experts: int,
    routing_weights: torch.Tensor,
    selected_experts: torch.Tensor,
    hidden_states: torch.Tensor,
    fc1_1_weight: torch.Tensor | None,
    fc1_2_weight: torch.Tensor | None,
    fc2_weight: torch.Tensor,
    fc1_1_2_weight: torch.Tensor | None = None,
    layer_key: str | None = None,
):
    if _fused_moe_forward is None:
        raise NotImplementedError("No fused MoE kernel is available. Please check your environment.")
    assert routing_weights.dtype in [torch.bfloat16, torch.float16], (
        f"routing_weights dtype must be bfloat16 or float16 for fused MoE kernel, but got {routing_weights.dtype}"
    )
    assert hidden_states.dtype in [torch.bfloat16, torch.float16], (
        f"hidden_states dtype must be bfloat16 or float16 for fused MoE kernel, but got {hidden_states.dtype}"
    )
    if layer_key is None:
        layer_key = PLACEMENTS.key_from_params(fc1_1_2_weight, fc2_weight, fc1_1_weight, fc1_2_weight)
    kwargs = {"layer_key": layer_key} if layer_key is not None else {}
    return _fused_moe_forward(
        num_experts, routing_weights, selected_experts, hidden_states, fc1_1_weight, fc1_2_weight, fc2_weight,
        fc1_1_2_weight, **kwargs,
    )


def hip_fused_moe_forward(
    num_experts: int,
    routing_weights: torch.Tensor,
    selected_experts: torch.Tensor,
    hidden_states: torch.Tensor,
    fc1_1_weight: torch.Tensor | None,
    fc1_2_weight: torch.Tensor | None,
    fc2_weight: torch.Tensor,
    fc1_1_2_weight: torch.Tensor | None = None,
    layer_key: str | None = None,
) -> torch.Tensor:
    """Raw HIP backend: [..., H] -> [..., H] for one GPU's physical copies."""
    if fc1_1_2_weight is not None:
        if fc1_1_weight is not None or fc1_2_weight is not None:
            raise ValueError("Provide either split fc1 weights or merged fc1_1_2_weight, not both.")
    elif fc1_1_weight is None or fc1_2_weight is None:
        raise ValueError("Split fc1 mode requires both fc1_1_weight and fc1_2_weight.")
    shape = hidden_states.shape
    hidden = hidden_states.reshape(-1, shape[-1]).contiguous()
    sel = selected_experts.reshape(hidden.shape[0], -1)
    # router weights in the hidden states' dtype (bf16 or fp16), which every
    # rounding point of the layer then uses
    w = routing_weights.reshape(sel.shape).to(hidden.dtype).contiguous()
    placement = PLACEMENTS.get(layer_key)
    mapping = sources = recorder = None
    source = 0
    if placement is not None:
        if placement.num_experts != int(num_experts):
            raise ValueError(
                f"layer {layer_key} was registered with {placement.num_experts} experts, called with {num_experts}"
            )
        if placement.num_slots != int(fc2_weight.shape[0]):
            raise ValueError(
                f"layer {layer_key} has {placement.num_slots} physical slots but the weights hold "
                f"{int(fc2_weight.shape[0])}"
            )
        mapping = placement.mapping_for_device(hidden.device)
        sources = placement.token_sources
        source = placement.source
        recorder = placement.record_slot_tokens
    elif int(fc2_weight.shape[0]) < int(num_experts):
        raise ValueError(
            f"{int(fc2_weight.shape[0])} expert weights cannot serve {num_experts} experts without a placement"
        )
    point = _ROUTER_WEIGHT_POINT
    if point == "auto":
        point = "combine" if placement is not None else "fc2_input"
    out = expert_layer(
        hidden, w, sel, fc2_weight, fc1_1_2_weight=fc1_1_2_weight, fc1_1_weight=fc1_1_weight,
        fc1_2_weight=fc1_2_weight, mapping=mapping, sources=sources, source=source, recorder=recorder,
        weighted_input=point == "fc2_input",
    )
    return out.reshape(shape)


def apply_veomni_fused_moe_patch(fused_moe_kernel: str = "hip") -> None:
    """Bind ``_fused_moe_forward``.  ``"hip"`` needs a gfx950 GPU; other names
    raise ``ValueError`` (a wrapper may intercept its own names first)."""
    global _fused_moe_forward
    if fused_moe_kernel == "hip":
        hw = HardwareRequirement(device_type="gpu", arch="gfx950")
        if not hw.is_satisfied():
            raise RuntimeError("fused_moe_kernel='hip' requires an AMD gfx950 (MI355X) GPU.")
        _fused_moe_forward = hip_fused_moe_forward
    else:
        raise ValueError(f"Invalid fused_moe_kernel: {fused_moe_kernel!r}. Expected one of: 'hip'.")


def _make_moe_experts_adapter(raw_forward):
    """OpSlot signature -> raw signature; router weights are cast to the
    hidden dtype and ``gate_up_proj`` is passed as merged fc1."""

    def adapter(self, hidden_states, top_k_index, top_k_weights):
        layer_key = PLACEMENTS.key_from_params(self.gate_up_proj, self.down_proj) or getattr(
            self, "_veomni_physical_load_layer_key", None
        )
        return raw_forward(
            num_experts=self.num_experts,
            routing_weights=top_k_weights.to(hidden_states.dtype),
            selected_experts=top_k_index,
            hidden_states=hidden_states,
            fc1_1_weight=None,
            fc1_2_weight=None,
            fc2_weight=self.down_proj,
            fc1_1_2_weight=self.gate_up_proj,
            layer_key=layer_key,
        )

    return adapter


def _hip_kernel_factory():
    return _make_moe_experts_adapter(hip_fused_moe_forward)


HIP_KERNEL_SPEC = KernelSpec(
    name="hip",
    op_name="moe_experts",
    variant="standard",
    factory=_hip_kernel_factory,
    hardware=HardwareRequirement(device_type="gpu", arch="gfx950"),
    description="gfx950 HIP SwiGLU grouped-GEMM fused MoE (PlaceMoE source-aware mapping)",
)
KERNEL_REGISTRY.register(HIP_KERNEL_SPEC)
