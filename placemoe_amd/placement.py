"""PlaceMoE placement tables on one GPU: layout ``L``, source-aware mapping ``M``,
owners, copy tables, and the per-layer state the fused op reads.

The on-disk contract is the reference's: ``LayerPlan`` invariants
(veomni/distributed/moe/hiermoe/placemoe/types.py:114-177), the schema-v2
artifact (veomni/distributed/moe/hiermoe/placemoe/artifacts.py:28-95), the
mirrored-R2 seed (placemoe/seeds.py:24-48), copy-weight materialisation
(veomni/distributed/parallel_plan.py:73-124) and mapping-only hot updates
(veomni/distributed/moe/hiermoe/expert_swap.py:10920-10972).  Validation runs
on the host once per plan; the device sees only int64 ``M`` and int32 copy
tables, cached per device.
"""

from __future__ import annotations

from collections.abc import Mapping
from dataclasses import dataclass, field
from typing import Any

import numpy as np
import torch

EMPTY_EXPERT = -1
PLACEMOE_ARTIFACT_SCHEMA_VERSION = 2


def _ro_int64(value) -> np.ndarray:
    arr = np.array(value, dtype=np.int64, copy=True)
    arr.setflags(write=False)
    return arr


@dataclass(frozen=True)
class PlaceMoETopology:
    ep_size: int
    ranks_per_node: int
    num_experts: int
    slots_per_rank: int

    def __post_init__(self) -> None:
        for name in ("ep_size", "ranks_per_node", "num_experts", "slots_per_rank"):
            if getattr(self, name) <= 0:
                raise ValueError(f"{name} must be positive.")
        if self.ep_size % self.ranks_per_node:
            raise ValueError("ep_size must be divisible by ranks_per_node.")
        if self.total_slots < self.num_experts:
            raise ValueError("Physical capacity cannot hold one copy of every expert.")

    @property
    def total_slots(self) -> int:
        return self.ep_size * self.slots_per_rank

    def rank_of_slot(self, slot: int) -> int:
        if not 0 <= slot < self.total_slots:
            raise ValueError(f"Physical slot {slot} is outside the topology.")
        return slot // self.slots_per_rank


@dataclass(frozen=True)
class LayerPlan:
    """Physical layout ``slot_to_logical`` (L), runtime owners and the
    source-aware mapping ``source_logical_to_physical`` (M)."""

    slot_to_logical: np.ndarray
    source_logical_to_physical: np.ndarray
    owner_slots: np.ndarray

    def __post_init__(self) -> None:
        object.__setattr__(self, "slot_to_logical", _ro_int64(self.slot_to_logical))
        object.__setattr__(self, "source_logical_to_physical", _ro_int64(self.source_logical_to_physical))
        object.__setattr__(self, "owner_slots", _ro_int64(self.owner_slots))

    @property
    def copy_counts(self) -> np.ndarray:
        L = self.slot_to_logical
        return np.bincount(L[L != EMPTY_EXPERT], minlength=int(self.owner_slots.shape[0]))

    def validate(self, topology: PlaceMoETopology, *, additional_copies: int | None = None) -> None:
        L, M, owners = self.slot_to_logical, self.source_logical_to_physical, self.owner_slots
        E, S = topology.num_experts, topology.total_slots
        if L.shape != (S,):
            raise ValueError("Layout length does not match the physical slot capacity.")
        if M.shape != (topology.ep_size, E):
            raise ValueError("Mapping shape does not match [source_rank, logical_expert].")
        if owners.shape != (E,):
            raise ValueError("owner_slots must contain one runtime owner per logical expert.")
        if bool(((L < EMPTY_EXPERT) | (L >= E)).any()):
            raise ValueError("Layout contains an invalid logical expert ID.")
        counts = self.copy_counts
        if bool((counts[:E] < 1).any()):
            raise ValueError("Every logical expert must retain at least one physical copy.")
        if additional_copies is not None and int(counts.sum()) - E != additional_copies:
            raise ValueError("Layout does not use the requested additional-copy budget.")
        if bool(((M < 0) | (M >= S)).any()):
            raise ValueError("Mapping references a slot outside the topology.")
        if not np.array_equal(L[M], np.broadcast_to(np.arange(E, dtype=np.int64), M.shape)):
            raise ValueError("Mapping references a copy of the wrong logical expert.")
        if bool(((owners < 0) | (owners >= S)).any()):
            raise ValueError("Runtime owner references a slot outside the topology.")
        if not np.array_equal(L[owners], np.arange(E, dtype=np.int64)):
            raise ValueError("Runtime owner slots do not match their logical experts.")

    def to_runtime_payload(self) -> dict[str, Any]:
        return {
            "slot_to_logical": self.slot_to_logical.tolist(),
            "owner_slots": self.owner_slots.tolist(),
            "source_logical_to_physical": self.source_logical_to_physical.tolist(),
        }

    @classmethod
    def from_runtime_payload(cls, payload: Mapping[str, Any]) -> "LayerPlan":
        return cls(
            slot_to_logical=payload["slot_to_logical"],
            owner_slots=payload["owner_slots"],
            source_logical_to_physical=payload["source_logical_to_physical"],
        )


def mirrored_r2_plan(topology: PlaceMoETopology) -> LayerPlan:
    """Two copies per expert: first half of the ranks serves expert e from
    slot (r, s) = divmod(e, slots_per_rank), the second half from the mirror
    slot ``ep_size/2`` ranks later (placemoe/seeds.py:24-48)."""
    if topology.ep_size % 2 or topology.total_slots != 2 * topology.num_experts:
        raise ValueError("Mirrored R2 requires an even EP size and exactly two copies per expert.")
    E, spr, half = topology.num_experts, topology.slots_per_rank, topology.ep_size // 2
    rank, local = np.divmod(np.arange(E, dtype=np.int64), spr)
    first = rank * spr + local
    second = (rank + half) * spr + local
    layout = np.full(topology.total_slots, EMPTY_EXPERT, dtype=np.int64)
    layout[first] = np.arange(E)
    layout[second] = np.arange(E)
    mapping = np.empty((topology.ep_size, E), dtype=np.int64)
    mapping[:half] = first
    mapping[half:] = second
    plan = LayerPlan(slot_to_logical=layout, owner_slots=first, source_logical_to_physical=mapping)
    plan.validate(topology, additional_copies=E)
    return plan


def build_placemoe_artifact(plans: Mapping[str, LayerPlan], topology: PlaceMoETopology, *,
                            source: Mapping[str, Any] | None = None) -> dict[str, Any]:
    """Schema-v2 runtime artifact (placemoe/artifacts.py:28-63)."""
    if not plans:
        raise ValueError("A PlaceMoE artifact must contain at least one layer plan.")
    layers = {}
    for name, plan in plans.items():
        if not name:
            raise ValueError("Layer names must be non-empty.")
        plan.validate(topology)
        layers[name] = plan.to_runtime_payload()
    return {
        "schema_version": PLACEMOE_ARTIFACT_SCHEMA_VERSION,
        "source": {**dict(source or {}), "algorithm": "placemoe-v1", "initial_layout": "preloaded",
                   "requires_static_preload": True},
        "topology": {"ep_size": topology.ep_size, "ranks_per_node": topology.ranks_per_node,
                     "num_experts": topology.num_experts, "num_physical_slots": topology.total_slots,
                     "slots_per_rank": topology.slots_per_rank},
        "replay": {"actions_by_step": {"1": []}},
        "layers": layers,
    }


def validate_placemoe_artifact(payload: Mapping[str, Any]) -> dict[str, LayerPlan]:
    """Check a schema-v2 artifact and return its plans (placemoe/artifacts.py:66-95)."""
    if int(payload.get("schema_version", -1)) != PLACEMOE_ARTIFACT_SCHEMA_VERSION:
        raise ValueError("Unsupported PlaceMoE artifact schema version.")
    src = payload.get("source")
    if not isinstance(src, Mapping) or src.get("algorithm") != "placemoe-v1":
        raise ValueError("Artifact was not produced by the PlaceMoE optimizer.")
    topo = payload.get("topology")
    if not isinstance(topo, Mapping):
        raise ValueError("PlaceMoE artifact is missing its topology.")
    topology = PlaceMoETopology(
        ep_size=int(topo["ep_size"]), ranks_per_node=int(topo.get("ranks_per_node", topo["ep_size"])),
        num_experts=int(topo["num_experts"]), slots_per_rank=int(topo["slots_per_rank"]),
    )
    if int(topo.get("num_physical_slots", -1)) != topology.total_slots:
        raise ValueError("Artifact physical-slot count does not match its topology.")
    rows = payload.get("layers")
    if not isinstance(rows, Mapping) or not rows:
        raise ValueError("PlaceMoE artifact must contain a non-empty layer table.")
    plans = {}
    for name, row in rows.items():
        if not isinstance(name, str) or not isinstance(row, dict):
            raise ValueError("PlaceMoE layer entries must map names to plan objects.")
        plan = LayerPlan.from_runtime_payload(row)
        plan.validate(topology)
        plans[name] = plan
    return plans


def copy_table(slot_to_logical, num_experts: int) -> tuple[np.ndarray, np.ndarray]:
    """CSR copy table: copies of expert e are ``slots[offsets[e]:offsets[e+1]]``
    in slot order (``copy_slots_for_device``, expert_swap.py:520-550)."""
    L = np.asarray(slot_to_logical, dtype=np.int64)
    active = np.nonzero(L != EMPTY_EXPERT)[0]
    order = active[np.argsort(L[active], kind="stable")]
    counts = np.bincount(L[active], minlength=num_experts)
    offsets = np.zeros(num_experts + 1, dtype=np.int32)
    np.cumsum(counts, out=offsets[1:])
    return offsets, order.astype(np.int32)


def materialize_copy_weights(logical: torch.Tensor, slot_to_logical) -> torch.Tensor:
    """W_copy[c] = W_logical[L[c]]; zeros where ``L[c] == -1``
    (``_hiermoe_initial_layout_shard``, veomni/distributed/parallel_plan.py:114-123)."""
    L = torch.as_tensor(np.asarray(slot_to_logical, dtype=np.int64))
    if bool(((L < EMPTY_EXPERT) | (L >= logical.shape[0])).any()):
        raise ValueError("slot_to_logical contains an invalid expert.")
    out = logical.new_zeros((L.numel(),) + tuple(logical.shape[1:]))
    active = torch.nonzero(L >= 0).flatten()
    if active.numel():
        idx = active.to(logical.device)
        out.index_copy_(0, idx, logical.index_select(0, L[active].to(logical.device)))
    return out


@dataclass
class LayerPlacement:
    """Per-layer placement state on one GPU (the single-rank ``ExpertLayerState``,
    expert_swap.py:433-586): ``M`` rows per source, copy tables, and the
    tokens each copy has seen since the last gradient fold."""

    key: str
    num_experts: int
    slot_to_logical: np.ndarray
    source_logical_to_physical: np.ndarray
    owner_slots: np.ndarray
    source: int = 0  # the source row used when no per-token sources are given
    token_sources: torch.Tensor | None = None  # optional int64 [T] per-token source ids
    accumulated_slot_tokens: torch.Tensor | None = None
    placement_version: int = 0
    _device_cache: dict = field(default_factory=dict)

    @classmethod
    def from_plan(cls, key: str, plan: LayerPlan, num_experts: int, source: int = 0) -> "LayerPlacement":
        M = plan.source_logical_to_physical
        L = plan.slot_to_logical
        if M.ndim != 2 or M.shape[1] != num_experts:
            raise ValueError(f"mapping for {key} must be [sources, {num_experts}]")
        if bool(((M < 0) | (M >= L.shape[0])).any()):
            raise ValueError(f"PlaceMoE mapping for {key} references an invalid slot.")
        if not np.array_equal(L[M], np.broadcast_to(np.arange(num_experts), M.shape)):
            raise ValueError(f"PlaceMoE mapping for {key} references the wrong expert.")
        if not 0 <= source < M.shape[0]:
            raise ValueError(f"source {source} outside the mapping's {M.shape[0]} rows")
        return cls(key=key, num_experts=num_experts, slot_to_logical=np.array(L),
                   source_logical_to_physical=np.array(M), owner_slots=np.array(plan.owner_slots), source=source)

    @property
    def num_slots(self) -> int:
        return int(self.slot_to_logical.shape[0])

    def mapping_for_device(self, device: torch.device) -> torch.Tensor:
        key = ("M", device)
        if key not in self._device_cache:
            self._device_cache[key] = torch.as_tensor(self.source_logical_to_physical, dtype=torch.int64).to(device)
        return self._device_cache[key]

    def copy_tables_for_device(self, device: torch.device) -> tuple[torch.Tensor, torch.Tensor]:
        key = ("copies", device)
        if key not in self._device_cache:
            off, slots = copy_table(self.slot_to_logical, self.num_experts)
            self._device_cache[key] = (torch.as_tensor(off).to(device), torch.as_tensor(slots).to(device))
        return self._device_cache[key]

    def install_mapping(self, source_logical_to_physical) -> int:
        """Mapping-only hot update: same L, new M (expert_swap.py:10920-10972).
        Returns 1 if the mapping changed."""
        lut = np.asarray(source_logical_to_physical, dtype=np.int64)
        if lut.shape != self.source_logical_to_physical.shape:
            raise RuntimeError(
                f"PlaceMoE mapping for {self.key} has shape {lut.shape}, "
                f"expected {self.source_logical_to_physical.shape}."
            )
        if bool(((lut < 0) | (lut >= self.num_slots)).any()):
            raise RuntimeError(f"PlaceMoE mapping for {self.key} references an invalid slot.")
        if not np.array_equal(self.slot_to_logical[lut], np.broadcast_to(np.arange(self.num_experts), lut.shape)):
            raise RuntimeError(f"PlaceMoE mapping for {self.key} references the wrong expert.")
        changed = not np.array_equal(lut, self.source_logical_to_physical)
        self.source_logical_to_physical = lut.copy()
        self._device_cache = {k: v for k, v in self._device_cache.items() if k[0] != "M"}
        self.placement_version += int(changed)
        return int(changed)

    def record_slot_tokens(self, counts: torch.Tensor) -> None:
        """Accumulate per-copy token counts on the device (no host sync);
        ``record_local_expert_token_counts``, expert_swap.py:6200-6218."""
        counts = counts.detach().to(torch.int64)
        if self.accumulated_slot_tokens is None or self.accumulated_slot_tokens.shape != counts.shape:
            self.accumulated_slot_tokens = counts.clone()
        else:
            self.accumulated_slot_tokens.add_(counts)

    def clear_slot_tokens(self) -> None:
        self.accumulated_slot_tokens = None

    @classmethod
    def from_layer_state(cls, state, source_rank: int, key: str | None = None) -> "LayerStatePlacement":
        """A placement that reads ``L`` and ``M`` from the reference's own
        per-layer state on every call instead of keeping a copy (see
        ``LayerStatePlacement``)."""
        return LayerStatePlacement(state, source_rank, key=key)


class LayerStatePlacement:
    """Placement backed by the reference's ``ExpertLayerState``
    (veomni/distributed/moe/hiermoe/expert_swap.py:433-586), read on every
    call, so that the reference's controller stays the one owner of ``M``.

    Each forward routes with ``state.source_mapping_for_device(device,
    source_rank)`` (expert_swap.py:502-510), the device row of ``M`` the
    reference's own EP path gathers from; a mapping-only hot update
    (``_install_hot_update_mapping``, expert_swap.py:10920-10972) replaces
    ``state.source_logical_to_physical`` and clears that cache, so the next
    forward here sees the new ``M``.  A state without a source-rank LUT
    routes with ``state.mapping_for_device(device)`` (the owner table, as the
    reference does).  With per-token ``token_sources`` the whole ``[S, E]``
    table goes to the device, cached per table object and placement version.

    Duck-typed: the state needs ``key``, ``num_experts``,
    ``logical_to_physical``, ``slot_to_logical`` (or None: one copy per
    expert), ``source_logical_to_physical``, ``placement_version`` and the two
    ``*_mapping_for_device`` methods.
    """

    def __init__(self, state, source_rank: int, key: str | None = None):
        self.state = state
        self.key = key if key is not None else str(state.key)
        self.source_rank = int(source_rank)
        self.source = 0  # row 0 of the one-row table handed to the routing kernels
        self.token_sources: torch.Tensor | None = None
        self.accumulated_slot_tokens: torch.Tensor | None = None
        self._cache: dict = {}

    @property
    def num_experts(self) -> int:
        return int(self.state.num_experts)

    @property
    def slot_to_logical(self) -> np.ndarray:
        L = self.state.slot_to_logical
        if L is None:
            # no slot layout: slot logical_to_physical[e] holds expert e
            owners = np.asarray(torch.as_tensor(self.state.logical_to_physical).cpu(), dtype=np.int64)
            L = np.full(int(owners.max()) + 1 if owners.size else 0, EMPTY_EXPERT, dtype=np.int64)
            L[owners] = np.arange(owners.size)
            return L
        return np.asarray(torch.as_tensor(L).cpu(), dtype=np.int64)

    @property
    def owner_slots(self) -> np.ndarray:
        return np.asarray(torch.as_tensor(self.state.logical_to_physical).cpu(), dtype=np.int64)

    @property
    def source_logical_to_physical(self) -> np.ndarray | None:
        M = self.state.source_logical_to_physical
        return None if M is None else np.asarray(torch.as_tensor(M).cpu(), dtype=np.int64)

    @property
    def placement_version(self) -> int:
        return int(self.state.placement_version)

    @property
    def num_slots(self) -> int:
        return int(self.slot_to_logical.shape[0])

    def mapping_for_device(self, device: torch.device) -> torch.Tensor:
        """``[S, E]`` int64 ``M`` on ``device`` for the routing kernels: the
        state's device row of this source rank as a one-row table, or the
        whole table when per-token sources are set."""
        M = self.state.source_logical_to_physical
        if self.token_sources is not None:
            if M is None:
                raise RuntimeError(f"HierMoE layer {self.key} has no source-rank route LUT.")
            key = ("M", device, id(M), self.placement_version)
            if key not in self._cache:
                self._cache = {k: v for k, v in self._cache.items() if k[0] != "M"}
                self._cache[key] = torch.as_tensor(M, dtype=torch.int64).to(device)
            return self._cache[key]
        if M is None:
            row = self.state.mapping_for_device(device)
        else:
            row = self.state.source_mapping_for_device(device, self.source_rank)
        return row.reshape(1, -1)

    def copy_tables_for_device(self, device: torch.device) -> tuple[torch.Tensor, torch.Tensor]:
        L = self.slot_to_logical
        key = ("copies", device, L.tobytes())
        if key not in self._cache:
            self._cache = {k: v for k, v in self._cache.items() if k[0] != "copies"}
            off, slots = copy_table(L, self.num_experts)
            self._cache[key] = (torch.as_tensor(off).to(device), torch.as_tensor(slots).to(device))
        return self._cache[key]

    def install_mapping(self, source_logical_to_physical) -> int:
        """Mapping-only hot update written into the state the way the
        reference's ``_install_hot_update_mapping`` writes it
        (expert_swap.py:10963-10972); returns 1 if ``M`` changed."""
        lut = torch.as_tensor(np.asarray(source_logical_to_physical, dtype=np.int64))
        M = self.state.source_logical_to_physical
        if M is not None and tuple(lut.shape) != tuple(M.shape):
            raise RuntimeError(f"PlaceMoE mapping for {self.key} has shape {tuple(lut.shape)}, "
                               f"expected {tuple(M.shape)}.")
        L = self.slot_to_logical
        if bool(((lut < 0) | (lut >= L.shape[0])).any()):
            raise RuntimeError(f"PlaceMoE mapping for {self.key} references an invalid slot.")
        if not np.array_equal(L[lut.numpy()], np.broadcast_to(np.arange(self.num_experts), tuple(lut.shape))):
            raise RuntimeError(f"PlaceMoE mapping for {self.key} references the wrong expert.")
        changed = M is None or not torch.equal(torch.as_tensor(M).cpu(), lut)
        self.state.source_logical_to_physical = lut.clone()
        self.state._device_source_mapping_cache.clear()
        self.state.placement_version += int(changed)
        return int(changed)

    def record_slot_tokens(self, counts: torch.Tensor) -> None:
        LayerPlacement.record_slot_tokens(self, counts)

    def clear_slot_tokens(self) -> None:
        self.accumulated_slot_tokens = None


class PlacementRegistry:
    """layer_key -> LayerPlacement, plus parameter -> layer_key lookup (the
    role of ``get_hiermoe_expert_layer_key_from_params``)."""

    def __init__(self) -> None:
        self.layers: dict[str, LayerPlacement] = {}
        self._param_keys: dict[int, str] = {}

    def register(self, placement: "LayerPlacement | LayerStatePlacement", *params: torch.Tensor) -> None:
        self.layers[placement.key] = placement
        for p in params:
            if p is not None:
                self._param_keys[id(p)] = placement.key

    def get(self, key: str | None) -> "LayerPlacement | LayerStatePlacement | None":
        return None if key is None else self.layers.get(key)

    def key_from_params(self, *params: torch.Tensor | None) -> str | None:
        for p in params:
            if p is not None and id(p) in self._param_keys:
                return self._param_keys[id(p)]
        return None

    def clear(self) -> None:
        self.layers.clear()
        self._param_keys.clear()


PLACEMENTS = PlacementRegistry()
