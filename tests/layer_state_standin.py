"""A stand-in for the reference's per-layer placement state
(``ExpertLayerState``, veomni/distributed/moe/hiermoe/expert_swap.py:433-586):
the fields and the two device-mapping caches that the HIP op's
``LayerStatePlacement`` reads, and a mapping-only hot update that writes them
the way ``_install_hot_update_mapping`` does (expert_swap.py:10963-10972)."""

from __future__ import annotations

from dataclasses import dataclass, field

import torch


@dataclass
class StandInLayerState:
    key: str
    num_experts: int
    logical_to_physical: torch.Tensor  # [E] owner slot of each expert
    slot_to_logical: torch.Tensor | None = None  # [C] (L)
    source_logical_to_physical: torch.Tensor | None = None  # [S, E] (M)
    placement_version: int = 0
    _device_mapping_cache: dict = field(default_factory=dict)
    _device_source_mapping_cache: dict = field(default_factory=dict)

    def mapping_for_device(self, device: torch.device) -> torch.Tensor:
        cached = self._device_mapping_cache.get(device)
        if cached is None:
            cached = self.logical_to_physical.to(device=device, non_blocking=True)
            self._device_mapping_cache[device] = cached
        return cached

    def source_mapping_for_device(self, device: torch.device, source_rank: int) -> torch.Tensor:
        if self.source_logical_to_physical is None:
            raise RuntimeError(f"HierMoE layer {self.key} has no source-rank route LUT.")
        key = (device, int(source_rank))
        cached = self._device_source_mapping_cache.get(key)
        if cached is None:
            cached = self.source_logical_to_physical[int(source_rank)].to(device=device, non_blocking=True)
            self._device_source_mapping_cache[key] = cached
        return cached

    def hot_update(self, lut) -> int:
        """What the reference's controller does on a mapping-only update."""
        lut = torch.as_tensor(lut, dtype=torch.long).cpu()
        changed = self.source_logical_to_physical is None or not torch.equal(self.source_logical_to_physical, lut)
        self.source_logical_to_physical = lut.clone()
        self._device_source_mapping_cache.clear()
        self.placement_version += int(changed)
        return int(changed)
