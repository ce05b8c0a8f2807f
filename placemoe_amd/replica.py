"""Replica-gradient fold for the copies held by one GPU.

``fold_replica_gradients`` is the single-GPU share of
``ExpertSwapManager.sync_redundant_gradients``
(veomni/distributed/moe/hiermoe/expert_swap.py:7220-7252): slots that saw no
tokens are treated as zero (``_zero_inactive_slot_grads_for_layer``,
:6250-6262), copies of each logical expert are summed (here in fp32;
``_replica_grad_contributions``, :6839-6876), and, with ``writeback``, every
copy receives the total (``_unpack_replica_grad``, :6886-6889).  The
cross-GPU exchange of partial sums is outside this build.
"""

from __future__ import annotations

import torch

from . import kernels
from .placement import PLACEMENTS, LayerPlacement


def fold_replica_gradients(placement: LayerPlacement, grads: torch.Tensor, *, writeback: bool = True,
                           use_slot_tokens: bool = True) -> torch.Tensor:
    """fp32 [E, ...] logical gradients from copy gradients ``grads`` [C, ...] (bf16)."""
    if int(grads.shape[0]) != placement.num_slots:
        raise ValueError(f"expected {placement.num_slots} copy gradients, got {int(grads.shape[0])}")
    off, slots = placement.copy_tables_for_device(grads.device)
    tokens = placement.accumulated_slot_tokens if use_slot_tokens else None
    return kernels.replica_fold(grads.contiguous(), off, slots, placement.num_experts, slot_tokens=tokens,
                                writeback=writeback)


@torch.no_grad()
def sync_redundant_gradients(modules: dict[str, torch.nn.Module]) -> dict[str, tuple[torch.Tensor, torch.Tensor]]:
    """Fold ``gate_up_proj.grad`` and ``down_proj.grad`` of every registered
    layer in place; returns the fp32 logical gradients per layer and clears
    the accumulated token counts."""
    out = {}
    for key, module in modules.items():
        placement = PLACEMENTS.get(key)
        if placement is None:
            continue
        results = []
        for param in (module.gate_up_proj, module.down_proj):
            if param.grad is None:
                param.grad = torch.zeros_like(param)
            results.append(fold_replica_gradients(placement, param.grad))
        placement.clear_slot_tokens()
        out[key] = (results[0], results[1])
    return out
