"""Per-layer replica-gradient fold overlapped with the backward (side stream,
post-accumulate-grad hooks) against the synchronous fold after the backward:
identical fp32 logical gradients and identical written-back copy gradients
over a stack of layers."""

import numpy as np
import pytest
import torch

import placemoe_amd
from placemoe_amd.dispatch import OpSlot
from placemoe_amd.placement import PLACEMENTS, LayerPlacement, LayerPlan
from placemoe_amd.workloads import make_workload
from tests.helpers import assert_exact

pytestmark = pytest.mark.gpu


class _Experts(torch.nn.Module):
    def __init__(self, num_experts, fc1, fc2):
        super().__init__()
        self.num_experts = num_experts
        self.gate_up_proj = torch.nn.Parameter(fc1)
        self.down_proj = torch.nn.Parameter(fc2)


def _stack(cuda, layers):
    """`layers` expert modules, each with its own weights, routing and placement."""
    mods, wl0 = {}, None
    for i in range(layers):
        wl = make_workload("fold", tokens=160, seed=2000 + i)
        wl0 = wl0 or wl
        m = _Experts(wl.num_experts, wl.fc1.to(cuda), wl.fc2.to(cuda))
        plan = LayerPlan(slot_to_logical=wl.slot_to_logical, source_logical_to_physical=wl.mapping.numpy(),
                         owner_slots=wl.owner_slots())
        key = f"layers.{i}.mlp.experts"
        p = LayerPlacement.from_plan(key, plan, wl.num_experts)
        p.token_sources = wl.sources.to(cuda)
        PLACEMENTS.register(p, m.gate_up_proj, m.down_proj)
        mods[key] = (m, wl)
    return mods, wl0


def _forward_backward(cuda, mods, wl0):
    slot = OpSlot("moe_experts", "standard")
    slot.bind("hip")
    h = wl0.hidden.to(cuda)
    for m, wl in mods.values():
        h = slot(m, h, wl.selected.to(cuda), wl.routing_weights.float().to(cuda))
    h.float().square().sum().backward()


def _run(cuda, mods, wl0, overlapped):
    for m, _ in mods.values():
        m.zero_grad(set_to_none=True)
    modules = {k: m for k, (m, _) in mods.items()}
    sync = placemoe_amd.OverlappedReplicaSync(modules) if overlapped else None
    try:
        _forward_backward(cuda, mods, wl0)
        folded = sync.finish() if overlapped else placemoe_amd.sync_redundant_gradients(modules)
        torch.cuda.synchronize()
        grads = {k: (m.gate_up_proj.grad.clone(), m.down_proj.grad.clone()) for k, (m, _) in mods.items()}
        return {k: (a.clone(), b.clone()) for k, (a, b) in folded.items()}, grads
    finally:
        if sync is not None:
            sync.remove()


def test_overlapped_fold_equals_synchronous_fold(cuda):
    PLACEMENTS.clear()
    try:
        mods, wl0 = _stack(cuda, 3)
        print("replica overlap: 3 layers of the fold shape, 160 tokens", flush=True)
        ref_fold, ref_grads = _run(cuda, mods, wl0, overlapped=False)
        ov_fold, ov_grads = _run(cuda, mods, wl0, overlapped=True)
        assert set(ov_fold) == set(ref_fold) == set(mods)
        for k in mods:
            for a, b, name in zip(ov_fold[k], ref_fold[k], ("gate_up", "down")):
                assert_exact(a, b, f"{k} fp32 {name}")
            for a, b, name in zip(ov_grads[k], ref_grads[k], ("gate_up", "down")):
                assert_exact(a, b, f"{k} written-back {name}")
        # every copy of an expert holds bf16 of the expert's fp32 total
        for k, (m, wl) in mods.items():
            L = np.asarray(wl.slot_to_logical)
            for c in range(L.size):
                assert_exact(ov_grads[k][1][c], ov_fold[k][1][L[c]].to(torch.bfloat16), f"{k} copy {c}")
    finally:
        PLACEMENTS.clear()


def test_overlapped_fold_disabled_for_accumulation(cuda):
    PLACEMENTS.clear()
    try:
        mods, wl0 = _stack(cuda, 2)
        sync = placemoe_amd.OverlappedReplicaSync({k: m for k, (m, _) in mods.items()})
        sync.enabled = False
        _forward_backward(cuda, mods, wl0)
        assert sync.finish() == {}
        # no fold happened: two copies of one expert that both saw tokens keep
        # their own (different) gradients
        key = list(mods)[-1]
        m, wl = mods[key]
        L = np.asarray(wl.slot_to_logical)
        tokens = PLACEMENTS.get(key).accumulated_slot_tokens.cpu().numpy()
        pair = next(np.nonzero((L == e) & (tokens > 0))[0][:2] for e in range(wl.num_experts)
                    if np.count_nonzero((L == e) & (tokens > 0)) >= 2)
        g = m.down_proj.grad
        assert not torch.equal(g[pair[0]], g[pair[1]])
        sync.remove()
    finally:
        PLACEMENTS.clear()
