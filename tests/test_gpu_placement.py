"""GPU checks of the placement plumbing around the layer: a mapping-only hot
update reaching the device routing, copy-weight materialisation, invalid
ids at the op boundary, and the fold's copy-table guard."""

import numpy as np
import pytest
import torch

import placemoe_amd
from oracle import moe_oracle as O
from placemoe_amd import experts, kernels
from placemoe_amd.placement import PLACEMENTS, LayerPlacement, LayerPlan, materialize_copy_weights
from placemoe_amd.workloads import make_workload
from tests.helpers import assert_bf16_close, assert_exact

pytestmark = pytest.mark.gpu


def _rotated_mapping(L, M):
    """Every (source, expert) moved to the next copy of its expert (slot order)."""
    out = M.copy()
    for e in range(M.shape[1]):
        copies = np.nonzero(L == e)[0]
        for s in range(M.shape[0]):
            i = int(np.nonzero(copies == M[s, e])[0][0])
            out[s, e] = copies[(i + 1) % len(copies)]
    return out


def test_mapping_hot_update_reaches_device_routing(cuda):
    # expert_swap.py:10920-10972 installs a new LUT for the same layout L and
    # drops the per-device cache (:502-510); the next call must route with it.
    placemoe_amd.apply_veomni_fused_moe_patch("hip")
    wl = make_workload("fold", tokens=192)
    L = wl.slot_to_logical
    M0 = wl.mapping.numpy()
    M1 = _rotated_mapping(L, M0)
    assert not np.array_equal(M0, M1)
    plan = LayerPlan(slot_to_logical=L, source_logical_to_physical=M0, owner_slots=wl.owner_slots())
    placement = LayerPlacement.from_plan("layers.3.mlp.experts", plan, wl.num_experts)
    placement.token_sources = wl.sources.to(cuda)
    fc1, fc2 = wl.fc1.to(cuda), wl.fc2.to(cuda)
    PLACEMENTS.register(placement, fc1, fc2)
    try:
        for step, M in enumerate((M0, M1)):
            if step == 1:
                assert placement.install_mapping(M1) == 1
                assert placement.placement_version == 1
            placement.clear_slot_tokens()
            dev_M = placement.mapping_for_device(cuda)
            assert_exact(dev_M, M, f"device M after step {step}")
            r = kernels.route(wl.selected.to(cuda), wl.C, mapping=dev_M, sources=placement.token_sources)
            phys = O.map_logical_to_physical(M, wl.sources.numpy(), wl.selected.numpy())
            assert_exact(r.phys, phys, f"phys step {step}")
            assert_exact(r.pos, O.scatter_index(phys), f"pos step {step}")
            out = placemoe_amd.fused_moe_forward(
                num_experts=wl.num_experts, routing_weights=wl.routing_weights.to(cuda),
                selected_experts=wl.selected.to(cuda), hidden_states=wl.hidden.to(cuda), fc1_1_weight=None,
                fc1_2_weight=None, fc2_weight=fc2, fc1_1_2_weight=fc1)
            fwd = O.moe_layer_forward(wl.hidden, wl.routing_weights, phys, wl.fc1, wl.fc2)
            assert_exact(placement.accumulated_slot_tokens, fwd["counts"], f"slot tokens step {step}")
            assert_bf16_close(out, fwd["out"], name=f"output step {step}")
        # An identical mapping is not a change.
        assert placement.install_mapping(M1) == 0 and placement.placement_version == 1
    finally:
        PLACEMENTS.clear()


@pytest.mark.parametrize("per_token", [False, True], ids=["source_rank_row", "per_token_sources"])
def test_layer_state_hot_update_reaches_device_routing(cuda, per_token):
    """The op reads M from the reference's layer state (a stand-in with its
    fields) on every call: a hot update written by the reference's controller
    (expert_swap.py:10963-10972), with no call into this package, changes the
    next forward's routing, bit-exact against the oracle."""
    from tests.layer_state_standin import StandInLayerState

    placemoe_amd.apply_veomni_fused_moe_patch("hip")
    wl = make_workload("fold", tokens=192)
    L = wl.slot_to_logical
    M0 = wl.mapping.numpy()
    M1 = _rotated_mapping(L, M0)
    rank = 3
    state = StandInLayerState(key="layers.5.mlp.experts", num_experts=wl.num_experts,
                              logical_to_physical=torch.as_tensor(wl.owner_slots()),
                              slot_to_logical=torch.as_tensor(L), source_logical_to_physical=torch.as_tensor(M0))
    placement = LayerPlacement.from_layer_state(state, source_rank=rank)
    if per_token:
        placement.token_sources = wl.sources.to(cuda)
    src = wl.sources.numpy() if per_token else np.full(wl.T, rank)
    fc1, fc2 = wl.fc1.to(cuda), wl.fc2.to(cuda)
    PLACEMENTS.register(placement, fc1, fc2)
    try:
        for step, M in enumerate((M0, M1)):
            if step == 1:
                assert state.hot_update(M1) == 1
                assert placement.placement_version == 1
            placement.clear_slot_tokens()
            phys = O.map_logical_to_physical(M, src, wl.selected.numpy())
            dev_M = placement.mapping_for_device(cuda)
            r = kernels.route(wl.selected.to(cuda), wl.C, mapping=dev_M, sources=placement.token_sources,
                              source=placement.source)
            assert_exact(r.phys, phys, f"phys step {step}")
            assert_exact(r.pos, O.scatter_index(phys), f"pos step {step}")
            out = placemoe_amd.fused_moe_forward(
                num_experts=wl.num_experts, routing_weights=wl.routing_weights.to(cuda),
                selected_experts=wl.selected.to(cuda), hidden_states=wl.hidden.to(cuda), fc1_1_weight=None,
                fc1_2_weight=None, fc2_weight=fc2, fc1_1_2_weight=fc1)
            fwd = O.moe_layer_forward(wl.hidden, wl.routing_weights, phys, wl.fc1, wl.fc2)
            assert_exact(placement.accumulated_slot_tokens, fwd["counts"], f"slot tokens step {step}")
            assert_bf16_close(out, fwd["out"], name=f"output step {step}")
    finally:
        PLACEMENTS.clear()


def test_materialize_copy_weights_on_device(cuda):
    # parallel_plan.py:114-123: W_copy[c] = W_logical[L[c]], zeros where L[c] == -1.
    g = torch.Generator(device=cuda).manual_seed(3)
    logical = torch.randn((6, 64, 40), generator=g, device=cuda).to(torch.bfloat16)
    L = np.array([3, -1, 0, 5, 3, -1, 1, 2, 4], dtype=np.int64)
    copies = materialize_copy_weights(logical, L)
    assert copies.device == logical.device and copies.dtype == logical.dtype
    ref = torch.zeros((L.size, 64, 40), dtype=torch.bfloat16)
    host = logical.cpu()
    for c, e in enumerate(L):
        if e >= 0:
            ref[c] = host[e]
    assert_exact(copies, ref, "materialised copies")
    assert torch.count_nonzero(copies[1]).item() == 0 and torch.count_nonzero(copies[5]).item() == 0
    with pytest.raises(ValueError):
        materialize_copy_weights(logical, np.array([0, 6]))


def _bad_call(cuda, wl, sel):
    return placemoe_amd.fused_moe_forward(
        num_experts=wl.C, routing_weights=wl.routing_weights.to(cuda).requires_grad_(True),
        selected_experts=sel, hidden_states=wl.hidden.to(cuda).requires_grad_(True), fc1_1_weight=None,
        fc1_2_weight=None, fc2_weight=wl.fc2.to(cuda), fc1_1_2_weight=wl.fc1.to(cuda))


def test_out_of_range_expert_id_raises(cuda, monkeypatch):
    # The reference's index_select on the LUT refuses an id outside the table
    # (expert_swap.py:5919-5920); here the device clamps it, flags the routing
    # status word, and the op raises ValueError: at the backward by default,
    # or in the forward itself with PLACEMOE_AMD_CHECK_ROUTES=1.
    placemoe_amd.apply_veomni_fused_moe_patch("hip")
    monkeypatch.delenv("PLACEMOE_AMD_CHECK_ROUTES", raising=False)
    wl = make_workload("toy", tokens=64)
    sel = wl.selected.clone()
    sel[5, 1] = wl.C  # one past the last expert
    sel = sel.to(cuda)
    out = _bad_call(cuda, wl, sel)
    # The backward looks at the status copy without waiting for it; once it
    # has landed (here: after a synchronisation) the backward raises.
    torch.cuda.synchronize()
    with pytest.raises(ValueError, match="outside"):
        out.sum().backward()
    # a valid call afterwards is unaffected
    good = _bad_call(cuda, wl, wl.selected.to(cuda))
    good.sum().backward()
    monkeypatch.setenv("PLACEMOE_AMD_CHECK_ROUTES", "1")
    sel[7, 0] = -3
    with pytest.raises(ValueError, match="outside"):
        _bad_call(cuda, wl, sel)


def test_forward_only_bad_id_is_reported_by_a_later_call(cuda, monkeypatch):
    placemoe_amd.apply_veomni_fused_moe_patch("hip")
    monkeypatch.delenv("PLACEMOE_AMD_CHECK_ROUTES", raising=False)
    wl = make_workload("toy", tokens=64)
    sel = wl.selected.clone()
    sel[0, 0] = 10_000
    with torch.no_grad():
        _bad_call(cuda, wl, sel.to(cuda))
        torch.cuda.synchronize()
        with pytest.raises(ValueError, match="outside"):
            _bad_call(cuda, wl, wl.selected.to(cuda))
        _bad_call(cuda, wl, wl.selected.to(cuda))  # reported once
    experts._PENDING_CHECKS.clear()


def test_pending_bad_id_is_reported_by_check_pending_routes(cuda, monkeypatch):
    """check_pending_routes(block=True) waits for the status copies and raises;
    without block it raises only for copies that have landed."""
    placemoe_amd.apply_veomni_fused_moe_patch("hip")
    monkeypatch.delenv("PLACEMOE_AMD_CHECK_ROUTES", raising=False)
    wl = make_workload("toy", tokens=64)
    sel = wl.selected.clone()
    sel[3, 0] = -1
    with torch.no_grad():
        _bad_call(cuda, wl, sel.to(cuda))
        with pytest.raises(ValueError, match="outside"):
            experts.check_pending_routes(block=True)
        experts.check_pending_routes(block=True)  # reported once
        _bad_call(cuda, wl, wl.selected.to(cuda))
        experts.check_pending_routes(block=True)
    assert not experts._PENDING_CHECKS


def test_fold_skips_and_flags_out_of_range_copy_slots(cuda):
    g = torch.Generator(device=cuda).manual_seed(9)
    C, P = 5, 1024
    grads = torch.randn((C, P), generator=g, device=cuda).to(torch.bfloat16)
    before = grads.clone()
    off = torch.tensor([0, 2, 4], dtype=torch.int32, device=cuda)
    slots = torch.tensor([0, 3, 1, 7], dtype=torch.int32, device=cuda)  # slot 7 does not exist
    status = torch.zeros(1, dtype=torch.int32, device=cuda)
    out = kernels.replica_fold(grads, off, slots, 2, writeback=True, status=status)
    assert int(status.item()) == 1
    ref0 = before[0].float() + before[3].float()
    assert torch.equal(out[0].cpu(), ref0.cpu())
    assert torch.equal(out[1].cpu(), before[1].float().cpu())  # slot 7 skipped
    assert_exact(grads[0], ref0.to(torch.bfloat16), "write-back copy 0")
    assert_exact(grads[1], before[1], "write-back copy 1")
    assert_exact(grads[2], before[2], "untouched copy 2")
    assert_exact(grads[4], before[4], "untouched copy 4")
    status.zero_()
    kernels.replica_fold(grads, off, torch.tensor([0, 3, 1, 2], dtype=torch.int32, device=cuda), 2,
                         status=status)
    assert int(status.item()) == 0


def test_fused_moe_rejects_mismatched_fc1(cuda):
    wl = make_workload("toy", tokens=32)
    x, w, sel = wl.hidden.to(cuda), wl.routing_weights.to(cuda), wl.selected.to(cuda)
    fc2 = wl.fc2.to(cuda)
    with pytest.raises(AssertionError, match="bfloat16"):
        experts.expert_layer(x, w, sel, fc2, fc1_1_2_weight=wl.fc1.float().to(cuda))
    with pytest.raises(AssertionError, match="shape"):
        experts.expert_layer(x, w, sel, fc2, fc1_1_2_weight=wl.fc1[:-1].contiguous().to(cuda))
