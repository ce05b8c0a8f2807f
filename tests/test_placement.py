"""Host-side placement tables: LayerPlan contract, artifacts, copy tables,
copy-weight materialisation and mapping-only hot updates."""

import numpy as np
import pytest
import torch

from placemoe_amd.placement import (
    LayerPlacement,
    LayerPlan,
    PlaceMoETopology,
    build_placemoe_artifact,
    copy_table,
    materialize_copy_weights,
    mirrored_r2_plan,
    validate_placemoe_artifact,
)

TOPO = PlaceMoETopology(ep_size=2, ranks_per_node=1, num_experts=4, slots_per_rank=3)
PLAN = LayerPlan(slot_to_logical=[0, 1, 0, 2, 3, 3], owner_slots=[0, 1, 3, 4],
                 source_logical_to_physical=[[0, 1, 3, 4], [2, 1, 3, 5]])


def test_topology_checks():
    with pytest.raises(ValueError, match="positive"):
        PlaceMoETopology(0, 1, 4, 2)
    with pytest.raises(ValueError, match="divisible"):
        PlaceMoETopology(3, 2, 4, 2)
    with pytest.raises(ValueError, match="cannot hold"):
        PlaceMoETopology(1, 1, 4, 2)
    assert TOPO.rank_of_slot(4) == 1
    with pytest.raises(ValueError):
        TOPO.rank_of_slot(6)


@pytest.mark.parametrize("mutate,match", [
    (lambda L, M, O: (L[:-1], M, O), "Layout length"),
    (lambda L, M, O: (L, M[:1], O), "Mapping shape"),
    (lambda L, M, O: (L, M, O[:-1]), "owner_slots"),
    (lambda L, M, O: ([0, 1, 0, 2, 3, 7], M, O), "invalid logical expert"),
    (lambda L, M, O: ([0, 1, 0, 2, 2, 2], M, O), "at least one physical copy"),
    (lambda L, M, O: (L, [[0, 1, 3, 4], [2, 1, 3, 9]], O), "outside the topology"),
    (lambda L, M, O: (L, [[0, 1, 3, 4], [2, 1, 4, 5]], O), "wrong logical expert"),
    (lambda L, M, O: (L, M, [0, 1, 3, 3]), "do not match"),
])
def test_layer_plan_rejections(mutate, match):
    L, M, O = mutate(list(PLAN.slot_to_logical), PLAN.source_logical_to_physical.tolist(), list(PLAN.owner_slots))
    with pytest.raises(ValueError, match=match):
        LayerPlan(slot_to_logical=L, source_logical_to_physical=M, owner_slots=O).validate(TOPO)


def test_budget_and_round_trip():
    PLAN.validate(TOPO, additional_copies=2)
    with pytest.raises(ValueError, match="budget"):
        PLAN.validate(TOPO, additional_copies=3)
    restored = LayerPlan.from_runtime_payload(PLAN.to_runtime_payload())
    assert np.array_equal(restored.slot_to_logical, PLAN.slot_to_logical)
    assert not PLAN.slot_to_logical.flags.writeable


def test_artifact_round_trip_and_rejection():
    payload = build_placemoe_artifact({"layers.0.experts": PLAN}, TOPO, source={"route_root": "/tmp/r"})
    plans = validate_placemoe_artifact(payload)
    assert np.array_equal(plans["layers.0.experts"].owner_slots, PLAN.owner_slots)
    payload["layers"]["layers.0.experts"]["source_logical_to_physical"][0][0] = 1
    with pytest.raises(ValueError, match="wrong logical expert"):
        validate_placemoe_artifact(payload)
    with pytest.raises(ValueError, match="schema"):
        validate_placemoe_artifact({"schema_version": 1})


def test_mirrored_r2_requires_even_two_copies():
    with pytest.raises(ValueError, match="Mirrored R2"):
        mirrored_r2_plan(PlaceMoETopology(3, 1, 6, 4))
    plan = mirrored_r2_plan(PlaceMoETopology(ep_size=4, ranks_per_node=2, num_experts=8, slots_per_rank=4))
    plan.validate(PlaceMoETopology(4, 2, 8, 4), additional_copies=8)


def test_copy_table_slot_order():
    off, slots = copy_table([0, 1, 3, 2, 3, -1, 0], 4)
    assert off.tolist() == [0, 2, 3, 4, 6]
    assert slots.tolist() == [0, 6, 1, 3, 2, 4]


def test_materialize_copy_weights_zero_empty_slots():
    logical = torch.arange(4 * 2 * 3, dtype=torch.float32).reshape(4, 2, 3)
    copies = materialize_copy_weights(logical, [2, -1, 0, 2])
    assert torch.equal(copies[0], logical[2]) and torch.equal(copies[3], logical[2])
    assert torch.equal(copies[2], logical[0]) and torch.count_nonzero(copies[1]) == 0
    with pytest.raises(ValueError):
        materialize_copy_weights(logical, [4])


def test_mapping_hot_update_checks():
    lp = LayerPlacement.from_plan("l0", PLAN, num_experts=4, source=1)
    assert lp.install_mapping([[2, 1, 3, 4], [0, 1, 3, 5]]) == 1
    assert lp.install_mapping([[2, 1, 3, 4], [0, 1, 3, 5]]) == 0
    with pytest.raises(RuntimeError, match="shape"):
        lp.install_mapping([[0, 1, 3, 4]])
    with pytest.raises(RuntimeError, match="invalid slot"):
        lp.install_mapping([[0, 1, 3, 4], [0, 1, 3, 6]])
    with pytest.raises(RuntimeError, match="wrong expert"):
        lp.install_mapping([[1, 1, 3, 4], [0, 1, 3, 5]])
    assert lp.placement_version == 1
    with pytest.raises(ValueError, match="source"):
        LayerPlacement.from_plan("l1", PLAN, num_experts=4, source=2)


def test_slot_token_accumulation():
    lp = LayerPlacement.from_plan("l0", PLAN, num_experts=4)
    lp.record_slot_tokens(torch.tensor([1, 0, 2, 0, 0, 3], dtype=torch.int32))
    lp.record_slot_tokens(torch.tensor([1, 1, 0, 0, 0, 0], dtype=torch.int32))
    assert lp.accumulated_slot_tokens.tolist() == [2, 1, 2, 0, 0, 3]
    lp.clear_slot_tokens()
    assert lp.accumulated_slot_tokens is None
