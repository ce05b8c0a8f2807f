"""The committed fixtures: the reference's known answers (as data) hold for
the oracle and the host-side placement code, and the oracle still reproduces
its own recorded small vectors."""

import json
import os

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from placemoe_amd.placement import LayerPlan, PlaceMoETopology, mirrored_r2_plan

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def kats():
    with open(os.path.join(GOLDEN, "reference_kats.json")) as f:
        return json.load(f)


def small(name="oracle_small.npz"):
    return dict(np.load(os.path.join(GOLDEN, name)))


def test_source_lut_kat():
    k = kats()["source_lut"]
    M = np.array(k["source_logical_to_physical"])
    phys = O.map_logical_to_physical(M, [k["source"]], k["selected"])
    assert phys.tolist() == k["expected_physical"]
    L = np.array(k["slot_to_logical"])
    assert np.array_equal(L[M], np.tile(np.arange(M.shape[1]), (M.shape[0], 1)))


def test_layer_plan_kats():
    k = kats()
    v = k["layer_plan_valid"]
    topo = PlaceMoETopology(v["ep_size"], v["ranks_per_node"], v["num_experts"], v["slots_per_rank"])
    plan = LayerPlan(v["slot_to_logical"], v["source_logical_to_physical"], v["owner_slots"])
    plan.validate(topo, additional_copies=v["additional_copies"])
    bad = k["layer_plan_wrong_expert"]
    topo = PlaceMoETopology(bad["ep_size"], bad["ranks_per_node"], bad["num_experts"], bad["slots_per_rank"])
    with pytest.raises(ValueError, match=bad["error"]):
        LayerPlan(bad["slot_to_logical"], bad["source_logical_to_physical"], bad["owner_slots"]).validate(
            topo, additional_copies=0)
    m = k["mirrored_r2"]
    plan = mirrored_r2_plan(PlaceMoETopology(m["ep_size"], m["ranks_per_node"], m["num_experts"], m["slots_per_rank"]))
    assert plan.slot_to_logical.tolist() == m["expected_slot_to_logical"]
    assert plan.source_logical_to_physical.tolist() == m["expected_source_rows"]


def test_replica_sum_kat():
    k = kats()["replica_sum"]
    L = np.array(k["slot_to_logical"])
    gate = torch.zeros((L.size, 4, 3))
    down = torch.zeros((L.size, 3, 3))
    for slot, v in k["gate_up_copy_values"].items():
        gate[int(slot)] = v
    for slot, v in k["down_copy_values"].items():
        down[int(slot)] = v
    e = k["logical_expert"]
    assert torch.all(O.replica_fold(gate.to(torch.bfloat16), L, 4)[e] == k["expected_gate_up"])
    assert torch.all(O.replica_fold(down.to(torch.bfloat16), L, 4)[e] == k["expected_down"])


@pytest.mark.parametrize("name,dtype", [("oracle_small.npz", torch.bfloat16),
                                        ("oracle_small_f16.npz", torch.float16)])
def test_oracle_reproduces_recorded_vectors(name, dtype):
    v = small(name)
    bf = lambda a: torch.as_tensor(a).to(dtype)  # noqa: E731
    phys, counts, offsets, pos = O.route(v["mapping"], v["sources"], v["selected"], v["slot_to_logical"].size)
    for name, got in (("phys", phys), ("counts", counts), ("offsets", offsets), ("pos", pos)):
        assert np.array_equal(got, v[name]), name
    fwd = O.moe_layer_forward(bf(v["hidden"]), bf(v["routing_weights"]), phys, bf(v["fc1"]), bf(v["fc2"]))
    bwd = O.moe_layer_backward(bf(v["grad_out"]), fwd, bf(v["routing_weights"]), bf(v["fc1"]), bf(v["fc2"]))
    for name, got in (("out", fwd["out"]), ("gu", fwd["gu"]), ("act", fwd["act"]), ("y", fwd["y"]),
                      ("dx", bwd["dx"]), ("dw", bwd["dw"]), ("dw1", bwd["dw1"]), ("dw2", bwd["dw2"])):
        assert np.array_equal(got.float().numpy(), v[name]), name
