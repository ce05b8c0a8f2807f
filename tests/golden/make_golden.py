"""Write the committed fixtures under tests/golden/.

* reference_kats.json - the reference's own known answers for this path, as
  data (inputs and expected outputs), transcribed from the reference's tests:
  source-LUT mapping (tests/distributed/test_hiermoe_forward_cover_planner.py:1010-1038),
  LayerPlan validation (tests/distributed/test_placemoe_optimizer.py:108-129,762-771),
  replica-gradient sums (tests/distributed/test_hiermoe.py:3286-3338).
* oracle_small.npz - small vectors produced by oracle/moe_oracle.py for a fixed
  seed (routing, layer forward and backward), re-checked by the CPU suite so a
  change in the oracle cannot pass silently, and used by the GPU suite.
* oracle_small_f16.npz - the same draws cast to fp16 instead of bf16, with the
  oracle's fp16 outputs.

Usage: python tests/golden/make_golden.py
"""

import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import moe_oracle as O  # noqa: E402

KATS = {
    "source_lut": {
        "slot_to_logical": [0, 1, 3, 2, 3, 0],
        "source_logical_to_physical": [[0, 1, 3, 2], [5, 1, 3, 4]],
        "selected": [[3, 2, 0]],
        "source": 0,
        "expected_physical": [[2, 3, 0]],
    },
    "layer_plan_valid": {
        "ep_size": 2, "ranks_per_node": 1, "num_experts": 4, "slots_per_rank": 3,
        "slot_to_logical": [0, 1, 0, 2, 3, 3], "owner_slots": [0, 1, 3, 4],
        "source_logical_to_physical": [[0, 1, 3, 4], [2, 1, 3, 5]], "additional_copies": 2,
    },
    "layer_plan_wrong_expert": {
        "ep_size": 2, "ranks_per_node": 1, "num_experts": 4, "slots_per_rank": 2,
        "slot_to_logical": [0, 1, 2, 3], "owner_slots": [0, 1, 2, 3],
        "source_logical_to_physical": [[1, 1, 2, 3], [0, 1, 2, 3]], "error": "wrong logical expert",
    },
    "mirrored_r2": {
        "ep_size": 4, "ranks_per_node": 2, "num_experts": 8, "slots_per_rank": 4,
        "expected_slot_to_logical": list(range(8)) + list(range(8)),
        "expected_source_rows": [list(range(8))] * 2 + [list(range(8, 16))] * 2,
    },
    "replica_sum": {
        "slot_to_logical": [0, 1, 3, 2, 3, -1],
        "gate_up_copy_values": {"2": 10.0, "4": 2.0}, "down_copy_values": {"2": 20.0, "4": 3.0},
        "logical_expert": 3, "expected_gate_up": 12.0, "expected_down": 23.0,
    },
}


def small_vectors(dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(424242)
    T, K, H, I, E, S = 48, 3, 64, 32, 5, 3
    L = np.array([0, 1, 2, 3, 4, 0, 2, 2], dtype=np.int64)
    C = L.size
    M = np.array([[0, 1, 2, 3, 4], [5, 1, 6, 3, 4], [0, 1, 7, 3, 4]], dtype=np.int64)
    src = torch.randint(0, S, (T,), generator=g).numpy()
    sel = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)]).numpy()
    x = torch.randn((T, H), generator=g).to(dtype)
    w = torch.rand((T, K), generator=g).to(dtype)
    w1 = (torch.randn((C, 2 * I, H), generator=g) * 0.1).to(dtype)
    w2 = (torch.randn((C, H, I), generator=g) * 0.1).to(dtype)
    dout = torch.randn((T, H), generator=g).to(dtype)
    phys, counts, offsets, pos = O.route(M, src, sel, C)
    fwd = O.moe_layer_forward(x, w, phys, w1, w2)
    bwd = O.moe_layer_backward(dout, fwd, w, w1, w2)
    f32 = lambda t: t.float().numpy()  # noqa: E731  bf16 and fp16 values are exact in fp32
    return dict(
        slot_to_logical=L, mapping=M, sources=src, selected=sel, hidden=f32(x), routing_weights=f32(w),
        fc1=f32(w1), fc2=f32(w2), grad_out=f32(dout), phys=phys, counts=counts, offsets=offsets, pos=pos,
        out=f32(fwd["out"]), gu=f32(fwd["gu"]), act=f32(fwd["act"]), y=f32(fwd["y"]), dx=f32(bwd["dx"]),
        dw=f32(bwd["dw"]), dw1=f32(bwd["dw1"]), dw2=f32(bwd["dw2"]),
    )


def main():
    with open(os.path.join(HERE, "reference_kats.json"), "w") as f:
        json.dump(KATS, f, indent=1)
    np.savez_compressed(os.path.join(HERE, "oracle_small.npz"), **small_vectors())
    np.savez_compressed(os.path.join(HERE, "oracle_small_f16.npz"), **small_vectors(torch.float16))
    print("wrote", HERE)


if __name__ == "__main__":
    main()
