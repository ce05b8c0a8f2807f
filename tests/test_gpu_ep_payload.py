"""GPU expert-parallel payloads (pmx_ep_dispatch_payload,
pmx_ep_combine_aggregate) against the CPU oracle: bit-exact integer
payloads and row copies, the reference's aggregation known answer, and the
dispatch + experts + combine round trip across ranks simulated on one GPU."""

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from placemoe_amd import ep_payload as EP
from placemoe_amd import kernels
from placemoe_amd.workloads import make_workload
from tests.helpers import assert_bf16_close
from tests.test_ep_payload import simulate_ep

pytestmark = pytest.mark.gpu


def _check_payload(cuda, hidden, phys, w, num_slots, R):
    got = EP.build_local_payload(hidden.to(cuda), torch.as_tensor(phys).to(cuda), w.to(cuda), num_slots, R,
                                 physical_experts=torch.as_tensor(phys).to(cuda))
    ref = O.build_local_payload(hidden, np.asarray(phys), w, num_slots, R)
    send_hidden, send_meta, send_w, utok, usplits, asplits, ranks = got
    assert usplits == ref["unique_send_splits"]
    assert asplits == ref["assignment_send_splits"]
    np.testing.assert_array_equal(send_meta.cpu().numpy(), ref["send_meta"])
    np.testing.assert_array_equal(utok.cpu().numpy(), ref["unique_tokens"])
    np.testing.assert_array_equal(ranks.cpu().numpy(), ref["target_ranks"])
    assert torch.equal(send_hidden.cpu(), ref["send_hidden"])
    assert torch.equal(send_w.cpu(), ref["send_weights"])


@pytest.mark.parametrize("seed,T,K,R,L,H", [(0, 7, 2, 2, 3, 8), (1, 300, 4, 4, 2, 64), (2, 129, 8, 3, 5, 40),
                                            (3, 50, 1, 4, 1, 16), (4, 1000, 32, 8, 4, 24)])
def test_payload_matches_oracle(cuda, seed, T, K, R, L, H):
    print(f"payload seed={seed} T={T} K={K} R={R} L={L} H={H}", flush=True)
    g = torch.Generator().manual_seed(seed)
    phys = torch.randint(0, R * L, (T, K), generator=g).numpy()
    hidden = torch.randn(T, H, generator=g).to(torch.bfloat16)
    w = torch.rand(T, K, generator=g).to(torch.bfloat16)
    _check_payload(cuda, hidden, phys, w, R * L, R)


def test_payload_at_qwen3_routing(cuda):
    """The config-2 routing (160 copies over 8 ranks of 20 slots), full size."""
    wl = make_workload("qwen3", weights=False)
    phys = O.map_logical_to_physical(wl.mapping.numpy(), wl.sources.numpy(), wl.selected.numpy())
    _check_payload(cuda, wl.hidden, phys, wl.routing_weights, wl.C, 8)


def test_payload_empty_and_bad_slot(cuda):
    got = EP.build_local_payload(torch.zeros((0, 8), dtype=torch.bfloat16, device=cuda),
                                 torch.zeros((0, 2), dtype=torch.long, device=cuda),
                                 torch.zeros((0, 2), dtype=torch.bfloat16, device=cuda), 4, 2)
    assert got[4] == [0, 0] and got[5] == [0, 0] and got[0].shape == (0, 8)
    with pytest.raises(ValueError, match="outside"):
        EP.build_local_payload(torch.zeros((1, 8), dtype=torch.bfloat16, device=cuda),
                               torch.tensor([[0, 9]], device=cuda), torch.ones((1, 2), dtype=torch.bfloat16,
                                                                                 device=cuda), 4, 2)


def test_aggregate_reference_known_answer(cuda):
    weighted = torch.tensor([[1.0], [2.0]], device=cuda)
    combined, splits = EP.aggregate_weighted_outputs(weighted, torch.tensor([3, 0], device=cuda), [1, 1],
                                                     key_stride=4)
    assert splits == [1, 1]
    torch.testing.assert_close(combined.cpu(), weighted.cpu())


@pytest.mark.parametrize("seed,N,H,R", [(0, 1, 8, 1), (1, 500, 64, 4), (2, 3000, 2048, 8)])
def test_combine_aggregate_matches_oracle(cuda, seed, N, H, R):
    g = torch.Generator().manual_seed(seed)
    splits = torch.multinomial(torch.ones(R), N, replacement=True, generator=g).bincount(minlength=R).tolist()
    # tokens ascending within each source rank, with repeats (several local experts per token)
    tokens = np.concatenate([np.sort(torch.randint(0, max(1, n // 2), (n,), generator=g).numpy()) for n in splits])
    y = torch.randn(N, H, generator=g).to(torch.bfloat16)
    pos = torch.randperm(N, generator=g)
    w = torch.rand(N, generator=g).to(torch.bfloat16)
    ranks = torch.repeat_interleave(torch.arange(R), torch.as_tensor(splits))
    got, gsplits = EP.combine_aggregate(y.to(cuda), pos.to(cuda), w.to(cuda), ranks.to(cuda),
                                        torch.as_tensor(tokens).to(cuda), R)
    weighted = (y[pos].float() * w.float()[:, None]).to(torch.bfloat16)
    ref, rsplits = O.aggregate_weighted_outputs(weighted, tokens, splits)
    assert gsplits == rsplits
    assert_bf16_close(got.cpu(), ref)


@pytest.mark.parametrize("seed,R,L,T,K,H", [(0, 2, 2, 16, 2, 32), (1, 4, 3, 24, 4, 64), (2, 8, 2, 12, 8, 16)])
def test_round_trip_across_simulated_ranks(cuda, seed, R, L, T, K, H):
    g = torch.Generator().manual_seed(seed)
    W = (torch.randn(R * L, H, H, generator=g) * 0.1).to(torch.bfloat16)
    hid = [torch.randn(T, H, generator=g).to(torch.bfloat16) for _ in range(R)]
    phys = [torch.randint(0, R * L, (T, K), generator=g).numpy() for _ in range(R)]
    w = [torch.rand(T, K, generator=g).to(torch.bfloat16) for _ in range(R)]

    def gpu_payload(hidden, ph, wt, num_slots, ranks):
        sh, meta, sw, utok, us, asp, tr = EP.build_local_payload(hidden, torch.as_tensor(ph).to(cuda), wt,
                                                                  num_slots, ranks,
                                                                  physical_experts=torch.as_tensor(ph).to(cuda))
        return {"send_hidden": sh, "send_meta": meta.cpu().numpy(), "send_weights": sw, "unique_tokens": utok.cpu(),
                "unique_send_splits": us, "assignment_send_splits": asp}

    def gpu_aggregate(weighted, tokens, splits, stride):
        return EP.aggregate_weighted_outputs(weighted, torch.as_tensor(tokens).to(cuda), splits, stride)

    outs = simulate_ep([h.to(cuda) for h in hid], phys, [x.to(cuda) for x in w], W.to(cuda), R, L,
                       payload=gpu_payload, aggregate=gpu_aggregate)
    for r in range(R):
        eager = torch.zeros(T, H, dtype=torch.float64)
        for t in range(T):
            for k in range(K):
                eager[t] += w[r][t, k].double() * (hid[r][t].double() @ W[phys[r][t, k]].double().t())
        assert_bf16_close(outs[r].cpu().to(torch.bfloat16), eager.float())
