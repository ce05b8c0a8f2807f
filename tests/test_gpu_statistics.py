"""GPU route statistics (pmx_route_statistics) against the CPU oracle:
exact integer counts, the reference's known answer, accumulation across
samples, per-token sources and invalid ids."""

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from placemoe_amd.statistics import RouteStatisticsRecorder, profile_route_statistics
from placemoe_amd.workloads import make_workload

pytestmark = pytest.mark.gpu


def test_reference_known_answer(cuda):
    samples = [[torch.tensor([[0, 1], [0, 2]]), torch.tensor([[2, 3], [1, 3]])]]
    stats = profile_route_statistics(samples, num_experts=4)
    np.testing.assert_array_equal(stats.demand, [[2, 1, 1, 0], [0, 1, 1, 2]])
    assert stats.affinity[0, 0, 1] == 1 and stats.affinity[0, 0, 2] == 1
    assert stats.affinity[1, 1, 3] == 1 and stats.affinity[1, 2, 3] == 1
    assert stats.affinity.sum() == 8


@pytest.mark.parametrize("seed,S,E,K,T", [(0, 2, 8, 2, 1000), (1, 8, 128, 8, 4096), (2, 16, 64, 4, 3000),
                                          (3, 1, 3, 1, 17), (4, 4, 256, 32, 200),
                                          # co-selection table in LDS: S*E*E <= 16384, many tokens per block
                                          (5, 1, 128, 8, 20000), (6, 4, 64, 6, 2500), (7, 1, 2, 2, 9000)])
def test_matches_oracle_over_samples(cuda, seed, S, E, K, T):
    print(f"stats seed={seed} S={S} E={E} K={K} T={T}", flush=True)
    g = torch.Generator().manual_seed(seed)
    samples = [[torch.randint(0, E, (T + 7 * s, K), generator=g) for s in range(S)] for _ in range(2)]
    stats = profile_route_statistics([[r.to(cuda) for r in smp] for smp in samples], num_experts=E)
    demand, affinity = O.route_statistics([[r.numpy() for r in smp] for smp in samples], E)
    np.testing.assert_array_equal(stats.demand, demand)
    np.testing.assert_array_equal(stats.affinity, affinity)


@pytest.mark.parametrize("seed,S,E,K,T", [(8, 8, 128, 8, 6000), (9, 2, 96, 6, 5000)])
def test_skewed_routing_with_repeats_matches_oracle(cuda, seed, S, E, K, T):
    # Global co-selection table (S*E*E > 16384) under heavy skew: most picks
    # fall on four experts, so many lanes of a wave hold the same pair, and
    # repeated experts inside a token (ea == eb) add nothing.
    print(f"stats skewed seed={seed} S={S} E={E} K={K} T={T}", flush=True)
    g = torch.Generator().manual_seed(seed)
    def draw(n):
        hot = torch.randint(0, 4, (n, K), generator=g)
        cold = torch.randint(0, E, (n, K), generator=g)
        return torch.where(torch.rand((n, K), generator=g) < 0.85, hot, cold)
    samples = [[draw(T + 5 * s) for s in range(S)]]
    stats = profile_route_statistics([[r.to(cuda) for r in smp] for smp in samples], num_experts=E)
    demand, affinity = O.route_statistics([[r.numpy() for r in smp] for smp in samples], E)
    np.testing.assert_array_equal(stats.demand, demand)
    np.testing.assert_array_equal(stats.affinity, affinity)


def test_per_token_sources_match_split_by_source(cuda):
    wl = make_workload("qwen3", device=cuda, weights=False)
    rec = RouteStatisticsRecorder(8, wl.num_experts)
    rec.record(wl.selected, wl.sources)
    assert not rec.invalid()
    stats = rec.statistics()
    sel, src = wl.selected.cpu().numpy(), wl.sources.cpu().numpy()
    demand, affinity = O.route_statistics([[sel[src == s] for s in range(8)]], wl.num_experts)
    np.testing.assert_array_equal(stats.demand, demand)
    np.testing.assert_array_equal(stats.affinity, affinity)
    assert stats.demand.sum() == wl.T * wl.K


def test_empty_route_and_reset(cuda):
    rec = RouteStatisticsRecorder(2, 4)
    rec.record(torch.zeros((0, 3), dtype=torch.int64, device=cuda), 1)
    rec.record(torch.tensor([[1, 1, 2]], device=cuda), 0)  # a repeated expert stays off the diagonal
    st = rec.statistics()
    assert st.demand.tolist() == [[0, 2, 1, 0], [0, 0, 0, 0]]
    assert st.affinity[0, 1, 2] == 2 and st.affinity[0, 2, 1] == 2 and st.affinity[0, 1, 1] == 0
    rec.reset()
    assert rec.statistics().demand.sum() == 0


def test_invalid_expert_id_raises(cuda):
    with pytest.raises(ValueError, match="invalid logical expert ID"):
        profile_route_statistics([[torch.tensor([[0, 4]], device=cuda)]], num_experts=4)
    rec = RouteStatisticsRecorder(2, 4)
    rec.record(torch.tensor([[0, 1], [2, 3]], device=cuda), torch.tensor([0, 5], device=cuda))
    assert rec.invalid()
    assert rec.statistics().demand.sum() == 2  # the token with a bad source is not counted
