"""Route statistics (placement planner input): the oracle against the
reference's known answer, a brute-force pair count and the invariants, and
the host API's argument checks (which run before any GPU call)."""

import itertools

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from placemoe_amd.statistics import ProfileStatistics, profile_route_statistics

# tests/distributed/test_placemoe_optimizer.py:50-73: one sample, two sources.
KAT_SAMPLES = [[np.array([[0, 1], [0, 2]]), np.array([[2, 3], [1, 3]])]]


def brute_force(samples, E):
    S = len(samples[0])
    demand = np.zeros((S, E))
    affinity = np.zeros((S, E, E))
    for sample in samples:
        for s, route in enumerate(sample):
            for row in np.asarray(route).tolist():
                for e in row:
                    demand[s, e] += 1
                for a, b in itertools.combinations(row, 2):
                    if a != b:
                        affinity[s, a, b] += 1
                        affinity[s, b, a] += 1
    return demand, affinity


def test_oracle_matches_reference_known_answer():
    demand, affinity = O.route_statistics(KAT_SAMPLES, 4)
    np.testing.assert_array_equal(demand, [[2, 1, 1, 0], [0, 1, 1, 2]])
    assert affinity[0, 0, 1] == 1 and affinity[0, 0, 2] == 1
    assert affinity[1, 1, 3] == 1 and affinity[1, 2, 3] == 1
    np.testing.assert_array_equal(affinity, affinity.transpose(0, 2, 1))
    # no other pair was co-selected
    assert affinity.sum() == 8


@pytest.mark.parametrize("seed,S,E,K,T", [(0, 1, 5, 2, 40), (1, 3, 7, 4, 25), (2, 2, 16, 8, 12), (3, 4, 3, 3, 30)])
def test_oracle_matches_brute_force_and_invariants(seed, S, E, K, T):
    rng = np.random.default_rng(seed)
    # repeats within a row included: a token may list one expert twice
    samples = [[rng.integers(0, E, size=(T + s, K)) for s in range(S)] for _ in range(2)]
    demand, affinity = O.route_statistics(samples, E)
    bd, ba = brute_force(samples, E)
    np.testing.assert_array_equal(demand, bd)
    np.testing.assert_array_equal(affinity, ba)
    for s in range(S):
        assert demand[s].sum() == 2 * (T + s) * K
        assert np.all(np.diagonal(affinity[s]) == 0)
    np.testing.assert_array_equal(affinity, affinity.transpose(0, 2, 1))


def test_a_one_sided_pair_count_is_caught():
    """A plausible mistake - counting each pair in one order only - fails the
    known answer's symmetry."""
    route = KAT_SAMPLES[0][0]
    one_sided = np.zeros((4, 4))
    for a, b in route.tolist():
        one_sided[a, b] += 1
    _, affinity = O.route_statistics(KAT_SAMPLES, 4)
    assert not np.array_equal(one_sided, affinity[0])


def test_profile_statistics_validation_mirrors_reference():
    ok = ProfileStatistics(demand=np.zeros((2, 3)), affinity=np.zeros((2, 3, 3)))
    assert ok.ep_size == 2 and ok.num_experts == 3 and not ok.demand.flags.writeable
    with pytest.raises(ValueError, match="demand must have shape"):
        ProfileStatistics(demand=np.zeros(3), affinity=np.zeros((1, 3, 3)))
    with pytest.raises(ValueError, match="affinity must have shape"):
        ProfileStatistics(demand=np.zeros((2, 3)), affinity=np.zeros((2, 3, 2)))
    with pytest.raises(ValueError, match="non-negative"):
        ProfileStatistics(demand=-np.ones((1, 2)), affinity=np.zeros((1, 2, 2)))
    asym = np.zeros((1, 2, 2))
    asym[0, 0, 1] = 1
    with pytest.raises(ValueError, match="symmetric"):
        ProfileStatistics(demand=np.zeros((1, 2)), affinity=asym)
    with pytest.raises(ValueError, match="diagonal"):
        ProfileStatistics(demand=np.zeros((1, 2)), affinity=np.eye(2)[None])


def test_profile_route_statistics_argument_errors():
    r = torch.zeros((3, 2), dtype=torch.int64)
    with pytest.raises(ValueError, match="At least one routing sample"):
        profile_route_statistics([], num_experts=4)
    with pytest.raises(ValueError, match="num_experts must be positive"):
        profile_route_statistics([[r]], num_experts=0)
    with pytest.raises(ValueError, match="same source ranks"):
        profile_route_statistics([[r, r], [r]], num_experts=4)
    with pytest.raises(ValueError, match=r"shape \[tokens, top_k\]"):
        profile_route_statistics([[torch.zeros(3, dtype=torch.int64)]], num_experts=4)
