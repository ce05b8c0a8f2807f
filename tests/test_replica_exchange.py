"""Cross-rank replica-gradient exchange, host side and oracle: the
reference's three known answers (tests/distributed/test_hiermoe.py), the
"every copy ends with the expert's total" invariant on random layouts, and
the schedule / grad-norm mask of ``placemoe_amd.replica`` against the oracle."""

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from placemoe_amd.replica import redundant_grad_norm_mask, replica_grad_schedule


def fill_grads(L, num_local, R, shape=(2, 2), value=None, dtype=torch.float32, seed=0):
    g = torch.Generator().manual_seed(seed)
    out = []
    for r in range(R):
        gu = torch.zeros((num_local,) + shape, dtype=dtype)
        dn = torch.zeros((num_local,) + shape[::-1], dtype=dtype)
        for ls in range(num_local):
            e = L[r * num_local + ls]
            if value is not None:
                a, b = value(r, ls, e)
                gu[ls].fill_(a)
                dn[ls].fill_(b)
            else:
                gu[ls] = torch.randn(shape, generator=g, dtype=torch.float64).to(dtype)
                dn[ls] = torch.randn(shape[::-1], generator=g, dtype=torch.float64).to(dtype)
        out.append((gu, dn))
    return out


def test_known_answer_two_rank_cover():
    # test_hiermoe.py:3200-3338: L = [0,1,3,2,3,-1]; expert 3 on rank 0 slot 2 and rank 1 slot 1.
    L = [0, 1, 3, 2, 3, -1]
    vals = {(0, 2): (10.0, 20.0), (1, 1): (2.0, 3.0)}
    grads = fill_grads(L, 3, 2, value=lambda r, ls, e: vals.get((r, ls), (0.0, 0.0)))
    out = O.replica_grad_sync(grads, L, [0, 1, 3, 2], 3)
    assert torch.all(out[0][0][2] == 12.0) and torch.all(out[0][1][2] == 23.0)
    assert torch.all(out[1][0][1] == 12.0) and torch.all(out[1][1][1] == 23.0)
    assert O.replica_grad_schedule(L, [0, 1, 3, 2], 3, 0, 2)["pairwise"]


def test_known_answer_three_copy_owner():
    # test_hiermoe.py:3545-3592: L = [0,-1,0,1,0,2], owners (2,3,5): expert 0 owned by rank 1.
    L, owners = [0, -1, 0, 1, 0, 2], [2, 3, 5]
    grads = fill_grads(L, 2, 3, value=lambda r, ls, e: (r + 1.0, 10.0 * (r + 1)) if ls == 0 else (0.0, 0.0))
    out = O.replica_grad_sync(grads, L, owners, 2)
    for r in range(3):
        assert torch.all(out[r][0][0] == 6.0) and torch.all(out[r][1][0] == 60.0)
    s = O.replica_grad_schedule(L, owners, 2, 1, 3)
    assert not s["pairwise"] and s["groups"][0][1] == 1


def test_known_answer_pair_graph():
    # test_hiermoe.py:3480-3540: L = [0,1,0,2,1,3,2,3], owners (0,1,3,5).
    L, owners = [0, 1, 0, 2, 1, 3, 2, 3], [0, 1, 3, 5]
    grads = fill_grads(L, 2, 4, value=lambda r, ls, e: (10.0 * (r + 1) + e, 100.0 * (r + 1) + e))
    out = O.replica_grad_sync(grads, L, owners, 2)
    expected = {0: (30.0, 300.0), 1: (42.0, 402.0), 2: (64.0, 604.0), 3: (76.0, 706.0)}
    for r in range(4):
        for ls in range(2):
            a, b = expected[L[r * 2 + ls]]
            assert torch.all(out[r][0][ls] == a) and torch.all(out[r][1][ls] == b)
    s = O.replica_grad_schedule(L, owners, 2, 0, 4)
    assert s["pairwise"] and s["globally_ordered_pairs"]


def random_layout(rng, R, num_local, E, max_ranks):
    """Each expert gets 1-4 copies on at most `max_ranks` ranks; free slots stay -1."""
    L = -np.ones(R * num_local, dtype=np.int64)
    free = list(rng.permutation(R * num_local))
    for e in range(E):
        L[free.pop()] = e
    for e in rng.permutation(E):
        if len(free) == 0:
            break
        ranks = {int(s) // num_local for s in np.nonzero(L == e)[0]}
        for s in list(free):
            if rng.random() < 0.3 and (s // num_local in ranks or len(ranks) < max_ranks):
                L[s] = e
                ranks.add(s // num_local)
                free.remove(s)
    owners = np.array([rng.choice(np.nonzero(L == e)[0]) for e in range(E)])
    return L, owners


def check_synced(out, grads, L, num_local):
    """Every copy of an expert with several copies holds the exact sum of all
    of its copies; every other slot is unchanged (float64)."""
    R = len(grads)
    L = np.asarray(L)
    for e in np.unique(L[L >= 0]):
        slots = np.nonzero(L == e)[0]
        for p in range(len(grads[0])):
            total = sum(grads[s // num_local][p][s % num_local] for s in slots)
            for s in slots:
                got = out[s // num_local][p][s % num_local]
                if not torch.allclose(got, total if len(slots) > 1 else grads[s // num_local][p][s % num_local],
                                      rtol=1e-12, atol=1e-12):
                    return False
    for s in np.nonzero(L < 0)[0]:
        for p in range(len(grads[0])):
            if not torch.equal(out[s // num_local][p][s % num_local], grads[s // num_local][p][s % num_local]):
                return False
    return True


@pytest.mark.parametrize("max_ranks", [2, 3])
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_oracle_sync_invariant(max_ranks, seed):
    rng = np.random.default_rng(seed)
    R, num_local, E = 4, 5, 9
    L, owners = random_layout(rng, R, num_local, E, max_ranks)
    grads = fill_grads(list(L), num_local, R, shape=(3, 4), dtype=torch.float64, seed=seed)
    out = O.replica_grad_sync(grads, L, owners, num_local)
    assert check_synced(out, grads, L, num_local)
    # a planted mistake (one copy missing the remote part) is caught
    bad = [tuple(t.clone() for t in g) for g in out]
    multi = [e for e in range(E) if len({s // num_local for s in np.nonzero(L == e)[0]}) > 1]
    s = int(np.nonzero(L == multi[0])[0][0])
    bad[s // num_local][0][s % num_local] = grads[s // num_local][0][s % num_local]
    assert not check_synced(bad, grads, L, num_local)


@pytest.mark.parametrize("seed", range(6))
def test_schedule_matches_oracle(seed):
    rng = np.random.default_rng(100 + seed)
    R, num_local, E = 4, 4, 7
    L, owners = random_layout(rng, R, num_local, E, 2 if seed % 2 else 4)
    for r in range(R):
        ref = O.replica_grad_schedule(L, owners, num_local, r, R)
        got = replica_grad_schedule(L, owners, num_local, r, R)
        assert [(g.logical_expert, g.owner_rank, g.copy_ranks, g.local_slots) for g in got.groups] == ref["groups"]
        assert got.pairwise == ref["pairwise"]
        assert got.globally_ordered_pairs == ref["globally_ordered_pairs"]
        mask = redundant_grad_norm_mask(L, owners, num_local, r)
        if mask is not None:
            assert mask.numpy().tolist() == O.owner_grad_norm_mask(owners, num_local, r).tolist()


def test_mirrored_r2_schedule_is_pairwise_single_wave():
    # Fixed mirrored R2 (every expert on ranks r and r + R/2): one peer per rank.
    R, num_local = 4, 2
    E = R * num_local // 2
    L = np.concatenate([np.arange(E), np.arange(E)])
    owners = np.arange(E)
    s = replica_grad_schedule(L, owners, num_local, 0, R)
    assert s.pairwise and not s.globally_ordered_pairs
    assert all(g.copy_ranks in ((0, 2), (1, 3)) for g in s.groups)


def test_schedule_errors_and_mask_without_replicas():
    with pytest.raises(RuntimeError, match="owner slot 1 for logical expert 0 is not in its copy group"):
        replica_grad_schedule([0, 1, 0, 2], [1, 1, 3], 2, 0, 2)
    assert redundant_grad_norm_mask([0, 1, 2, 3], [0, 1, 2, 3], 2, 0) is None
    m = redundant_grad_norm_mask([0, 1, 0, 2], [2, 1, 3], 2, 1)
    assert m.tolist() == [True, True]
