"""Expert-parallel payload oracle: the reference's known answer for the
combine aggregation, a dictionary-based pure-Python payload, and the
reference's end-to-end property (rank-dedup dispatch + experts + combine ==
eager MoE) with the ranks simulated in one process, in float64."""

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O


def test_aggregate_reference_known_answer():
    # tests/distributed/test_hiermoe.py:1116-1128
    weighted = torch.tensor([[1.0], [2.0]])
    combined, splits = O.aggregate_weighted_outputs(weighted, [3, 0], [1, 1], key_stride=4)
    assert splits == [1, 1]
    torch.testing.assert_close(combined, weighted)


def brute_payload(phys, num_slots, R):
    T, K = phys.shape
    L = num_slots // R
    pairs = {}  # (rank, token) -> list of (k, slot)
    for t in range(T):
        for k in range(K):
            r = int(phys[t, k]) // L
            pairs.setdefault((r, t), []).append((k, int(phys[t, k])))
    keys = sorted(pairs)
    usplits = [sum(1 for r, _ in keys if r == q) for q in range(R)]
    meta, unique_tokens = [], []
    ordinal_in_rank = {}
    for r, t in keys:
        ordinal_in_rank[(r, t)] = sum(1 for rr, tt in keys if rr == r and tt < t)
        unique_tokens.append(t)
    for r, t in keys:
        for k, slot in pairs[(r, t)]:
            meta.append((ordinal_in_rank[(r, t)], slot - r * L, t))
    return usplits, np.array(meta, dtype=np.int32).reshape(-1, 3), np.array(unique_tokens)


@pytest.mark.parametrize("seed,T,K,R,L", [(0, 7, 2, 2, 3), (1, 20, 4, 4, 2), (2, 13, 8, 3, 5), (3, 5, 1, 4, 1)])
def test_payload_matches_brute_force(seed, T, K, R, L):
    rng = np.random.default_rng(seed)
    phys = rng.integers(0, R * L, size=(T, K))
    hidden = torch.randn(T, 4, dtype=torch.float64)
    w = torch.rand(T, K, dtype=torch.float64)
    p = O.build_local_payload(hidden, phys, w, R * L, R)
    usplits, meta, utok = brute_payload(phys, R * L, R)
    assert p["unique_send_splits"] == usplits
    assert p["assignment_send_splits"] == np.bincount(phys.reshape(-1) // L, minlength=R).tolist()
    np.testing.assert_array_equal(p["send_meta"], meta)
    np.testing.assert_array_equal(p["unique_tokens"], utok)
    torch.testing.assert_close(p["send_hidden"], hidden[torch.as_tensor(utok)])


def simulate_ep(hidden_by_rank, phys_by_rank, w_by_rank, expert_weight, R, L, payload=O.build_local_payload,
                aggregate=O.aggregate_weighted_outputs):
    """dispatch -> all-to-all (simulated) -> per-slot linear experts -> combine
    -> all-to-all back -> fp32 index_add into the source tokens."""
    pays = [payload(hidden_by_rank[r], phys_by_rank[r], w_by_rank[r], R * L, R) for r in range(R)]
    outs = []
    partial_by_src = {r: [] for r in range(R)}
    for q in range(R):  # receiving rank
        hid, meta, wts, ranks = [], [], [], []
        for r in range(R):
            p = pays[r]
            uo = np.concatenate([[0], np.cumsum(p["unique_send_splits"])])
            ao = np.concatenate([[0], np.cumsum(p["assignment_send_splits"])])
            hid.append(p["send_hidden"][uo[q]:uo[q + 1]])
            meta.append(np.asarray(p["send_meta"])[ao[q]:ao[q + 1]])
            wts.append(p["send_weights"][ao[q]:ao[q + 1]])
            ranks += [r] * int(ao[q + 1] - ao[q])
        recv_hidden, recv_meta, recv_w = torch.cat(hid), np.concatenate(meta), torch.cat(wts)
        usplit = [int(h.shape[0]) for h in hid]
        uoff = np.concatenate([[0], np.cumsum(usplit)])[np.asarray(ranks, dtype=np.int64)]
        rows = recv_hidden[torch.as_tensor(uoff + recv_meta[:, 0])]
        slots = q * L + recv_meta[:, 1]
        y = torch.stack([rows[i] @ expert_weight[slots[i]].t() for i in range(rows.shape[0])]) \
            if rows.shape[0] else rows
        weighted = y * recv_w
        asplits = [int(m.shape[0]) for m in meta]
        sums, splits = aggregate(weighted, recv_meta[:, 2], asplits, None)
        off = np.concatenate([[0], np.cumsum(splits)])
        for r in range(R):
            partial_by_src[r].append(sums[off[r]:off[r + 1]])
    for r in range(R):
        partial = torch.cat(partial_by_src[r])
        out = torch.zeros((hidden_by_rank[r].shape[0], partial.shape[1]), dtype=torch.float64, device=partial.device)
        out.index_add_(0, torch.as_tensor(pays[r]["unique_tokens"], device=partial.device), partial.double())
        outs.append(out)
    return outs


@pytest.mark.parametrize("seed,R,L,T,K", [(0, 2, 2, 6, 2), (1, 4, 3, 9, 4), (2, 3, 4, 5, 3)])
def test_dispatch_combine_round_trip_equals_eager_moe(seed, R, L, T, K):
    g = torch.Generator().manual_seed(seed)
    H = 5
    W = torch.randn(R * L, H, H, dtype=torch.float64, generator=g)
    hid = [torch.randn(T, H, dtype=torch.float64, generator=g) for _ in range(R)]
    phys = [torch.randint(0, R * L, (T, K), generator=g).numpy() for _ in range(R)]
    w = [torch.rand(T, K, dtype=torch.float64, generator=g) for _ in range(R)]
    outs = simulate_ep(hid, phys, w, W, R, L)
    for r in range(R):
        eager = torch.zeros(T, H, dtype=torch.float64)
        for t in range(T):
            for k in range(K):
                eager[t] += w[r][t, k] * (hid[r][t] @ W[phys[r][t, k]].t())
        # the aggregation sums in fp32 (the reference's index_add); the
        # reference's own round-trip test allows 1e-5 (test_hiermoe.py:996)
        torch.testing.assert_close(outs[r], eager, rtol=1e-5, atol=1e-5)


def test_a_dropped_dedup_is_caught():
    """A plausible mistake - sending one row per assignment instead of per
    (rank, token) - changes the unique splits the brute force expects."""
    phys = np.array([[0, 1], [2, 3]])  # R=2, L=2: token 0 sends twice to rank 0
    usplits, _, _ = brute_payload(phys, 4, 2)
    assert usplits == [1, 1]
    assert np.bincount(phys.reshape(-1) // 2, minlength=2).tolist() == [2, 2]
