"""Replica-gradient exchange on the GPU: every rank's pack / unpack through
the C-ABI (``pmx_replica_exchange_pack`` / ``_unpack``), with the ranks
simulated in one process and the transfers done by handing buffers over.
Checked against the oracle's restatement of the reference
(``replica_grad_sync``) and against the exact float64 totals."""

import ctypes

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from placemoe_amd import _capi
from placemoe_amd.replica import ReplicaGradExchange, replica_grad_schedule

from tests.test_replica_exchange import fill_grads, random_layout

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def hand_over(sends, r):
    """What rank r receives: {dtype: {source: buffer}}."""
    out = {}
    for src, per_dtype in enumerate(sends):
        for dtype, bufs in per_dtype.items():
            if r in bufs:
                out.setdefault(dtype, {})[src] = bufs[r]
    return out


def run_exchange(L, owners, num_local, grads):
    R = len(grads)
    ex = [ReplicaGradExchange(replica_grad_schedule(L, owners, num_local, r, R), r, grads[r]) for r in range(R)]
    if ex[0].schedule.pairwise:
        sends = [e.pairwise_send() for e in ex]
        for r in range(R):
            ex[r].pairwise_finish(hand_over(sends, r))
    else:
        sends = [e.owner_reduce_send() for e in ex]
        bcast = [ex[r].owner_reduce_finish(hand_over(sends, r)) for r in range(R)]
        for r in range(R):
            ex[r].owner_broadcast_finish(hand_over(bcast, r))
    torch.cuda.synchronize()
    return ex


def to_dev(grads, dtypes):
    return [tuple(t.to(DEV, dt).contiguous() for t, dt in zip(g, dtypes)) for g in grads]


def exact_totals(grads64, L, num_local):
    """float64 copy gradients after an exact exchange."""
    out = [tuple(t.clone() for t in g) for g in grads64]
    L = np.asarray(L)
    for e in np.unique(L[L >= 0]):
        slots = np.nonzero(L == e)[0]
        if len(slots) < 2:
            continue
        for p in range(len(grads64[0])):
            tot = sum(grads64[s // num_local][p][s % num_local] for s in slots)
            for s in slots:
                out[s // num_local][p][s % num_local] = tot
    return out


@pytest.mark.parametrize("case", ["cover", "owner3", "pair_graph"])
def test_reference_known_answers(case):
    if case == "cover":
        L, owners, nl, R = [0, 1, 3, 2, 3, -1], [0, 1, 3, 2], 3, 2
        vals = {(0, 2): (10.0, 20.0), (1, 1): (2.0, 3.0)}
        fn = lambda r, ls, e: vals.get((r, ls), (0.0, 0.0))  # noqa: E731
    elif case == "owner3":
        L, owners, nl, R = [0, -1, 0, 1, 0, 2], [2, 3, 5], 2, 3
        fn = lambda r, ls, e: (r + 1.0, 10.0 * (r + 1)) if ls == 0 else (0.0, 0.0)  # noqa: E731
    else:
        L, owners, nl, R = [0, 1, 0, 2, 1, 3, 2, 3], [0, 1, 3, 5], 2, 4
        fn = lambda r, ls, e: (10.0 * (r + 1) + e, 100.0 * (r + 1) + e)  # noqa: E731
    cpu = fill_grads(L, nl, R, shape=(3, 5), value=fn)
    expect = O.replica_grad_sync(cpu, L, owners, nl)
    for dtypes in ((torch.float32, torch.float32), (torch.bfloat16, torch.float32)):
        grads = to_dev(cpu, dtypes)
        run_exchange(L, owners, nl, grads)
        for r in range(R):
            for p in range(2):
                ref = expect[r][p].to(dtypes[p])  # the known answers are exact in both dtypes except 402 / 604 / 706 in bf16
                torch.testing.assert_close(grads[r][p].cpu(), ref, rtol=0, atol=0)


@pytest.mark.parametrize("max_ranks", [2, 3])
@pytest.mark.parametrize("seed", [0, 1, 2, 3])
@pytest.mark.parametrize("dtypes", [(torch.bfloat16, torch.bfloat16), (torch.float32, torch.float32),
                                    (torch.bfloat16, torch.float32), (torch.float16, torch.float16)])
def test_random_layouts_match_oracle(max_ranks, seed, dtypes):
    rng = np.random.default_rng(seed)
    R, nl, E = 4, 6, 11
    L, owners = random_layout(rng, R, nl, E, max_ranks)
    # P = 35 and 280: a ragged tail of the 16-byte vectors and a whole number of them
    cpu64 = fill_grads(list(L), nl, R, shape=(5, 7), dtype=torch.float64, seed=seed)
    cpu64 = [(gu, torch.randn(nl, 14, 20, dtype=torch.float64, generator=torch.Generator().manual_seed(seed + r)))
             for r, (gu, _) in enumerate(cpu64)]
    cpu = [tuple(t.to(dt) for t, dt in zip(g, dtypes)) for g in cpu64]
    grads = to_dev(cpu, dtypes)
    run_exchange(L, owners, nl, grads)
    oracle = O.replica_grad_sync(cpu, L, owners, nl)
    exact = exact_totals([tuple(t.double() for t in g) for g in cpu], L, nl)
    for r in range(R):
        for p, dt in enumerate(dtypes):
            got = grads[r][p].cpu().double()
            ex = exact[r][p]
            scale = ex.abs().max().item() + 1e-30
            if dt in (torch.bfloat16, torch.float16):
                # partial sums cross ranks in the 16-bit gradient dtype (the reference's buffer
                # dtype), so a total is rounded at most twice: the sending rank's partial, then
                # the fp32 total (bf16: 8 significant bits, fp16: 11)
                ulp = 2 ** -7 if dt == torch.bfloat16 else 2 ** -10
                assert (got - ex).abs().max().item() <= ulp * ex.abs().max().item() + 1e-6
                assert (got - oracle[r][p].double()).abs().max().item() / scale <= 1e-2
            else:
                assert (got - ex).abs().max().item() / scale <= 1e-6
                assert (got - oracle[r][p].double()).abs().max().item() / scale <= 1e-5


def test_buffers_follow_reference_layout():
    # Pairwise send buffer to the peer: items expert-major, parameter-minor,
    # each the local sum (as _pack_replica_grad_items lays them out).
    L, owners, nl = [0, 1, 2, 0, 1, 3], [0, 1, 2, 5], 3
    cpu = fill_grads(L, nl, 2, shape=(2, 3), dtype=torch.float32, seed=7)
    grads = to_dev(cpu, (torch.float32, torch.float32))
    ex = ReplicaGradExchange(replica_grad_schedule(L, owners, nl, 0, 2), 0, grads[0])
    buf = ex.pairwise_send()[torch.float32][1].cpu()
    want = torch.cat([cpu[0][0][0].reshape(-1), cpu[0][1][0].reshape(-1), cpu[0][0][1].reshape(-1),
                      cpu[0][1][1].reshape(-1)])
    torch.testing.assert_close(buf, want, rtol=0, atol=0)


def test_bad_slot_sets_status():
    g = torch.randn(4, 64, device=DEV).to(torch.bfloat16)
    before = g.clone()
    off = torch.tensor([0, 2], dtype=torch.int32, device=DEV)
    slots = torch.tensor([1, 9], dtype=torch.int32, device=DEV)  # 9 is outside [0, 4)
    out = torch.zeros(64, dtype=torch.bfloat16, device=DEV)
    o_off = torch.tensor([0, 1], dtype=torch.int32, device=DEV)
    o_ptr = torch.tensor([out.data_ptr()], dtype=torch.int64, device=DEV)
    status = torch.zeros(1, dtype=torch.int32, device=DEV)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _capi.call("pmx_replica_exchange_pack", g.data_ptr(), 0, 64, 4, 1, off.data_ptr(), slots.data_ptr(),
               o_off.data_ptr(), o_ptr.data_ptr(), status.data_ptr(), stream)
    torch.cuda.synchronize()
    assert int(status.item()) == 1
    torch.testing.assert_close(out, before[1], rtol=0, atol=0)
    assert torch.equal(g, before)


def test_inactive_slots_are_zeroed_first():
    # _zero_inactive_slot_grads_for_layer (expert_swap.py:6250-6262): a copy
    # that saw no tokens contributes nothing and then receives the total.
    L, owners, nl = [0, 1, 0, 1], [0, 1], 2
    cpu = fill_grads(L, nl, 2, value=lambda r, ls, e: (10.0 * (r + 1) + e, 100.0 * (r + 1) + e))
    grads = to_dev(cpu, (torch.float32, torch.float32))
    tokens = [torch.tensor([5, 0]), torch.tensor([3, 2])]  # rank 0's copy of expert 1 is idle
    R = 2
    ex = [ReplicaGradExchange(replica_grad_schedule(L, owners, nl, r, R), r, grads[r], slot_tokens=tokens[r])
          for r in range(R)]
    sends = [e.pairwise_send() for e in ex]
    for r in range(R):
        ex[r].pairwise_finish(hand_over(sends, r))
    torch.cuda.synchronize()
    for r in range(R):
        assert torch.all(grads[r][0][0].cpu() == 10.0 + 20.0)        # expert 0: both copies active
        assert torch.all(grads[r][0][1].cpu() == 21.0)               # expert 1: only rank 1's copy
        assert torch.all(grads[r][1][1].cpu() == 201.0)
    # a count vector of the wrong length is ignored, as in the reference
    g2 = to_dev(cpu, (torch.float32, torch.float32))
    ReplicaGradExchange(replica_grad_schedule(L, owners, nl, 0, R), 0, g2[0], slot_tokens=torch.tensor([0, 0, 0]))
    torch.testing.assert_close(g2[0][0].cpu(), cpu[0][0], rtol=0, atol=0)
