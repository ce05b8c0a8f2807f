"""GPU parity of the integer routing path (map, histogram, scan, stable scatter
index) and the exact row permute, against the CPU oracle: bit-exact."""

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from placemoe_amd import kernels
from placemoe_amd.workloads import make_workload
from tests.helpers import assert_exact

pytestmark = pytest.mark.gpu


def _oracle_route(M, src, sel, C):
    return O.route(M, src, sel, C)


def _check_route(cuda, sel, C, M=None, src=None, source=0):
    sel_t = torch.as_tensor(sel, dtype=torch.int64)
    r = kernels.route(
        sel_t.to(cuda), C,
        mapping=None if M is None else torch.as_tensor(M, dtype=torch.int64).to(cuda),
        sources=None if src is None else torch.as_tensor(src, dtype=torch.int64).to(cuda),
        source=source,
    )
    T = sel_t.shape[0]
    if M is None:
        M_ = np.arange(C, dtype=np.int64).reshape(1, C)
        src_ = np.zeros(T, dtype=np.int64)
    else:
        M_ = np.asarray(M)
        src_ = np.full(T, source, dtype=np.int64) if src is None else np.asarray(src)
    phys, counts, offsets, pos = _oracle_route(M_, src_, sel_t.numpy().reshape(T, -1), C)
    assert kernels.route_status(r) == 0
    assert_exact(r.phys, phys, "phys")
    assert_exact(r.counts, counts, "counts")
    assert_exact(r.offsets, offsets, "offsets")
    assert_exact(r.pos, pos, "pos")
    return r


@pytest.mark.parametrize("name", ["toy", "qwen3", "dsv3", "skew", "fold"])
def test_route_full_size_configs_bit_exact(cuda, name):
    wl = make_workload(name, weights=False)
    src = None if wl.sources is None else wl.sources.numpy()
    print(f"route {name}: T={wl.T} K={wl.K} C={wl.C}", flush=True)
    r = _check_route(cuda, wl.selected.numpy(), wl.C, M=wl.mapping.numpy(), src=src)
    # size-independent properties: pos is a permutation, groups are contiguous
    pos = r.pos.cpu().numpy().reshape(-1)
    assert np.array_equal(np.sort(pos), np.arange(pos.size))
    phys = r.phys.cpu().numpy().reshape(-1)
    off = r.offsets.cpu().numpy()
    assert np.all((pos >= off[phys]) & (pos < off[phys + 1]))


def test_route_reference_lut_known_answer(cuda):
    # tests/distributed/test_hiermoe_forward_cover_planner.py:1032-1038:
    # LUT row 0 = (0,1,3,2) maps [[3,2,0]] -> [[2,3,0]]; row 1 = (5,1,3,4).
    M = np.array([[0, 1, 3, 2], [5, 1, 3, 4]])
    r = _check_route(cuda, np.array([[3, 2, 0]]), 6, M=M, source=0)
    assert r.phys.cpu().tolist() == [[2, 3, 0]]
    r1 = _check_route(cuda, np.array([[3, 2, 0]]), 6, M=M, source=1)
    assert r1.phys.cpu().tolist() == [[4, 3, 5]]


@pytest.mark.parametrize(
    "T,K,C,seed",
    [(1, 1, 1, 0), (1, 8, 3, 1), (63, 2, 5, 2), (64, 1, 7, 3), (65, 3, 9, 4), (2049, 2, 17, 5),
     (3000, 8, 4096, 6), (700, 4, 9000, 7), (40000, 8, 160, 8), (70000, 8, 1, 9),
     (9000, 8, 1023, 10), (9000, 8, 1025, 11), (300000, 2, 37, 12)],
)
def test_route_identity_random_edges(cuda, T, K, C, seed):
    g = np.random.default_rng(seed)
    sel = g.integers(0, C, size=(T, K))
    _check_route(cuda, sel, C)


def test_route_all_to_one_copy_and_empty_groups(cuda):
    sel = np.full((5000, 4), 3)
    r = _check_route(cuda, sel, 10)
    c = r.counts.cpu().tolist()
    assert c[3] == 20000 and sum(c) == 20000


def test_route_zero_tokens(cuda):
    r = kernels.route(torch.empty((0, 4), dtype=torch.int64, device=cuda), 6)
    assert r.counts.cpu().tolist() == [0] * 6
    assert r.offsets.cpu().tolist() == [0] * 7
    assert kernels.route_status(r) == 0
    # The same through the C ABI with a workspace full of stale bytes: no
    # assignment means no invalid id, whatever the workspace held before.
    from placemoe_amd import _capi

    lib = _capi.load()
    ws_bytes = lib.pmx_route_workspace_bytes(0, 6)
    ws = torch.full((ws_bytes,), 0xFF, dtype=torch.uint8, device=cuda)
    counts = torch.full((6,), -1, dtype=torch.int32, device=cuda)
    offsets = torch.full((7,), -1, dtype=torch.int32, device=cuda)
    stream = torch.cuda.current_stream(cuda).cuda_stream
    _capi.call("pmx_route", None, None, None, 0, 1, 6, 0, 4, 6, None, counts.data_ptr(), offsets.data_ptr(),
               None, ws.data_ptr(), ws_bytes, stream)
    assert counts.cpu().tolist() == [0] * 6 and offsets.cpu().tolist() == [0] * 7
    assert kernels.route_status(kernels.Routing(phys=None, counts=counts, offsets=offsets, pos=None,
                                                workspace=ws)) == 0


def test_route_out_of_range_is_flagged_not_faulting(cuda):
    sel = torch.tensor([[0, 9], [1, 2]], dtype=torch.int64, device=cuda)
    r = kernels.route(sel, 4)
    assert kernels.route_status(r) != 0
    pos = r.pos.cpu().numpy().reshape(-1)
    assert np.array_equal(np.sort(pos), np.arange(4))


def test_route_flag_from_one_chunk_of_many(cuda):
    # One id out of range deep inside a batch of hundreds of chunks: the
    # status word is the OR over every chunk's flag.
    g = np.random.default_rng(11)
    sel = g.integers(0, 100, size=(20000, 8))
    sel[15000, 3] = 100
    r = kernels.route(torch.as_tensor(sel).to(cuda), 100)
    assert kernels.route_status(r) != 0
    pos = r.pos.cpu().numpy().reshape(-1)
    assert np.array_equal(np.sort(pos), np.arange(pos.size))
    sel[15000, 3] = 99
    _check_route(cuda, sel, 100)


@pytest.mark.parametrize("T,K,H", [(1, 1, 8), (37, 3, 1024), (513, 8, 2048), (100, 2, 7168), (31, 2, 13)])
def test_scatter_is_exact_copy(cuda, T, K, H):
    g = torch.Generator().manual_seed(T * 7 + H)
    x = torch.randn((T, H), generator=g).to(torch.bfloat16)
    sel = torch.randint(0, 5, (T, K), generator=g)
    r = kernels.route(sel.to(cuda), 5)
    xp = kernels.moe_scatter(x.to(cuda), r.pos)
    expect = O.permute(x, r.pos.cpu().numpy())
    assert_exact(xp, expect, "Xp")
