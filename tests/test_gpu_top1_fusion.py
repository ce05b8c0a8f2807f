"""Top-1 epilogue fusions: the router-weighted combine inside the fc2 GEMM
and the unpermute gradient inside the fc1 dgrad are bit-identical to the
separate kernels they replace (and a top-1 layer with them to the layer
without them); the combine gradient walked in row order equals the
token-order one; the scatter's row-source map is the inverse of the scatter
index; row targets outside the output are never written."""

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from placemoe_amd import _capi, experts, kernels
from placemoe_amd.workloads import make_workload
from tests.helpers import assert_bf16_close, assert_exact

pytestmark = pytest.mark.gpu

GROUPS = {
    "ragged": [130, 0, 1, 17, 256, 5, 0, 64],
    "big": [1500, 700, 129],
    "tiny": [1, 2, 3, 0, 0, 4],
}


def _offsets(counts, cuda):
    off = np.zeros(len(counts) + 1, dtype=np.int64)
    np.cumsum(counts, out=off[1:])
    return off, torch.as_tensor(off, dtype=torch.int32).to(cuda)


def _perm(A, seed, cuda):
    """pos [A, 1] (token -> row, a random permutation) and its inverse row -> token."""
    g = torch.Generator().manual_seed(seed)
    pos = torch.randperm(A, generator=g).to(torch.int32)
    inv = torch.empty_like(pos)
    inv[pos.long()] = torch.arange(A, dtype=torch.int32)
    return pos.view(A, 1).to(cuda), inv.to(cuda)


@pytest.mark.parametrize("K", [1, 8])
def test_scatter_row_source_inverts_pos(cuda, K):
    T, C, H = 1000, 12, 64
    g = torch.Generator().manual_seed(40 + K)
    sel = torch.stack([torch.randperm(C, generator=g)[:K] for _ in range(T)]).to(torch.int64)
    r = kernels.route(sel.to(cuda), C)
    x = torch.randn((T, H), generator=g).to(torch.bfloat16).to(cuda)
    w = torch.rand((T, K), generator=g).to(torch.bfloat16)
    xp, src, row_w = kernels.moe_scatter_src(x, r.pos, w.to(cuda))
    assert_exact(xp, kernels.moe_scatter(x, r.pos), "rows")
    pos = O.scatter_index(sel.numpy()).ravel()
    expect = np.empty(T * K, dtype=np.int32)
    expect[pos] = np.arange(T * K, dtype=np.int32)
    assert_exact(src, torch.from_numpy(expect), "row sources")
    assert_exact(row_w, w.reshape(-1)[torch.from_numpy(expect).long()], "row weights")
    xp2, src2, none = kernels.moe_scatter_src(x, r.pos)
    assert none is None
    assert_exact(xp2, xp, "rows without weights")
    assert_exact(src2, src, "row sources without weights")


@pytest.mark.parametrize("T,H", [(1000, 64), (777, 7168), (3000, 2048), (5, 8), (4096, 4104)])
def test_top1_permute_in_row_order_matches_token_order(cuda, T, H):
    """With the row map requested, the top-1 permute copies rows in their
    storage order; without it, in token order: the rows must agree."""
    pos, inv = _perm(T, 90 + T, cuda)
    g = torch.Generator(device=cuda).manual_seed(T)
    x = torch.randn((T, H), generator=g, device=cuda).to(torch.bfloat16)
    w = torch.rand((T, 1), generator=g, device=cuda).to(torch.bfloat16)
    print(f"permute row order: T={T} H={H}", flush=True)
    xp_token = kernels.moe_scatter(x, pos)
    xp_row, src, row_w = kernels.moe_scatter_src(x, pos, w)
    assert_exact(xp_row, xp_token, "rows")
    assert_exact(src, inv, "row map")
    assert_exact(row_w, w.reshape(-1)[inv.long()], "row weights")


def test_top1_permute_rows_not_named_by_pos(cuda):
    """A pos that names some rows twice and some not at all (not what
    pmx_route produces, but the entry point takes any pos): the unnamed rows
    get row_src -1 and zeros, whatever the output buffers held before."""
    T, H = 300, 256
    pos, _ = _perm(T, 17, cuda)
    pos[::7] = pos[1::7][: pos[::7].numel()]  # every 7th token lands on its neighbour's row
    pos[5] = T + 3  # outside the rows: skipped
    named = torch.zeros(T, dtype=torch.bool, device=cuda)
    named[pos[(pos >= 0) & (pos < T)].long()] = True
    g = torch.Generator(device=cuda).manual_seed(3)
    x = torch.randn((T, H), generator=g, device=cuda).to(torch.bfloat16)
    w = torch.rand((T, 1), generator=g, device=cuda).to(torch.bfloat16)
    print(f"permute rows not named: T={T} H={H} unnamed={int((~named).sum())}", flush=True)
    for _ in range(2):  # the second call gets recycled (non-zero) buffers from the allocator
        xp, src, _ = kernels.moe_scatter_src(x, pos, w)
        torch.cuda.synchronize()
        assert int((~named).sum()) > 0
        assert (src[~named] == -1).all(), "unnamed rows keep a stale row map entry"
        assert (xp[~named] == 0).all(), "unnamed rows are not zero"
        ok = named.nonzero().flatten()
        assert_exact(xp[ok], x[src[ok].long()], "named rows")
        assert (pos.view(-1)[src[ok].long()] == ok.to(pos.dtype)).all(), "row map does not invert pos"
        del xp, src


@pytest.mark.parametrize("T,H", [(1000, 64), (777, 7168), (3000, 2048), (5, 8), (4096, 4104), (300, 14336)])
def test_combine_bwd_top1_rows_matches_token_order(cuda, T, H):
    pos, inv = _perm(T, 70 + T, cuda)
    g = torch.Generator(device=cuda).manual_seed(H)
    dout = torch.randn((T, H), generator=g, device=cuda).to(torch.bfloat16)
    y = torch.randn((T, H), generator=g, device=cuda).to(torch.bfloat16)
    w = torch.rand((T, 1), generator=g, device=cuda).to(torch.bfloat16)
    print(f"combine gradient row order: T={T} H={H}", flush=True)
    dy, dw = kernels.combine_bwd(dout, y, pos, w)
    dy2, dw2 = kernels.combine_bwd_top1_rows(dout, y, inv, w)
    assert_exact(dy2, dy, "dY")
    assert_exact(dw2, dw, "dw")


def test_combine_bwd_top1_rows_skips_invalid_row_tokens(cuda):
    T, H = 64, 128
    pos, inv = _perm(T, 5, cuda)
    g = torch.Generator(device=cuda).manual_seed(6)
    dout = torch.randn((T, H), generator=g, device=cuda).to(torch.bfloat16)
    y = torch.randn((T, H), generator=g, device=cuda).to(torch.bfloat16)
    w = torch.rand((T, 1), generator=g, device=cuda).to(torch.bfloat16)
    dy_ref, dw_ref = kernels.combine_bwd(dout, y, pos, w)
    bad = inv.clone()
    lost = [int(inv[3]), int(inv[7])]
    bad[3], bad[7] = -1, T
    dy = torch.full((T, H), 7.0, device=cuda, dtype=torch.bfloat16)
    dw = torch.full((T, 1), 9.0, device=cuda, dtype=torch.bfloat16)
    stream = torch.cuda.current_stream().cuda_stream
    _capi.call("pmx_combine_bwd_top1_rows", dout.data_ptr(), y.data_ptr(), bad.data_ptr(), w.data_ptr(), T, H,
               dy.data_ptr(), dw.data_ptr(), stream)
    torch.cuda.synchronize()
    keep = [r for r in range(T) if r not in (3, 7)]
    assert_exact(dy[keep], dy_ref[keep], "dY of valid rows")
    assert torch.count_nonzero(dy[[3, 7]]) == 0, "rows with an invalid token must be zero"
    ok = [t for t in range(T) if t not in lost]
    assert_exact(dw[ok], dw_ref[ok], "dw of tokens with a valid row")
    assert torch.all(dw[lost] == 9.0), "tokens whose row is invalid keep their dw"


@pytest.mark.parametrize("groups", list(GROUPS))
@pytest.mark.parametrize("N,K", [(256, 128), (72, 200)])
def test_nt_combine_top1_matches_separate_kernels(cuda, groups, N, K):
    counts = GROUPS[groups]
    off, doff = _offsets(counts, cuda)
    A, G = int(off[-1]), len(counts)
    g = torch.Generator().manual_seed(A + N + K)
    a = torch.randn((A, K), generator=g).to(torch.bfloat16)
    b = (torch.randn((G, N, K), generator=g) * 0.05).to(torch.bfloat16)
    w = torch.rand((A, 1), generator=g).to(torch.bfloat16)
    pos, inv = _perm(A, A + 1, cuda)
    print(f"nt combine top-1 groups={groups} N={N} K={K}", flush=True)
    a_d, b_d, w_d = a.to(cuda), b.to(cuda), w.to(cuda)
    y_ref = kernels.group_gemm_nt(a_d, b_d, doff)
    out_ref = kernels.combine_fwd(y_ref, pos, w_d)
    y, out = kernels.group_gemm_nt_combine_top1(a_d, b_d, doff, inv, w_d.reshape(-1)[inv.long()].contiguous())
    assert_exact(y, y_ref, "fc2 rows")
    assert_exact(out, out_ref, "combined rows")
    out_oracle = O.combine_forward(O.grouped_gemm_nt(a, b, off), pos.cpu().numpy(), w)
    assert_bf16_close(out, out_oracle, name="combine vs oracle")


@pytest.mark.parametrize("groups", list(GROUPS))
@pytest.mark.parametrize("N,K,split", [(256, 128, False), (200, 72, False), (256, 192, True)])
def test_nn_unpermute_top1_matches_separate_kernels(cuda, groups, N, K, split):
    counts = GROUPS[groups]
    off, doff = _offsets(counts, cuda)
    A, G = int(off[-1]), len(counts)
    g = torch.Generator().manual_seed(A * 5 + N + K)
    a = torch.randn((A, K), generator=g).to(torch.bfloat16).to(cuda)
    b = (torch.randn((G, K, N), generator=g) * 0.05).to(torch.bfloat16).to(cuda)
    b0, b1 = (b[:, : K // 2].contiguous(), b[:, K // 2 :].contiguous()) if split else (b, None)
    pos, inv = _perm(A, A + 2, cuda)
    print(f"nn unpermute top-1 groups={groups} N={N} K={K} split={split}", flush=True)
    dx_ref = kernels.moe_gather(kernels.group_gemm_nn(a, b0, doff, b_second=b1), pos)
    dx = kernels.group_gemm_nn_unpermute_top1(a, b0, doff, inv, b_second=b1)
    assert_exact(dx, dx_ref, "unpermuted rows")


def test_row_targets_outside_the_output_are_not_written(cuda):
    counts = [300, 0, 212]
    off, doff = _offsets(counts, cuda)
    A, G, N, K = int(off[-1]), len(counts), 128, 64
    g = torch.Generator().manual_seed(77)
    a = torch.randn((A, K), generator=g).to(torch.bfloat16).to(cuda)
    b_nt = (torch.randn((G, N, K), generator=g) * 0.05).to(torch.bfloat16).to(cuda)
    b_nn = (torch.randn((G, K, N), generator=g) * 0.05).to(torch.bfloat16).to(cuda)
    w = torch.rand((A,), generator=g).to(torch.bfloat16).to(cuda)
    _, inv = _perm(A, 78, cuda)
    row_w = w[inv.long()].contiguous()
    bad = inv.clone()
    lost = bad[[3, 100, 450]].long().cpu()  # the tokens of three rows whose targets go bad
    bad[3], bad[100], bad[450] = -1, A, 2**31 - 1
    sentinel = torch.full((A, N), 7.0, dtype=torch.bfloat16, device=cuda)
    stream = torch.cuda.current_stream(cuda).cuda_stream
    y = torch.empty((A, N), dtype=torch.bfloat16, device=cuda)
    out = sentinel.clone()
    _capi.call("pmx_group_gemm_nt_combine_top1", a.data_ptr(), b_nt.data_ptr(), doff.data_ptr(), G, A, N, K,
               y.data_ptr(), bad.data_ptr(), row_w.data_ptr(), out.data_ptr(), stream)
    _, out_ok = kernels.group_gemm_nt_combine_top1(a, b_nt, doff, inv, row_w)
    keep = torch.ones(A, dtype=torch.bool)
    keep[lost] = False
    assert_exact(out[keep.to(cuda)], out_ok[keep.to(cuda)], "combined rows with valid targets")
    assert_exact(out[lost.to(cuda)], sentinel[lost.to(cuda)], "rows with bad targets untouched")
    dx = sentinel.clone()
    _capi.call("pmx_group_gemm_nn_unpermute_top1", a.data_ptr(), b_nn.data_ptr(), None, K * N, 0, doff.data_ptr(),
               G, A, N, K, bad.data_ptr(), dx.data_ptr(), stream)
    dx_ok = kernels.group_gemm_nn_unpermute_top1(a, b_nn, doff, inv)
    assert_exact(dx[keep.to(cuda)], dx_ok[keep.to(cuda)], "unpermuted rows with valid targets")
    assert_exact(dx[lost.to(cuda)], sentinel[lost.to(cuda)], "rows with bad targets untouched")
    # the combine takes all three of its arguments or none
    with pytest.raises(ValueError):
        _capi.call("pmx_group_gemm_nt_combine_top1", a.data_ptr(), b_nt.data_ptr(), doff.data_ptr(), G, A, N, K,
                   y.data_ptr(), inv.data_ptr(), None, out.data_ptr(), stream)


def _layer_run(cuda, wl, split):
    x = wl.hidden.to(cuda).requires_grad_(True)
    w = wl.routing_weights.to(cuda).requires_grad_(True)
    fc2 = wl.fc2.to(cuda).requires_grad_(True)
    I = wl.fc2.shape[2]
    src = None if wl.sources is None else wl.sources.to(cuda)
    if split:
        fc1a = wl.fc1[:, :I].contiguous().to(cuda).requires_grad_(True)
        fc1b = wl.fc1[:, I:].contiguous().to(cuda).requires_grad_(True)
        out = experts.expert_layer(x, w, wl.selected.to(cuda), fc2, fc1_1_weight=fc1a, fc1_2_weight=fc1b,
                                   mapping=wl.mapping.to(cuda), sources=src)
        params = (x, w, fc1a, fc1b, fc2)
    else:
        fc1 = wl.fc1.to(cuda).requires_grad_(True)
        out = experts.expert_layer(x, w, wl.selected.to(cuda), fc2, fc1_1_2_weight=fc1,
                                   mapping=wl.mapping.to(cuda), sources=src)
        params = (x, w, fc1, fc2)
    dout = torch.randn(out.shape, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16).to(cuda)
    out.backward(dout)
    torch.cuda.synchronize()
    return out.detach().clone(), [p.grad.clone() for p in params]


@pytest.mark.parametrize("split", [False, True])
def test_top1_layer_fused_equals_separate_kernels(cuda, split):
    wl = make_workload("dsv3", tokens=3000, num_slots=6)
    assert wl.selected.shape[1] == 1
    print(f"top-1 layer fused vs separate, dsv3 shape, 3000 rows, 6 slots, split={split}", flush=True)
    prev = experts.set_top1_fusion(True)
    try:
        out_f, grads_f = _layer_run(cuda, wl, split)
        experts.set_top1_fusion(False)
        out_s, grads_s = _layer_run(cuda, wl, split)
    finally:
        experts.set_top1_fusion(prev)
    assert_exact(out_f, out_s, "layer output")
    for i, (a, b) in enumerate(zip(grads_f, grads_s)):
        assert_exact(a, b, f"gradient {i}")
