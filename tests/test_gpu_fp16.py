"""GPU parity of the fp16 entry points (the *_f16 twins of the float path).

The reference's fused MoE op takes bf16 or fp16 hidden states and router
weights (veomni/ops/kernels/moe/__init__.py:44-49) and rounds in the input
dtype.  Every kernel here is checked against the oracle run on the same fp16
inputs at FP16_REL (a few fp16 ulps; any bf16 rounding left in a kernel
would exceed it), and bit for bit where the arithmetic order is the oracle's
(single products, k-ordered sums, row copies) or where a fused entry point
replaces two unfused ones.  Both GEMM layouts run: K a multiple of 64 takes
the four-wave kernel (fc1 + SwiGLU, fc2 dgrad, weight gradients), other K
the eight-wave kernel."""

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from placemoe_amd import ep_payload as EP
from placemoe_amd import experts, kernels
from placemoe_amd.placement import copy_table
from placemoe_amd.workloads import make_workload
from tests.helpers import FP16_REL, assert_bf16_close, assert_exact

pytestmark = pytest.mark.gpu

F16 = torch.float16
SWIGLU_REL = 1.5 * FP16_REL  # two chained roundings after the GEMM's


def _offsets(counts):
    off = np.zeros(len(counts) + 1, dtype=np.int64)
    np.cumsum(counts, out=off[1:])
    return off


def _dev(off, cuda):
    return torch.as_tensor(off, dtype=torch.int32).to(cuda)


def _close(actual, expected, rel=FP16_REL, name="tensor"):
    assert actual.dtype == F16, f"{name}: dtype {actual.dtype}"
    assert_bf16_close(actual, expected, rel=rel, name=name)


GROUPS = {"ragged": [130, 0, 1, 17, 256, 5, 0, 64], "big": [1500, 700, 129], "tiny": [1, 2, 3, 0, 0, 4]}


@pytest.mark.parametrize("groups", list(GROUPS))
@pytest.mark.parametrize("H,I", [(256, 128), (200, 72)])
def test_fc1_swiglu_f16(cuda, groups, H, I):
    off = _offsets(GROUPS[groups])
    A, G = int(off[-1]), len(GROUPS[groups])
    g = torch.Generator().manual_seed(A + H + I)
    x = torch.randn((A, H), generator=g).to(F16)
    w1 = (torch.randn((G, 2 * I, H), generator=g) * 0.05).to(F16)
    print(f"fp16 fc1 groups={groups} H={H} I={I}", flush=True)
    gu, act = kernels.gemm_fc1_swiglu(x.to(cuda), w1.to(cuda), w1.to(cuda).view(-1)[I * H:], 2 * I * H,
                                      _dev(off, cuda), G, I)
    gu_ref = O.grouped_gemm_nt(x, w1, off)
    _close(gu, gu_ref, name="gate_up")
    _close(act, O.swiglu_forward(gu_ref[:, :I], gu_ref[:, I:]), rel=SWIGLU_REL, name="act")


@pytest.mark.parametrize("groups", list(GROUPS))
@pytest.mark.parametrize("N,K", [(256, 128), (72, 200)])
def test_nt_and_top1_combine_f16(cuda, groups, N, K):
    counts = GROUPS[groups]
    off = _offsets(counts)
    A, G = int(off[-1]), len(counts)
    g = torch.Generator().manual_seed(3 * A + N + K)
    a = torch.randn((A, K), generator=g).to(F16)
    b = (torch.randn((G, N, K), generator=g) * 0.05).to(F16)
    print(f"fp16 nt groups={groups} N={N} K={K}", flush=True)
    c = kernels.group_gemm_nt(a.to(cuda), b.to(cuda), _dev(off, cuda))
    _close(c, O.grouped_gemm_nt(a, b, off), name="nt")
    # top-1 fused combine: bit-identical to the GEMM followed by the combine kernel
    pos = torch.randperm(A, generator=g).to(torch.int32).reshape(A, 1)
    w = torch.rand((A, 1), generator=g).to(F16)
    x = torch.randn((A, K), generator=g).to(F16)
    _, row_tok, row_w = kernels.moe_scatter_src(x.to(cuda), pos.to(cuda), w.to(cuda))
    c1, out = kernels.group_gemm_nt_combine_top1(a.to(cuda), b.to(cuda), _dev(off, cuda), row_tok, row_w)
    assert_exact(c1, c, "nt (fused call)")
    assert_exact(out, kernels.combine_fwd(c, pos.to(cuda), w.to(cuda)), "combine in the fc2 epilogue")


@pytest.mark.parametrize("groups", list(GROUPS))
@pytest.mark.parametrize("N,K,split", [(256, 128, False), (384, 320, True), (72, 208, True)])
def test_nn_and_top1_unpermute_f16(cuda, groups, N, K, split):
    counts = GROUPS[groups]
    off = _offsets(counts)
    A, G = int(off[-1]), len(counts)
    g = torch.Generator().manual_seed(5 * A + N + K)
    a = torch.randn((A, K), generator=g).to(F16)
    b = (torch.randn((G, K, N), generator=g) * 0.05).to(F16)
    b0, b1 = (b[:, :K // 2].contiguous(), b[:, K // 2:].contiguous()) if split else (b, None)
    print(f"fp16 nn groups={groups} N={N} K={K} split={split}", flush=True)
    c = kernels.group_gemm_nn(a.to(cuda), b0.to(cuda), _dev(off, cuda),
                              b_second=None if b1 is None else b1.to(cuda))
    _close(c, O.grouped_gemm_nn(a, b, off), name="nn")
    pos = torch.randperm(A, generator=g).to(torch.int32).reshape(A, 1)
    _, row_tok, _ = kernels.moe_scatter_src(a.to(cuda), pos.to(cuda))
    dx = kernels.group_gemm_nn_unpermute_top1(a.to(cuda), b0.to(cuda), _dev(off, cuda), row_tok,
                                              b_second=None if b1 is None else b1.to(cuda))
    assert_exact(dx, kernels.moe_gather(c, pos.to(cuda)), "unpermute in the fc1-dgrad epilogue")


@pytest.mark.parametrize("groups", list(GROUPS))
@pytest.mark.parametrize("H,I", [(256, 128), (200, 72)])
def test_fc2_dgrad_swiglu_f16(cuda, groups, H, I):
    off = _offsets(GROUPS[groups])
    A, G = int(off[-1]), len(GROUPS[groups])
    g = torch.Generator().manual_seed(7 * A + H + I)
    dy = torch.randn((A, H), generator=g).to(F16)
    w2 = (torch.randn((G, H, I), generator=g) * 0.05).to(F16)
    gu = torch.randn((A, 2 * I), generator=g).to(F16)
    print(f"fp16 fc2 dgrad groups={groups} H={H} I={I}", flush=True)
    dg1 = kernels.gemm_fc2_dgrad_swiglu(dy.to(cuda), w2.to(cuda), gu.to(cuda), _dev(off, cuda))
    d_gate, d_up = O.swiglu_backward(O.grouped_gemm_nn(dy, w2, off), gu[:, :I], gu[:, I:])
    _close(dg1[:, :I], d_gate, rel=SWIGLU_REL, name="d_gate")
    _close(dg1[:, I:], d_up, rel=SWIGLU_REL, name="d_up")


@pytest.mark.parametrize("groups", list(GROUPS))
@pytest.mark.parametrize("M,N,split", [(256, 128, False), (384, 320, True), (72, 200, False)])
def test_tn_wgrad_f16(cuda, groups, M, N, split):
    counts = GROUPS[groups]
    off = _offsets(counts)
    A = int(off[-1])
    g = torch.Generator().manual_seed(11 * A + M + N)
    a = torch.randn((A, M), generator=g).to(F16)
    b = torch.randn((A, N), generator=g).to(F16)
    print(f"fp16 tn groups={groups} M={M} N={N} split={split}", flush=True)
    if split:
        c0, c1 = kernels.group_gemm_tn(a.to(cuda), b.to(cuda), _dev(off, cuda), split=M // 2)
        c = torch.cat([c0, c1], dim=1)
    else:
        c = kernels.group_gemm_tn(a.to(cuda), b.to(cuda), _dev(off, cuda))
    _close(c, O.grouped_gemm_tn(a, b, off), name="tn")
    for gi, cnt in enumerate(counts):
        if cnt == 0:
            assert torch.count_nonzero(c[gi]).item() == 0, "empty group must store zeros"


def test_mfma_lane_layout_identity_f16(cuda):
    # X @ I^T = X exactly, through both layouts' fp16 MFMAs (K = 128: four
    # waves for fc1 kinds; the plain NT kind runs eight waves).
    A, H = 200, 128
    x = torch.randn((A, H)).to(F16)
    eye = torch.eye(H).to(F16).reshape(1, H, H)
    c = kernels.group_gemm_nt(x.to(cuda), eye.to(cuda), _dev(_offsets([A]), cuda))
    assert_exact(c, x, "X @ I^T")
    w1 = torch.cat([eye, eye], dim=1).contiguous().to(cuda)  # gate = up = I
    gu, _ = kernels.gemm_fc1_swiglu(x.to(cuda), w1, w1.view(-1)[H * H:], 2 * H * H, _dev(_offsets([A]), cuda), 1, H)
    assert_exact(gu[:, :H], x, "fc1 gate of X @ I^T")
    assert_exact(gu[:, H:], x, "fc1 up of X @ I^T")


@pytest.mark.parametrize("T,K,H", [(257, 2, 1024), (1024, 8, 2048), (96, 1, 7168), (33, 4, 4096), (19, 3, 33)])
def test_combine_and_gather_f16(cuda, T, K, H):
    g = torch.Generator().manual_seed(T + K + H)
    sel = torch.randint(0, 7, (T, K), generator=g)
    y = torch.randn((T * K, H), generator=g).to(F16)
    w = torch.rand((T, K), generator=g).to(F16)
    dout = torch.randn((T, H), generator=g).to(F16)
    print(f"fp16 combine T={T} K={K} H={H}", flush=True)
    r = kernels.route(sel.to(cuda), 7)
    pos = r.pos.cpu().numpy()
    # k-ordered fp32 sums of single products: the oracle's order, bit for bit
    assert_exact(kernels.combine_fwd(y.to(cuda), r.pos, w.to(cuda)), O.combine_forward(y, pos, w), "combine out")
    assert_exact(kernels.moe_gather(y.to(cuda), r.pos), O.unpermute_grad(y, pos), "gather")
    dy, dw = kernels.combine_bwd(dout.to(cuda), y.to(cuda), r.pos, w.to(cuda))
    dy_ref, dw_ref = O.combine_backward(dout, y, pos, w)
    assert_exact(dy, dy_ref, "combine dy")
    _close(dw, dw_ref, name="combine dw")
    if K == 1 and H % 8 == 0:
        _, row_tok, _ = kernels.moe_scatter_src(dout.to(cuda), r.pos)
        dy1, dw1 = kernels.combine_bwd_top1_rows(dout.to(cuda), y.to(cuda), row_tok, w.to(cuda))
        assert_exact(dy1, dy, "top-1 rows dy")
        assert_exact(dw1, dw, "top-1 rows dw")


def test_segment_sum_f16(cuda):
    g = torch.Generator().manual_seed(20260806)
    source = torch.randn((257, 2048), generator=g).to(F16)
    index = torch.randint(31, (257,), generator=g)
    got = kernels.segment_sum(source.to(cuda), index.to(cuda), 31)
    _close(got, O.segment_sum(source, index.numpy(), 31), name="segment sum")


@pytest.mark.parametrize("R,I", [(512, 768), (129, 100)])
def test_weighted_input_rows_f16(cuda, R, I):
    g = torch.Generator().manual_seed(R + I)
    act = torch.randn((R, I), generator=g).to(F16)
    w = torch.rand((R,), generator=g).to(F16)
    assert_exact(kernels.weight_rows(act.to(cuda), w.to(cuda)), O.weight_rows(act, w), "act_w")
    daw = torch.randn((R, I), generator=g).to(F16)
    gu = (torch.randn((R, 2 * I), generator=g) * 2).to(F16)
    act = O.swiglu_forward(gu[:, :I], gu[:, I:])
    row_src = torch.randperm(R, generator=g).to(torch.int32)
    dg1, dw = kernels.swiglu_bwd_weighted(daw.to(cuda), gu.to(cuda), act.to(cuda), w.to(cuda), row_src.to(cuda), R)
    ref_dg1, ref_row = O.swiglu_backward_weighted(daw, gu, act, w)
    ref_dw = torch.empty(R, dtype=F16)
    ref_dw[row_src.long()] = ref_row
    _close(dg1, ref_dg1, rel=SWIGLU_REL, name="dG1")
    _close(dw, ref_dw, name="dw")


@pytest.mark.parametrize("name,tokens,slots,weighted", [("toy", 256, None, False), ("qwen3", 256, None, False),
                                                        ("dsv3", 512, 4, False), ("skew", 384, None, True)])
def test_layer_f16_matches_oracle(cuda, name, tokens, slots, weighted):
    wl = make_workload(name, tokens=tokens, num_slots=slots)
    x, w = wl.hidden.to(F16), wl.routing_weights.to(F16)
    fc1, fc2 = wl.fc1.to(F16), wl.fc2.to(F16)
    g = torch.Generator().manual_seed(7)
    dout = torch.randn((wl.T, wl.H), generator=g).to(F16)
    src = wl.sources.numpy() if wl.sources is not None else np.zeros(wl.T, dtype=np.int64)
    phys = O.map_logical_to_physical(wl.mapping.numpy(), src, wl.selected.numpy())
    if weighted:
        fwd = O.moe_layer_forward_weighted_input(x, w, phys, fc1, fc2)
        bwd = O.moe_layer_backward_weighted_input(dout, fwd, w, fc1, fc2)
    else:
        fwd = O.moe_layer_forward(x, w, phys, fc1, fc2)
        bwd = O.moe_layer_backward(dout, fwd, w, fc1, fc2)
    print(f"fp16 layer {name}: T={wl.T} K={wl.K} H={wl.H} I={wl.I} C={wl.C} weighted={weighted}", flush=True)
    xd, wd = x.to(cuda).requires_grad_(True), w.to(cuda).requires_grad_(True)
    f1, f2 = fc1.to(cuda).requires_grad_(True), fc2.to(cuda).requires_grad_(True)
    out = experts.expert_layer(xd, wd, wl.selected.to(cuda), f2, fc1_1_2_weight=f1, mapping=wl.mapping.to(cuda),
                               sources=None if wl.sources is None else wl.sources.to(cuda), weighted_input=weighted)
    out.backward(dout.to(cuda))
    rel = 1.5 * FP16_REL  # the layer chains several rounded stages
    _close(out, fwd["out"], rel=rel, name="out")
    _close(xd.grad, bwd["dx"], rel=rel, name="d_hidden")
    _close(wd.grad, bwd["dw"], rel=rel, name="d_routing_weights")
    _close(f1.grad, bwd["dw1"], rel=rel, name="d_gate_up_proj")
    _close(f2.grad, bwd["dw2"], rel=rel, name="d_down_proj")


def test_public_op_f16(cuda):
    import placemoe_amd

    placemoe_amd.apply_veomni_fused_moe_patch("hip")
    wl = make_workload("toy", tokens=64)
    out = placemoe_amd.fused_moe_forward(
        num_experts=wl.C, routing_weights=wl.routing_weights.to(F16).to(cuda),
        selected_experts=wl.selected.to(cuda), hidden_states=wl.hidden.to(F16).to(cuda), fc1_1_weight=None,
        fc1_2_weight=None, fc2_weight=wl.fc2.to(F16).to(cuda), fc1_1_2_weight=wl.fc1.to(F16).to(cuda),
    )
    fwd = O.moe_layer_forward_weighted_input(wl.hidden.to(F16), wl.routing_weights.to(F16), wl.selected.numpy(),
                                             wl.fc1.to(F16), wl.fc2.to(F16))
    _close(out, fwd["out"], rel=1.5 * FP16_REL, name="fused_moe_forward fp16")


def test_dsv3_shape_gemms_f16(cuda):
    # The DeepSeek-V3 share's weight shapes (H 7168, I 2048, 16 copies) over
    # 2048 rows: every kind at full width and depth, in both layouts' fp16 paths.
    H, I, G = 7168, 2048, 16
    counts = np.random.default_rng(3).multinomial(2048, np.full(G, 1.0 / G))
    off = _offsets(counts)
    A = int(off[-1])
    g = torch.Generator().manual_seed(31)
    x = torch.randn((A, H), generator=g).to(F16)
    w1 = (torch.randn((G, 2 * I, H), generator=g) * 0.006).to(F16)
    w2 = (torch.randn((G, H, I), generator=g) * 0.006).to(F16)
    dy = torch.randn((A, H), generator=g).to(F16)
    o = _dev(off, cuda)
    print(f"fp16 dsv3-shape GEMMs A={A}", flush=True)
    gu, act = kernels.gemm_fc1_swiglu(x.to(cuda), w1.to(cuda), w1.to(cuda).view(-1)[I * H:], 2 * I * H, o, G, I)
    gu_ref = O.grouped_gemm_nt(x, w1, off)
    act_ref = O.swiglu_forward(gu_ref[:, :I], gu_ref[:, I:])
    _close(gu, gu_ref, name="gu")
    _close(act, act_ref, rel=SWIGLU_REL, name="act")
    _close(kernels.group_gemm_nt(act_ref.to(cuda), w2.to(cuda), o), O.grouped_gemm_nt(act_ref, w2, off), name="fc2")
    dg1 = kernels.gemm_fc2_dgrad_swiglu(dy.to(cuda), w2.to(cuda), gu_ref.to(cuda), o)
    d_gate, d_up = O.swiglu_backward(O.grouped_gemm_nn(dy, w2, off), gu_ref[:, :I], gu_ref[:, I:])
    dg1_ref = torch.cat([d_gate, d_up], dim=1)
    _close(dg1, dg1_ref, rel=SWIGLU_REL, name="dG1")
    _close(kernels.group_gemm_nn(dg1_ref.to(cuda), w1.to(cuda), o), O.grouped_gemm_nn(dg1_ref, w1, off),
           name="fc1 dgrad")
    _close(kernels.group_gemm_tn(dy.to(cuda), act_ref.to(cuda), o), O.grouped_gemm_tn(dy, act_ref, off),
           name="fc2 wgrad")
    _close(kernels.group_gemm_tn(dg1_ref.to(cuda), x.to(cuda), o), O.grouped_gemm_tn(dg1_ref, x, off),
           name="fc1 wgrad")


def test_replica_fold_f16(cuda):
    # (the exchange's fp16 type runs in tests/test_gpu_replica_exchange.py)
    g = torch.Generator().manual_seed(12)
    C, E, P = 12, 8, 1000
    L = np.array([0, 1, 2, 3, 4, 5, 6, 7, 0, 1, 2, 3])
    grads = torch.randn((C, P), generator=g).to(F16)
    offs, slots = copy_table(L, E)
    offs_d = torch.as_tensor(offs, dtype=torch.int32).to(cuda)
    slots_d = torch.as_tensor(slots, dtype=torch.int32).to(cuda)
    gd = grads.to(cuda)
    out = kernels.replica_fold(gd, offs_d, slots_d, E, writeback=True)
    ref = O.replica_fold(grads, L, E)
    torch.testing.assert_close(out.cpu(), ref, rtol=1e-5, atol=1e-5)
    for c in range(C):
        assert_exact(gd[c], ref[L[c]].to(F16), f"copy {c} write-back")


def test_ep_combine_aggregate_f16(cuda):
    g = torch.Generator().manual_seed(2)
    N, H, R = 500, 64, 4
    splits = torch.multinomial(torch.ones(R), N, replacement=True, generator=g).bincount(minlength=R).tolist()
    tokens = np.concatenate([np.sort(torch.randint(0, max(1, n // 2), (n,), generator=g).numpy()) for n in splits])
    y = torch.randn(N, H, generator=g).to(F16)
    pos = torch.randperm(N, generator=g)
    w = torch.rand(N, generator=g).to(F16)
    ranks = torch.repeat_interleave(torch.arange(R), torch.as_tensor(splits))
    got, gsplits = EP.combine_aggregate(y.to(cuda), pos.to(cuda), w.to(cuda), ranks.to(cuda),
                                        torch.as_tensor(tokens).to(cuda), R)
    weighted = (y[pos].float() * w.float()[:, None]).to(F16)
    ref, rsplits = O.aggregate_weighted_outputs(weighted, tokens, splits)
    assert gsplits == rsplits
    _close(got.cpu(), ref, name="EP combine")
