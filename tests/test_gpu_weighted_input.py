"""The reference's non-EP arithmetic on the GPU: the router weight applied to
the fc2 input (veomni/ops/kernels/moe/group_gemm.py:458-629), through the C ABI.

* ``pmx_weight_rows`` equals the oracle's bf16 product bit for bit (one fp32
  product, rounded once); the scalar path (widths off 16 bytes) too.
* ``pmx_swiglu_bwd_weighted`` against the oracle within the bf16 bar (its
  sigmoid differs from torch's by a few fp32 ulp before the bf16 rounding,
  and the row sums run in another order); dw entries that no row names keep
  what they held.
* The layer with ``weighted_input=True`` against the oracle's non-EP layer,
  forward and every gradient, within the bf16 bar.
* With power-of-two router weights the two branches must agree bit for bit
  (every product with a weight is exact): output and fc2 weight gradient with
  the shipped library; with the eight-wave test build, whose fc2 dgrad with
  the SwiGLU epilogue and plain fc2 dgrad share one main loop, also dx, the
  fc1 weight gradient and the copy gradients.
* The public op takes the non-EP arithmetic without a placement, and the EP
  arithmetic with ``set_router_weight_point("combine")``.
"""

import numpy as np
import pytest
import torch

import placemoe_amd
from oracle import moe_oracle as O
from placemoe_amd import _capi, build, experts, kernels
from placemoe_amd.workloads import make_workload
from tests.helpers import assert_bf16_close, assert_exact

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


@pytest.mark.parametrize("R,N,offset", [(1000, 768, 0), (37, 8, 0), (300, 100, 0), (64, 256, 1), (1, 1, 0)])
def test_weight_rows_bitwise(cuda, R, N, offset):
    g = torch.Generator().manual_seed(R + N)
    act = torch.randn((R * N + offset,), generator=g).to(BF)
    w = torch.rand((R,), generator=g).to(BF)
    print(f"weight_rows R={R} N={N} offset={offset}", flush=True)
    a_dev = act.to(cuda)[offset:].view(R, N)  # offset 1: not 16-byte aligned (scalar path)
    got = kernels.weight_rows(a_dev, w.to(cuda))
    assert_exact(got, O.weight_rows(act[offset:].view(R, N), w), "act_w")


@pytest.mark.parametrize("R,I", [(512, 768), (300, 96), (129, 100), (64, 8), (5, 1024)])
def test_swiglu_bwd_weighted_matches_oracle(cuda, R, I):
    g = torch.Generator().manual_seed(R * 7 + I)
    daw = torch.randn((R, I), generator=g).to(BF)
    gu = (torch.randn((R, 2 * I), generator=g) * 2).to(BF)
    act = O.swiglu_forward(gu[:, :I], gu[:, I:])
    w = torch.rand((R,), generator=g).to(BF)
    row_src = torch.randperm(R, generator=g).to(torch.int32)
    print(f"swiglu_bwd_weighted R={R} I={I}", flush=True)
    dg1, dw = kernels.swiglu_bwd_weighted(daw.to(cuda), gu.to(cuda), act.to(cuda), w.to(cuda), row_src.to(cuda), R)
    ref_dg1, ref_row = O.swiglu_backward_weighted(daw, gu, act, w)
    ref_dw = torch.empty(R, dtype=BF)
    ref_dw[row_src.long()] = ref_row
    assert_bf16_close(dg1[:, :I], ref_dg1[:, :I], name="d_gate")
    assert_bf16_close(dg1[:, I:], ref_dg1[:, I:], name="d_up")
    assert_bf16_close(dw, ref_dw, name="dw")


def test_swiglu_bwd_weighted_skips_unnamed_dw(cuda):
    R, I, A = 64, 128, 100
    g = torch.Generator(device=cuda).manual_seed(3)
    daw, act = (torch.randn((R, I), generator=g, device=cuda).to(BF) for _ in range(2))
    gu = torch.randn((R, 2 * I), generator=g, device=cuda).to(BF)
    w = torch.rand((R,), generator=g, device=cuda).to(BF)
    row_src = torch.arange(R, dtype=torch.int32, device=cuda) * 2 - 3  # -3, -1, 1, ... 125: some outside [0, A)
    dg1 = torch.empty((R, 2 * I), dtype=BF, device=cuda)
    dw = torch.full((A,), 7.0, dtype=BF, device=cuda)
    _capi.call("pmx_swiglu_bwd_weighted", daw.data_ptr(), gu.data_ptr(), act.data_ptr(), w.data_ptr(),
               row_src.data_ptr(), R, I, A, dg1.data_ptr(), dw.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    named = [int(k) for k in row_src.cpu() if 0 <= k < A]
    untouched = sorted(set(range(A)) - set(named))
    assert (dw.cpu()[untouched] == 7.0).all(), "a dw entry no row names was written"
    ref_dg1, ref_row = O.swiglu_backward_weighted(daw.cpu(), gu.cpu(), act.cpu(), w.cpu())
    ok = [r for r in range(R) if 0 <= int(row_src[r]) < A]
    assert_bf16_close(dw.cpu()[[int(row_src[r]) for r in ok]], ref_row[ok], name="named dw")
    assert_bf16_close(dg1.cpu(), ref_dg1, name="dG1")


def _layer(cuda, wl, w, dout, weighted_input, split=False):
    x = wl.hidden.to(cuda).requires_grad_(True)
    wd = w.to(cuda).requires_grad_(True)
    fc2 = wl.fc2.to(cuda).requires_grad_(True)
    kw = {}
    if split:
        I = wl.I
        a = wl.fc1[:, :I].contiguous().to(cuda).requires_grad_(True)
        b = wl.fc1[:, I:].contiguous().to(cuda).requires_grad_(True)
        kw = dict(fc1_1_weight=a, fc1_2_weight=b)
    else:
        fc1 = wl.fc1.to(cuda).requires_grad_(True)
        kw = dict(fc1_1_2_weight=fc1)
    out = experts.expert_layer(x, wd, wl.selected.to(cuda), fc2, mapping=wl.mapping.to(cuda),
                               sources=None if wl.sources is None else wl.sources.to(cuda),
                               weighted_input=weighted_input, **kw)
    out.backward(dout.to(cuda))
    d_fc1 = torch.cat([kw["fc1_1_weight"].grad, kw["fc1_2_weight"].grad], 1) if split else kw["fc1_1_2_weight"].grad
    experts.check_pending_routes(block=True)
    return dict(out=out.detach(), dx=x.grad, dw=wd.grad, dw1=d_fc1, dw2=fc2.grad)


@pytest.mark.parametrize("name,tokens,split", [("qwen3", 256, False), ("skew", 384, True), ("dsv3", 512, False)])
def test_weighted_input_layer_matches_oracle(cuda, name, tokens, split):
    wl = make_workload(name, tokens=tokens, num_slots=4 if name == "dsv3" else None)
    print(f"non-EP layer {name}: T={wl.T} K={wl.K} H={wl.H} I={wl.I} C={wl.C} split={split}", flush=True)
    g = torch.Generator().manual_seed(9)
    dout = torch.randn((wl.T, wl.H), generator=g).to(BF)
    src = wl.sources.numpy() if wl.sources is not None else np.zeros(wl.T, dtype=np.int64)
    phys = O.map_logical_to_physical(wl.mapping.numpy(), src, wl.selected.numpy())
    fwd = O.moe_layer_forward_weighted_input(wl.hidden, wl.routing_weights, phys, wl.fc1, wl.fc2)
    bwd = O.moe_layer_backward_weighted_input(dout, fwd, wl.routing_weights, wl.fc1, wl.fc2)
    got = _layer(cuda, wl, wl.routing_weights, dout, True, split=split)
    assert_bf16_close(got["out"], fwd["out"], name="out")
    for k in ("dx", "dw", "dw1", "dw2"):
        assert_bf16_close(got[k], bwd[k], name=k)


def _pow2_weights(wl, seed):
    j = np.random.default_rng(seed).integers(0, 6, size=tuple(wl.routing_weights.shape))
    return torch.pow(2.0, -torch.as_tensor(j, dtype=torch.float64)).to(BF)


@pytest.mark.parametrize("name,tokens", [("qwen3", 256), ("dsv3", 512)])
def test_power_of_two_weights_branches_agree(cuda, name, tokens):
    wl = make_workload(name, tokens=tokens, num_slots=4 if name == "dsv3" else None)
    w = _pow2_weights(wl, 5)
    dout = torch.randn((wl.T, wl.H), generator=torch.Generator().manual_seed(4)).to(BF)
    print(f"power-of-two weights {name}: T={wl.T} K={wl.K}", flush=True)
    ep = _layer(cuda, wl, w, dout, False)
    ni = _layer(cuda, wl, w, dout, True)
    assert torch.equal(ep["out"], ni["out"]), "outputs differ"
    assert torch.equal(ep["dw2"], ni["dw2"]), "fc2 weight gradients differ"
    for k in ("dx", "dw1"):
        assert_bf16_close(ni[k], ep[k], name=k)
    assert_bf16_close(ni["dw"], ep["dw"], name="dw")
    variant = build.variant_path("w8")
    assert variant.exists(), f"{variant} is not built (python -m placemoe_amd.build)"
    with _capi.using(variant):
        ep8 = _layer(cuda, wl, w, dout, False)
        ni8 = _layer(cuda, wl, w, dout, True)
    for k in ("out", "dx", "dw1", "dw2"):
        assert torch.equal(ep8[k], ni8[k]), f"eight-wave build: {k} differs between the branches"


def test_public_op_router_weight_point(cuda):
    placemoe_amd.apply_veomni_fused_moe_patch("hip")
    wl = make_workload("toy", tokens=64)
    args = dict(num_experts=wl.C, routing_weights=wl.routing_weights.to(cuda), selected_experts=wl.selected.to(cuda),
                hidden_states=wl.hidden.to(cuda), fc1_1_weight=None, fc1_2_weight=None, fc2_weight=wl.fc2.to(cuda),
                fc1_1_2_weight=wl.fc1.to(cuda))
    phys = wl.selected.numpy()  # no placement: slot == expert id
    non_ep = O.moe_layer_forward_weighted_input(wl.hidden, wl.routing_weights, phys, wl.fc1, wl.fc2)["out"]
    ep = O.moe_layer_forward(wl.hidden, wl.routing_weights, phys, wl.fc1, wl.fc2)["out"]
    assert_bf16_close(placemoe_amd.fused_moe_forward(**args), non_ep, name="auto, no placement")
    prev = placemoe_amd.set_router_weight_point("combine")
    try:
        assert_bf16_close(placemoe_amd.fused_moe_forward(**args), ep, name="combine")
        placemoe_amd.set_router_weight_point("fc2_input")
        assert_bf16_close(placemoe_amd.fused_moe_forward(**args), non_ep, name="fc2_input")
    finally:
        placemoe_amd.set_router_weight_point(prev)
    with pytest.raises(ValueError, match="router weight point"):
        placemoe_amd.set_router_weight_point("after_fc1")
