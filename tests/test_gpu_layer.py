"""End-to-end GPU parity of the expert layer (forward and backward) through the
reference's op boundary, against the CPU oracle, at each configuration's
layer shape with a CPU-sized token count."""

import numpy as np
import pytest
import torch

import placemoe_amd
from oracle import moe_oracle as O
from placemoe_amd import experts, kernels
from placemoe_amd.dispatch import OpSlot
from placemoe_amd.placement import PLACEMENTS, LayerPlacement, LayerPlan
from placemoe_amd.workloads import make_workload
from tests.helpers import assert_bf16_close, assert_exact

pytestmark = pytest.mark.gpu

# (config, tokens, dsv3 slots, run backward)
CASES = [("toy", 256, None, False), ("qwen3", 256, None, True), ("dsv3", 512, 4, True), ("skew", 384, None, True),
         ("fold", 192, None, True)]


def _oracle_layer(wl, dout):
    src = wl.sources.numpy() if wl.sources is not None else np.zeros(wl.T, dtype=np.int64)
    phys = O.map_logical_to_physical(wl.mapping.numpy(), src, wl.selected.numpy())
    fwd = O.moe_layer_forward(wl.hidden, wl.routing_weights, phys, wl.fc1, wl.fc2)
    bwd = O.moe_layer_backward(dout, fwd, wl.routing_weights, wl.fc1, wl.fc2) if dout is not None else None
    return fwd, bwd


@pytest.mark.parametrize("name,tokens,slots,backward", CASES)
def test_layer_forward_backward_matches_oracle(cuda, name, tokens, slots, backward):
    wl = make_workload(name, tokens=tokens, num_slots=slots)
    print(f"layer {name}: T={wl.T} K={wl.K} H={wl.H} I={wl.I} C={wl.C}", flush=True)
    g = torch.Generator().manual_seed(7)
    dout = torch.randn((wl.T, wl.H), generator=g).to(torch.bfloat16) if backward else None
    fwd, bwd = _oracle_layer(wl, dout)

    x = wl.hidden.to(cuda).requires_grad_(backward)
    w = wl.routing_weights.to(cuda).requires_grad_(backward)
    fc1 = wl.fc1.to(cuda).requires_grad_(backward)
    fc2 = wl.fc2.to(cuda).requires_grad_(backward)
    out = experts.expert_layer(
        x, w, wl.selected.to(cuda), fc2, fc1_1_2_weight=fc1, mapping=wl.mapping.to(cuda),
        sources=None if wl.sources is None else wl.sources.to(cuda),
    )
    assert_bf16_close(out, fwd["out"], name="out")
    if backward:
        out.backward(dout.to(cuda))
        assert_bf16_close(x.grad, bwd["dx"], name="d_hidden")
        assert_bf16_close(w.grad, bwd["dw"], name="d_routing_weights")
        assert_bf16_close(fc1.grad, bwd["dw1"], name="d_gate_up_proj")
        assert_bf16_close(fc2.grad, bwd["dw2"], name="d_down_proj")


def test_split_and_merged_fc1_are_bitwise_identical(cuda):
    # tests/ops/test_fused_moe_split_vs_merged.py:143-152: split vs merged
    # forward, fc1 and fc2 weight gradients bitwise identical.
    wl = make_workload("qwen3", tokens=128)
    I = wl.I
    dout = torch.randn((wl.T, wl.H), generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).to(cuda)
    common = dict(mapping=wl.mapping.to(cuda), sources=wl.sources.to(cuda))
    x1 = wl.hidden.to(cuda).requires_grad_(True)
    fc1 = wl.fc1.to(cuda).requires_grad_(True)
    fc2a = wl.fc2.to(cuda).requires_grad_(True)
    out_m = experts.expert_layer(x1, wl.routing_weights.to(cuda), wl.selected.to(cuda), fc2a, fc1_1_2_weight=fc1,
                                 **common)
    out_m.backward(dout)
    x2 = wl.hidden.to(cuda).requires_grad_(True)
    g_w = wl.fc1[:, :I].contiguous().to(cuda).requires_grad_(True)
    u_w = wl.fc1[:, I:].contiguous().to(cuda).requires_grad_(True)
    fc2b = wl.fc2.to(cuda).requires_grad_(True)
    out_s = experts.expert_layer(x2, wl.routing_weights.to(cuda), wl.selected.to(cuda), fc2b, fc1_1_weight=g_w,
                                 fc1_2_weight=u_w, **common)
    out_s.backward(dout)
    assert_exact(out_s, out_m, "forward")
    assert_exact(fc2b.grad, fc2a.grad, "fc2 grad")
    assert_exact(torch.cat([g_w.grad, u_w.grad], dim=1), fc1.grad, "fc1 grad")
    assert_exact(x2.grad, x1.grad, "hidden grad")


class _Experts(torch.nn.Module):
    def __init__(self, num_experts, fc1, fc2):
        super().__init__()
        self.num_experts = num_experts
        self.gate_up_proj = torch.nn.Parameter(fc1)
        self.down_proj = torch.nn.Parameter(fc2)


def test_opslot_adapter_with_registered_placement_and_fold(cuda):
    wl = make_workload("fold", tokens=96)
    module = _Experts(wl.num_experts, wl.fc1.to(cuda), wl.fc2.to(cuda))
    plan = LayerPlan(slot_to_logical=wl.slot_to_logical, source_logical_to_physical=wl.mapping.numpy(),
                     owner_slots=wl.owner_slots())
    placement = LayerPlacement.from_plan("layers.0.mlp.experts", plan, wl.num_experts)
    placement.token_sources = wl.sources.to(cuda)
    PLACEMENTS.register(placement, module.gate_up_proj, module.down_proj)
    try:
        slot = OpSlot("moe_experts", "standard")
        slot.bind("hip")
        assert slot.use_non_eager_impl
        x = wl.hidden.to(cuda)
        out = slot(module, x, wl.selected.to(cuda), wl.routing_weights.float().to(cuda))
        fwd, _ = _oracle_layer(wl, None)
        assert_bf16_close(out, fwd["out"], name="opslot out")
        out.float().square().sum().backward()
        counts = placement.accumulated_slot_tokens.cpu().numpy()
        assert_exact(counts, fwd["counts"], "recorded slot tokens")
        grads = {k: p.grad.clone() for k, p in (("gate_up", module.gate_up_proj), ("down", module.down_proj))}
        folded = placemoe_amd.sync_redundant_gradients({"layers.0.mlp.experts": module})
        ref_gu = O.replica_fold(grads["gate_up"].cpu(), wl.slot_to_logical, wl.num_experts, counts)
        ref_dn = O.replica_fold(grads["down"].cpu(), wl.slot_to_logical, wl.num_experts, counts)
        gu, dn = folded["layers.0.mlp.experts"]
        torch.testing.assert_close(gu.cpu(), ref_gu, rtol=0, atol=1e-5 * ref_gu.abs().max().item())
        torch.testing.assert_close(dn.cpu(), ref_dn, rtol=0, atol=1e-5 * ref_dn.abs().max().item())
        # write-back: every copy now holds bf16(total of its expert)
        L = wl.slot_to_logical
        for c in range(len(L)):
            assert_exact(module.down_proj.grad[c], ref_dn[L[c]].to(torch.bfloat16), f"copy {c} write-back")
    finally:
        PLACEMENTS.clear()


def test_fused_moe_forward_public_op(cuda):
    placemoe_amd.apply_veomni_fused_moe_patch("hip")
    wl = make_workload("toy", tokens=64)
    out = placemoe_amd.fused_moe_forward(
        num_experts=wl.C, routing_weights=wl.routing_weights.to(cuda), selected_experts=wl.selected.to(cuda),
        hidden_states=wl.hidden.to(cuda), fc1_1_weight=None, fc1_2_weight=None, fc2_weight=wl.fc2.to(cuda),
        fc1_1_2_weight=wl.fc1.to(cuda),
    )
    phys = wl.selected.numpy()  # no placement registered: slot == expert id, the non-EP arithmetic
    fwd = O.moe_layer_forward_weighted_input(wl.hidden, wl.routing_weights, phys, wl.fc1, wl.fc2)
    assert_bf16_close(out, fwd["out"], name="fused_moe_forward")


def _eager_moe(num_experts, routing_weights, selected_experts, hidden, fc1_1, fc1_2, fc2):
    """The reference test's per-expert loop (tests/ops/test_fused_moe_split_vs_merged.py:21-44),
    run on the CPU in float32 (a reference for bf16 results)."""
    out = torch.zeros_like(hidden)
    mask = torch.nn.functional.one_hot(selected_experts, num_classes=num_experts).permute(2, 1, 0)
    for e in torch.greater(mask.sum(dim=(-1, -2)), 0).nonzero():
        idx = int(e[0])
        top_k_pos, token_idx = torch.where(mask[idx])
        x = hidden[token_idx]
        gate = torch.nn.functional.linear(x, fc1_1[idx])
        up = torch.nn.functional.linear(x, fc1_2[idx])
        y = torch.nn.functional.linear(torch.nn.functional.silu(gate) * up, fc2[idx])
        out.index_add_(0, token_idx, y * routing_weights[token_idx, top_k_pos, None])
    return out


@pytest.mark.parametrize("num_tokens,num_experts,hidden_dim,ffn_dim,topk,seed", [
    (512, 128, 2048, 768, 8, 0),    # Qwen3-30B-A3B
    (256, 64, 2048, 1408, 6, 1),    # Moonlight-16B-A3B
])
def test_reference_split_vs_merged_shapes(cuda, num_tokens, num_experts, hidden_dim, ffn_dim, topk, seed):
    # tests/ops/test_fused_moe_split_vs_merged.py:45-161: the same inputs and
    # checks, through the public op with the hip backend bound.
    placemoe_amd.apply_veomni_fused_moe_patch("hip")
    print(f"reference shape T={num_tokens} E={num_experts} H={hidden_dim} I={ffn_dim} k={topk}", flush=True)
    torch.manual_seed(seed)
    bf = torch.bfloat16
    hidden = 0.1 * torch.randn(num_tokens, hidden_dim, dtype=bf)
    logits = torch.randn(num_tokens, num_experts, dtype=torch.float32)
    routing_weights, selected = torch.topk(torch.softmax(logits, dim=-1), topk, dim=-1)
    routing_weights = routing_weights.to(bf)
    fc1_1 = 0.1 * torch.randn(num_experts, ffn_dim, hidden_dim, dtype=bf)
    fc1_2 = 0.1 * torch.randn(num_experts, ffn_dim, hidden_dim, dtype=bf)
    fc1_12 = torch.cat([fc1_1, fc1_2], dim=1).contiguous()
    fc2 = 0.1 * torch.randn(num_experts, hidden_dim, ffn_dim, dtype=bf)

    def run(split):
        hs = hidden.to(cuda).requires_grad_(True)
        w2 = fc2.to(cuda).requires_grad_(True)
        if split:
            a, b = fc1_1.to(cuda).requires_grad_(True), fc1_2.to(cuda).requires_grad_(True)
            out = placemoe_amd.fused_moe_forward(num_experts=num_experts, routing_weights=routing_weights.to(cuda),
                                                 selected_experts=selected.to(cuda), hidden_states=hs,
                                                 fc1_1_weight=a, fc1_2_weight=b, fc2_weight=w2)
            out.sum().backward()
            return out, hs.grad, w2.grad, torch.cat([a.grad, b.grad], dim=1)
        w1 = fc1_12.to(cuda).requires_grad_(True)
        out = placemoe_amd.fused_moe_forward(num_experts=num_experts, routing_weights=routing_weights.to(cuda),
                                             selected_experts=selected.to(cuda), hidden_states=hs,
                                             fc1_1_weight=None, fc1_2_weight=None, fc2_weight=w2,
                                             fc1_1_2_weight=w1)
        out.sum().backward()
        return out, hs.grad, w2.grad, w1.grad

    out_s, dh_s, dw2_s, dw1_s = (t.cpu() for t in run(True))
    out_m, dh_m, dw2_m, dw1_m = (t.cpu() for t in run(False))
    torch.testing.assert_close(out_s, out_m, rtol=0, atol=0)
    torch.testing.assert_close(dh_s, dh_m, rtol=3e-2, atol=3e-2)
    torch.testing.assert_close(dw2_s, dw2_m, rtol=0, atol=0)
    torch.testing.assert_close(dw1_s, dw1_m, rtol=0, atol=0)

    he = hidden.float().requires_grad_(True)
    e1 = fc1_1.float().requires_grad_(True)
    e2 = fc1_2.float().requires_grad_(True)
    e3 = fc2.float().requires_grad_(True)
    out_e = _eager_moe(num_experts, routing_weights.float(), selected, he, e1, e2, e3)
    out_e.sum().backward()
    torch.testing.assert_close(out_m.float(), out_e.detach(), rtol=1e-2, atol=1e-2)
    torch.testing.assert_close(dh_m.float(), he.grad, rtol=5e-2, atol=5e-2)
    torch.testing.assert_close(dw2_m.float(), e3.grad, rtol=1e-2, atol=1e-2)
    torch.testing.assert_close(dw1_m.float(), torch.cat([e1.grad, e2.grad], dim=1), rtol=3e-2, atol=3e-2)


def test_layer_with_no_tokens(cuda):
    # An empty micro-batch: every kernel returns early; gradients are empty or zero.
    wl = make_workload("qwen3", tokens=16)
    H = wl.H
    x = torch.zeros((0, H), dtype=torch.bfloat16, device=cuda, requires_grad=True)
    w = torch.zeros((0, wl.K), dtype=torch.bfloat16, device=cuda, requires_grad=True)
    sel = torch.zeros((0, wl.K), dtype=torch.int64, device=cuda)
    fc1 = wl.fc1.to(cuda).requires_grad_(True)
    fc2 = wl.fc2.to(cuda).requires_grad_(True)
    out = experts.expert_layer(x, w, sel, fc2, fc1_1_2_weight=fc1, mapping=wl.mapping.to(cuda),
                               sources=torch.zeros(0, dtype=torch.int64, device=cuda))
    assert out.shape == (0, H)
    out.backward(torch.zeros_like(out))
    assert x.grad.shape == (0, H) and w.grad.shape == (0, wl.K)
    assert torch.count_nonzero(fc1.grad).item() == 0 and torch.count_nonzero(fc2.grad).item() == 0


@pytest.mark.parametrize("name,tokens,slots,weighted_input", [
    ("qwen3", 512, None, False), ("dsv3", 1024, 4, False), ("qwen3", 512, None, True), ("dsv3", 1024, 4, True)])
def test_backward_on_one_or_two_streams_is_bitwise_identical(cuda, name, tokens, slots, weighted_input):
    wl = make_workload(name, tokens=tokens, num_slots=slots)
    print(f"backward streams {name}: T={wl.T} K={wl.K} C={wl.C} weighted_input={weighted_input}", flush=True)
    dout = torch.randn((wl.T, wl.H), generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).to(cuda)
    src = None if wl.sources is None else wl.sources.to(cuda)
    results = []
    prev = experts.set_backward_overlap(None)
    try:
        for overlap in (True, False):
            experts.set_backward_overlap(overlap)
            x = wl.hidden.to(cuda).requires_grad_(True)
            w = wl.routing_weights.to(cuda).requires_grad_(True)
            fc1 = wl.fc1.to(cuda).requires_grad_(True)
            fc2 = wl.fc2.to(cuda).requires_grad_(True)
            out = experts.expert_layer(x, w, wl.selected.to(cuda), fc2, fc1_1_2_weight=fc1,
                                       mapping=wl.mapping.to(cuda), sources=src, weighted_input=weighted_input)
            out.backward(dout)
            torch.cuda.synchronize()
            results.append([t.clone() for t in (x.grad, w.grad, fc1.grad, fc2.grad)])
    finally:
        experts.set_backward_overlap(prev)
    for a, b, n in zip(results[0], results[1], ("d_hidden", "d_weights", "d_gate_up", "d_down")):
        assert_exact(a, b, f"{n}: two streams vs one")
