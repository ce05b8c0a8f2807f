"""The fused MoE op adds no host synchronisation, the gate the reference runs
its fused forward under (tests/models/test_model_forward_no_implicit_sync.py:
129-133, 665-677, with torch's sync debug mode).

Two checks at the Qwen3-30B-A3B layer shape (512 tokens, 128 experts on 160
copies, source-aware M, top-8; and without a placement, 128 experts, where the
op takes the non-EP arithmetic), forward and backward through the public op:
  - torch's sync debug mode set to "error" raises on any synchronising torch
    call inside the op;
  - behind a bounded spin kernel queued first on the stream, the host
    finishes enqueueing the whole forward and backward while that kernel still
    runs, so no call of the op (torch or HIP) waited for the GPU.
"""

import time

import pytest
import torch

import placemoe_amd
from placemoe_amd import experts
from placemoe_amd.placement import PLACEMENTS, LayerPlacement, LayerPlan
from placemoe_amd.workloads import make_workload

pytestmark = pytest.mark.gpu

KEY = "layers.0.mlp.experts"


class _Case:
    def __init__(self, cuda, placed):
        placemoe_amd.apply_veomni_fused_moe_patch("hip")
        wl = make_workload("qwen3", tokens=512)
        self.placement = None
        self.E = wl.num_experts
        self.x = wl.hidden.to(cuda)
        self.w = wl.routing_weights.to(cuda)
        self.sel = wl.selected.to(cuda)
        if placed:
            plan = LayerPlan(slot_to_logical=wl.slot_to_logical, source_logical_to_physical=wl.mapping.numpy(),
                             owner_slots=wl.owner_slots())
            self.placement = LayerPlacement.from_plan(KEY, plan, wl.num_experts)
            self.placement.token_sources = wl.sources.to(cuda)
            self.fc1 = wl.fc1.to(cuda)
            self.fc2 = wl.fc2.to(cuda)
        else:
            # one copy per logical expert: slot == expert id
            first = [list(wl.slot_to_logical).index(e) for e in range(wl.num_experts)]
            self.fc1 = wl.fc1[first].contiguous().to(cuda)
            self.fc2 = wl.fc2[first].contiguous().to(cuda)
        g = torch.Generator(device=cuda).manual_seed(5)
        self.dout = torch.randn(self.x.shape, generator=g, device=cuda).to(torch.bfloat16)

    def step(self):
        """One forward + backward; returns the four gradients."""
        x = self.x.detach().requires_grad_(True)
        w = self.w.detach().requires_grad_(True)
        fc1 = self.fc1.detach().requires_grad_(True)
        fc2 = self.fc2.detach().requires_grad_(True)
        if self.placement is not None:
            PLACEMENTS.register(self.placement, fc1, fc2)
        out = placemoe_amd.fused_moe_forward(
            num_experts=self.E, routing_weights=w, selected_experts=self.sel, hidden_states=x,
            fc1_1_weight=None, fc1_2_weight=None, fc2_weight=fc2, fc1_1_2_weight=fc1)
        out.backward(self.dout)
        return out, x.grad, w.grad, fc1.grad, fc2.grad


@pytest.fixture(params=[True, False], ids=["placed_ep", "unplaced_non_ep"])
def case(cuda, request):
    c = _Case(cuda, request.param)
    try:
        yield c
    finally:
        experts.check_pending_routes(block=True)
        PLACEMENTS.clear()


def test_fwd_bwd_under_sync_debug_mode_error(case):
    ref = case.step()  # warm-up: device caches (M on the device, side stream) and the allocator's pool
    torch.cuda.synchronize()
    prev = torch.cuda.get_sync_debug_mode()
    torch.cuda.set_sync_debug_mode("error")
    try:
        got = case.step()
    finally:
        torch.cuda.set_sync_debug_mode(prev)
    torch.cuda.synchronize()
    for a, b, name in zip(got, ref, ("out", "dx", "dw", "d_gate_up", "d_down")):
        assert torch.equal(a, b), f"{name} differs from the same call outside sync debug mode"


def test_host_never_waits_for_the_gpu(case):
    case.step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    case.step()
    host_s = time.perf_counter() - t0  # includes this call's GPU time: an upper bound on enqueueing
    torch.cuda.synchronize()
    # Calibrate the spin kernel, then queue one that outlasts the enqueueing many times over.
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    cycles = 10_000_000
    start.record()
    torch.cuda._sleep(cycles)
    end.record()
    end.synchronize()
    per_cycle_s = start.elapsed_time(end) / 1e3 / cycles
    spin_s = min(max(0.5, 20.0 * host_s), 3.0)
    print(f"host fwd+bwd {host_s * 1e3:.1f} ms; spin {spin_s:.2f} s", flush=True)
    torch.cuda._sleep(int(spin_s / per_cycle_s))
    spin_done = torch.cuda.Event()
    spin_done.record()
    t0 = time.perf_counter()
    case.step()
    enqueue_s = time.perf_counter() - t0
    still_spinning = not spin_done.query()
    torch.cuda.synchronize()
    assert still_spinning, (
        f"the spin kernel queued before the layer had finished when the host returned from the layer's "
        f"forward + backward ({enqueue_s * 1e3:.1f} ms): some call waited for the GPU"
    )
