"""The op boundary mirrors the reference's registry, OpSlot and fused-op
contracts (veomni/ops/kernel_registry.py, veomni/ops/dispatch.py,
veomni/ops/kernels/moe/__init__.py): names, argument meaning and error types.
Hardware is mocked, as in tests/ops/test_moe_hw_gate.py."""

import pytest
import torch

import placemoe_amd
from placemoe_amd import fused_moe, kernel_registry
from placemoe_amd.dispatch import OpSlot
from placemoe_amd.kernel_registry import KERNEL_REGISTRY, HardwareRequirement, KernelRegistry, KernelSpec


def _spec(name="k", hw=HardwareRequirement(device_type="any")):
    return KernelSpec(name=name, op_name="op", variant="v", factory=lambda: (lambda *a: "ran"), hardware=hw)


def test_registry_resolve_semantics():
    reg = KernelRegistry()
    reg.register(_spec())
    assert reg.resolve("op", "v", "eager") is None
    assert reg.resolve("op", "v", "k")() == "ran"
    with pytest.raises(KeyError, match="Unknown kernel"):
        reg.resolve("op", "v", "nope")
    with pytest.raises(ValueError, match="Duplicate"):
        reg.register(_spec())
    reg.register(_spec(), force=True)
    assert reg.list_available("op", "v") == ["k"]


def test_hardware_gate_raises_runtime_error(monkeypatch):
    reg = KernelRegistry()
    reg.register(_spec("g", HardwareRequirement(device_type="gpu", arch="gfx950")))
    monkeypatch.setattr(kernel_registry, "gpu_available", lambda: False)
    with pytest.raises(RuntimeError, match="arch='gfx950'"):
        reg.resolve("op", "v", "g")
    monkeypatch.setattr(kernel_registry, "gpu_available", lambda: True)
    monkeypatch.setattr(kernel_registry, "gpu_arch", lambda: "gfx942")
    monkeypatch.setattr(kernel_registry, "gpu_compute_capability", lambda: 94)
    with pytest.raises(RuntimeError):
        reg.resolve("op", "v", "g")
    monkeypatch.setattr(kernel_registry, "gpu_arch", lambda: "gfx950")
    assert reg.resolve("op", "v", "g")() == "ran"


def test_hip_kernel_registered_for_moe_experts():
    assert "hip" in KERNEL_REGISTRY.list_available("moe_experts", "standard")


def test_opslot_contract(monkeypatch):
    slot = OpSlot("moe_experts", "standard")
    assert not slot.use_non_eager_impl
    with pytest.raises(RuntimeError, match="no kernel bound"):
        slot(None)
    slot.bind("eager")
    assert not slot.use_non_eager_impl and "eager" in repr(slot)
    monkeypatch.setattr(kernel_registry, "gpu_available", lambda: True)
    monkeypatch.setattr(kernel_registry, "gpu_arch", lambda: "gfx950")
    monkeypatch.setattr(kernel_registry, "gpu_compute_capability", lambda: 95)
    slot.bind("hip")
    assert slot.use_non_eager_impl and callable(slot.bound_kernel())
    with pytest.raises(KeyError):
        slot.bind("triton")


def test_fused_moe_forward_errors(monkeypatch):
    monkeypatch.setattr(fused_moe, "_fused_moe_forward", None)
    x = torch.zeros((2, 8), dtype=torch.bfloat16)
    w = torch.zeros((2, 1), dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError):
        placemoe_amd.fused_moe_forward(1, w, torch.zeros((2, 1), dtype=torch.long), x, None, None, None)
    monkeypatch.setattr(fused_moe, "_fused_moe_forward", lambda *a, **k: "called")
    with pytest.raises(AssertionError, match="routing_weights dtype"):
        fused_moe.fused_moe_forward(1, w.float(), None, x, None, None, None)
    with pytest.raises(AssertionError, match="hidden_states dtype"):
        fused_moe.fused_moe_forward(1, w, None, x.float(), None, None, None)
    assert fused_moe.fused_moe_forward(1, w, None, x, None, None, None) == "called"


def test_apply_patch_names_and_gate(monkeypatch):
    with pytest.raises(ValueError, match="Invalid fused_moe_kernel"):
        placemoe_amd.apply_veomni_fused_moe_patch("triton")
    monkeypatch.setattr(kernel_registry, "gpu_available", lambda: False)
    with pytest.raises(RuntimeError, match="gfx950"):
        placemoe_amd.apply_veomni_fused_moe_patch("hip")


def test_raw_forward_weight_combination_errors():
    x = torch.zeros((2, 8), dtype=torch.bfloat16)
    w = torch.zeros((2, 1), dtype=torch.bfloat16)
    sel = torch.zeros((2, 1), dtype=torch.long)
    fc = torch.zeros((1, 8, 8), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="not both"):
        fused_moe.hip_fused_moe_forward(1, w, sel, x, fc, fc, fc, fc1_1_2_weight=fc)
    with pytest.raises(ValueError, match="Split fc1 mode"):
        fused_moe.hip_fused_moe_forward(1, w, sel, x, fc, None, fc)
    # bf16 or fp16, the weights in the hidden states' dtype (checked before any device work)
    with pytest.raises(AssertionError, match="like the hidden states"):
        fused_moe.hip_fused_moe_forward(1, w, sel, x.half(), None, None, fc, fc1_1_2_weight=fc)
    with pytest.raises(AssertionError, match="bfloat16 or float16"):
        fused_moe.hip_fused_moe_forward(1, w, sel, x.float(), None, None, fc, fc1_1_2_weight=fc)


def test_kernels_refuse_cpu_tensors():
    from placemoe_amd import kernels

    with pytest.raises(AssertionError, match="GPU tensors"):
        kernels.route(torch.zeros((2, 2), dtype=torch.long), 4)
