"""The registration snippet that the repository's integration guide tells a
maintainer to add to the reference runs as written: executed in a namespace
that stands in for the reference module (veomni/ops/kernels/moe/__init__.py:
its KERNEL_REGISTRY, KernelSpec, HardwareRequirement, module-level
``_fused_moe_forward`` and ``apply_veomni_fused_moe_patch``), it registers
the "hip" backend and lets the patch function bind it.  Hardware is mocked."""

import re
from pathlib import Path

import pytest

from placemoe_amd import kernel_registry
from placemoe_amd.fused_moe import hip_fused_moe_forward
from placemoe_amd.kernel_registry import HardwareRequirement, KernelRegistry, KernelSpec

DOC = Path(__file__).resolve().parent.parent / "INTEGRATION.md"


def _section_3_snippet() -> str:
    text = DOC.read_text()
    start = text.index("## 3. Registering the backend with the reference")
    end = text.index("\n## 4.", start)
    blocks = re.findall(r"```python\n(.*?)```", text[start:end], flags=re.S)
    assert len(blocks) == 1, "the registration section holds one python snippet"
    return blocks[0]


def test_integration_snippet_registers_and_binds_the_hip_backend(monkeypatch):
    calls = []

    def reference_apply_patch(name="triton"):  # the reference's own patch function
        calls.append(name)
        ns["_fused_moe_forward"] = f"reference:{name}"

    ns = {
        "KERNEL_REGISTRY": KernelRegistry(),
        "KernelSpec": KernelSpec,
        "HardwareRequirement": HardwareRequirement,
        "_fused_moe_forward": None,
        "apply_veomni_fused_moe_patch": reference_apply_patch,
    }
    exec(compile(_section_3_snippet(), str(DOC), "exec"), ns)

    reg = ns["KERNEL_REGISTRY"]
    assert reg.list_available("moe_experts", "standard") == ["hip"]
    monkeypatch.setattr(kernel_registry, "gpu_available", lambda: True)
    monkeypatch.setattr(kernel_registry, "gpu_compute_capability", lambda: 95)
    adapter = reg.resolve("moe_experts", "standard", "hip")
    assert callable(adapter)
    monkeypatch.setattr(kernel_registry, "gpu_compute_capability", lambda: 90)
    with pytest.raises(RuntimeError, match="compute_capability>=95"):
        reg.resolve("moe_experts", "standard", "hip")

    ns["apply_veomni_fused_moe_patch"]("hip")
    assert ns["_fused_moe_forward"] is hip_fused_moe_forward and calls == []
    ns["apply_veomni_fused_moe_patch"]("triton")
    assert ns["_fused_moe_forward"] == "reference:triton" and calls == ["triton"]
