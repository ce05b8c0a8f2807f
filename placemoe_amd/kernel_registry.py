"""(op, variant, impl) -> KernelSpec registry with hardware gates.

Same contract as the reference's registry
(veomni/ops/kernel_registry.py:35-165): ``resolve`` returns ``None`` for
``"eager"``, raises ``KeyError`` for an unknown implementation and
``RuntimeError`` when the hardware gate fails; duplicate registration raises
``ValueError`` unless ``force=True``.  The hardware gate adds an ``arch``
field so a kernel built for one GPU ISA (``gfx950``) is refused elsewhere.
"""

from __future__ import annotations

import logging
from dataclasses import dataclass
from typing import Callable

import torch

logger = logging.getLogger(__name__)


def gpu_available() -> bool:
    return torch.cuda.is_available()


def gpu_arch() -> str:
    """The GPU ISA name of device 0 (e.g. ``gfx950``), or ``""`` without a GPU."""
    if not gpu_available():
        return ""
    props = torch.cuda.get_device_properties(0)
    return str(getattr(props, "gcnArchName", "")).split(":")[0]


def gpu_compute_capability() -> int:
    """major*10 + minor as torch reports it (0 without a GPU)."""
    if not gpu_available():
        return 0
    major, minor = torch.cuda.get_device_capability()
    return major * 10 + minor


@dataclass(frozen=True)
class HardwareRequirement:
    device_type: str  # "gpu" | "npu" | "any"
    min_compute_capability: int | None = None
    max_compute_capability: int | None = None
    arch: str | None = None  # exact GPU ISA, e.g. "gfx950"

    def is_satisfied(self) -> bool:
        if self.device_type == "any":
            return True
        if self.device_type == "npu":
            return False
        if self.device_type != "gpu":
            raise ValueError(f"Unknown device_type: {self.device_type!r} (expected 'gpu' | 'npu' | 'any')")
        if not gpu_available():
            return False
        if self.arch is not None and gpu_arch() != self.arch:
            return False
        cc = gpu_compute_capability()
        if self.min_compute_capability is not None and cc < self.min_compute_capability:
            return False
        if self.max_compute_capability is not None and cc > self.max_compute_capability:
            return False
        return True

    def describe(self) -> str:
        parts = [f"device_type='{self.device_type}'"]
        if self.arch is not None:
            parts.append(f"arch='{self.arch}'")
        lo, hi = self.min_compute_capability, self.max_compute_capability
        if lo is not None and hi is not None:
            parts.append(f"{lo}<=compute_capability<={hi}")
        elif lo is not None:
            parts.append(f"compute_capability>={lo}")
        elif hi is not None:
            parts.append(f"compute_capability<={hi}")
        return ", ".join(parts)


@dataclass(frozen=True)
class KernelSpec:
    name: str
    op_name: str
    variant: str
    factory: Callable[[], Callable]
    hardware: HardwareRequirement
    description: str = ""


class KernelRegistry:
    def __init__(self) -> None:
        self._specs: dict[tuple[str, str], dict[str, KernelSpec]] = {}

    def register(self, spec: KernelSpec, force: bool = False) -> None:
        bucket = self._specs.setdefault((spec.op_name, spec.variant), {})
        if spec.name in bucket and not force:
            raise ValueError(
                f"Duplicate kernel registration: op='{spec.op_name}', variant='{spec.variant}', name='{spec.name}'"
            )
        if spec.name in bucket:
            logger.info("kernel %s/%s/%s replaced", spec.op_name, spec.variant, spec.name)
        bucket[spec.name] = spec

    def resolve(self, op_name: str, variant: str, impl_name: str) -> Callable | None:
        if impl_name == "eager":
            return None
        bucket = self._specs.get((op_name, variant), {})
        if impl_name not in bucket:
            raise KeyError(
                f"Unknown kernel '{impl_name}' for op='{op_name}', variant='{variant}'. "
                f"Available: {list(bucket) + ['eager']}"
            )
        spec = bucket[impl_name]
        if not spec.hardware.is_satisfied():
            raise RuntimeError(
                f"Kernel '{impl_name}' for op='{op_name}' requires {spec.hardware.describe()}, "
                "but the current hardware does not satisfy this."
            )
        return spec.factory()

    def list_available(self, op_name: str, variant: str) -> list[str]:
        return list(self._specs.get((op_name, variant), {}))


KERNEL_REGISTRY = KernelRegistry()
