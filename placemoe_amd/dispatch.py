"""OpSlot: the named dispatch point the model calls for ``moe_experts``.

Same contract as the reference (veomni/ops/dispatch.py:38-102): ``bind``
resolves through the registry, ``use_non_eager_impl`` guards the call site,
calling an unbound or eager slot raises ``RuntimeError``.
"""

from __future__ import annotations

import logging
from typing import Any, Callable

from .kernel_registry import KERNEL_REGISTRY

logger = logging.getLogger(__name__)


class OpSlot:
    def __init__(self, op_name: str, variant: str):
        self.op_name = op_name
        self.variant = variant
        self._kernel: Callable | None = None
        self._impl_name: str | None = None

    def bind(self, impl_name: str) -> None:
        if self._impl_name is not None and self._impl_name != impl_name:
            logger.warning(
                "OpSlot('%s', '%s') rebound from '%s' to '%s'", self.op_name, self.variant, self._impl_name, impl_name
            )
        self._kernel = KERNEL_REGISTRY.resolve(self.op_name, self.variant, impl_name)
        self._impl_name = impl_name

    @property
    def use_non_eager_impl(self) -> bool:
        return self._kernel is not None

    def bound_kernel(self) -> Callable | None:
        return self._kernel

    def __call__(self, *args: Any, **kwargs: Any) -> Any:
        if self._kernel is None:
            raise RuntimeError(
                f"OpSlot('{self.op_name}', '{self.variant}') has no kernel bound. "
                "Call .bind() first or check .use_non_eager_impl before calling."
            )
        return self._kernel(*args, **kwargs)

    def __repr__(self) -> str:
        state = "unbound" if self._impl_name is None else ("eager" if self._kernel is None else f"kernel={self._kernel}")
        return f"OpSlot(op_name={self.op_name!r}, variant={self.variant!r}, {state})"


# The slot generated modeling code calls for the MoE experts forward.
veomni_moe_experts_forward = OpSlot("moe_experts", "standard")
