"""Shared comparison helpers for the parity tests.

Floating-point bar: the max relative error of a bf16 tensor is
max|actual - expected| / max|expected| and must be <= 1e-2; in addition every
element must satisfy |actual - expected| <= 2e-2 * |expected| + 1e-2 * max|expected|.
fp32 replica-gradient sums use 1e-5 in the same normwise sense.  fp16
results are checked against the fp16 oracle at FP16_REL.
"""

import numpy as np
import torch

BF16_REL = 1e-2
FOLD_REL = 1e-5
# fp16 results against the fp16 oracle: a few fp16 ulps (2^-10 relative) of
# accumulation-order difference; a bf16 rounding anywhere would exceed it.
FP16_REL = 2e-3


def max_rel_err(actual: torch.Tensor, expected: torch.Tensor) -> float:
    a = actual.detach().float().cpu()
    b = expected.detach().float().cpu()
    scale = b.abs().max().item()
    if scale == 0.0:
        return a.abs().max().item() if a.numel() else 0.0
    return (a - b).abs().max().item() / scale


def assert_bf16_close(actual, expected, rel=BF16_REL, name="tensor"):
    a = actual.detach().float().cpu()
    b = expected.detach().float().cpu()
    assert a.shape == b.shape, f"{name}: shape {tuple(a.shape)} != {tuple(b.shape)}"
    if b.numel() == 0:
        return
    assert torch.isfinite(a).all(), f"{name}: non-finite values"
    err = max_rel_err(a, b)
    assert err <= rel, f"{name}: max relative error {err:.3e} > {rel:.0e}"
    scale = b.abs().max().item()
    torch.testing.assert_close(a, b, rtol=2 * rel, atol=rel * scale, msg=lambda m: f"{name}: {m}")


def assert_exact(actual, expected, name="tensor"):
    a = actual.detach().cpu() if isinstance(actual, torch.Tensor) else torch.as_tensor(actual)
    b = expected.detach().cpu() if isinstance(expected, torch.Tensor) else torch.as_tensor(np.asarray(expected))
    assert tuple(a.shape) == tuple(b.shape), f"{name}: shape {tuple(a.shape)} != {tuple(b.shape)}"
    if a.dtype in (torch.bfloat16, torch.float16) or b.dtype in (torch.bfloat16, torch.float16):
        assert a.dtype == b.dtype, f"{name}: dtype {a.dtype} != {b.dtype}"
        a, b = a.view(torch.int16), b.view(torch.int16)
    else:
        a, b = a.to(torch.int64), b.to(torch.int64)
    bad = (a != b).nonzero()
    assert bad.numel() == 0, f"{name}: {bad.shape[0]} mismatches, first at {bad[0].tolist()}"
