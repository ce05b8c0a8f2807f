"""Pins the oracle's fp16 arithmetic (CPU).  The reference's fused MoE op
takes bf16 or fp16 (veomni/ops/kernels/moe/__init__.py:44-49) and its ops
round in the input dtype; the oracle's rounding points follow the input
dtype.  No reference test or fixture holds fp16 values for this path, so
the checks are the float64 eager model of the reference op test
(tests/ops/test_fused_moe_split_vs_merged.py:21-44), run at fp16's
resolution, and planted bf16 roundings that those checks must catch."""

import numpy as np
import torch

from oracle import moe_oracle as O
from tests.test_oracle_kat import _eager_moe_f64

F16 = torch.float16


def _case(seed, dt, T=64, K=2, H=64, I=32, C=5):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((T, H), generator=g).to(dt)
    w = torch.rand((T, K), generator=g).to(dt)
    phys = np.random.default_rng(seed).integers(0, C, size=(T, K))
    phys[0, :] = C - 1  # a token routed twice to the same copy
    w1 = (torch.randn((C, 2 * I, H), generator=g) * 0.2).to(dt)
    w2 = (torch.randn((C, H, I), generator=g) * 0.2).to(dt)
    dout = torch.randn((T, H), generator=g).to(dt)
    return x, w, phys, w1, w2, dout


def _errors(dt, seed):
    x, w, phys, w1, w2, dout = _case(seed, dt)
    fwd = O.moe_layer_forward(x, w, phys, w1, w2)
    bwd = O.moe_layer_backward(dout, fwd, w, w1, w2)
    assert fwd["out"].dtype == dt and bwd["dx"].dtype == dt and bwd["dw1"].dtype == dt
    xd, wd = x.double().requires_grad_(True), w.double().requires_grad_(True)
    w1d, w2d = w1.double().requires_grad_(True), w2.double().requires_grad_(True)
    ref = _eager_moe_f64(xd, wd, phys, w1d, w2d)
    ref.backward(dout.double())
    pairs = (("out", fwd["out"], ref.detach()), ("dx", bwd["dx"], xd.grad), ("dw", bwd["dw"], wd.grad),
             ("dw1", bwd["dw1"], w1d.grad), ("dw2", bwd["dw2"], w2d.grad))
    return {n: (a.double() - b).abs().max().item() / b.abs().max().item() for n, a, b in pairs}


def test_fp16_layer_against_float64_autograd():
    # fp16 keeps 11 significant bits against bf16's 8: the fp16 layer is held
    # to 2e-3 (measured <= 1.2e-3), which the bf16 arithmetic of the same
    # inputs exceeds (4e-3 .. 7e-3), so the bar tells the two apart.
    for seed in range(3):
        e16 = _errors(F16, seed)
        assert max(e16.values()) < 2e-3, e16
        e_bf = _errors(torch.bfloat16, seed)
        assert max(e_bf.values()) > 2e-3, e_bf


def test_fp16_swiglu_rounding_points():
    # act against float64 silu(g) * u of the same fp16 gate/up values: two
    # fp16 roundings (<= 2^-11 each); a bf16 rounding left in the SwiGLU
    # (the planted mistake) is caught.
    g = torch.Generator().manual_seed(4)
    gate = (torch.randn(4096, generator=g) * 3).to(F16)
    up = torch.randn(4096, generator=g).to(F16)
    exact = torch.nn.functional.silu(gate.double()) * up.double()

    def err(a):
        return (a.double() - exact).abs().max().item() / exact.abs().max().item()

    act = O.swiglu_forward(gate, up)
    assert act.dtype == F16 and err(act) < 1.5e-3
    planted = (O.silu_f32(gate.float()).to(torch.bfloat16).float() * up.float()).to(torch.bfloat16).to(F16)
    assert err(planted) > 1.5e-3
    # backward: d_up = fp16(fp16(silu(g)) * dact) and d_gate through silu' -
    # against float64 autograd of silu(g) * u
    dact = torch.randn(4096, generator=g).to(F16)
    gd, ud = gate.double().requires_grad_(True), up.double().requires_grad_(True)
    (torch.nn.functional.silu(gd) * ud).backward(dact.double())
    d_gate, d_up = O.swiglu_backward(dact, gate, up)
    assert d_gate.dtype == F16 and d_up.dtype == F16
    for a, b in ((d_gate, gd.grad), (d_up, ud.grad)):
        assert (a.double() - b).abs().max().item() / b.abs().max().item() < 1.5e-3


def test_fp16_combine_against_float64():
    g = torch.Generator().manual_seed(9)
    T, K, H = 50, 4, 24
    y = torch.randn((T * K, H), generator=g).to(F16)
    w = torch.rand((T, K), generator=g).to(F16)
    pos = np.random.default_rng(1).permutation(T * K).reshape(T, K)
    out = O.combine_forward(y, pos, w)
    exact = (y.double()[torch.as_tensor(pos)] * w.double()[:, :, None]).sum(dim=1)
    assert out.dtype == F16
    assert (out.double() - exact).abs().max().item() / exact.abs().max().item() < 2e-3
    dout = torch.randn((T, H), generator=g).to(F16)
    dy, dw = O.combine_backward(dout, y, pos, w)
    dw_exact = (dout.double()[:, None, :] * y.double()[torch.as_tensor(pos)]).sum(dim=2)
    assert dy.dtype == F16 and dw.dtype == F16
    assert (dw.double() - dw_exact).abs().max().item() / dw_exact.abs().max().item() < 2e-3
    dy_exact = torch.empty((T * K, H), dtype=torch.float64)
    dy_exact[torch.as_tensor(pos).reshape(-1)] = (dout.double()[:, None, :] * w.double()[:, :, None]).reshape(-1, H)
    assert (dy.double() - dy_exact).abs().max().item() / dy_exact.abs().max().item() < 1e-3
