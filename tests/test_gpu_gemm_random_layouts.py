"""Randomised sweep of the grouped GEMM entry points: copy counts from 1 to
160, ragged, tiny and empty copies, hidden and intermediate sizes on and off
the 64-row K-tile (so both the buffer->LDS and the register-staged operand
paths run), every kind, against fp32 products of the same bf16 operands on
the GPU (a floating-point kernel's reference).  The top-1 entry points must
equal the plain GEMM followed by the separate row operation bit for bit.
Tolerance: the bf16 bar of ``tests/helpers.py`` (max relative error 1e-2).
"""

import numpy as np
import pytest
import torch

from placemoe_amd import kernels
from tests.helpers import assert_bf16_close

pytestmark = pytest.mark.gpu

CASES_PER_SEED = 12


def _groups(rng):
    G = int(rng.choice([1, 2, 5, 16, 40, 96, 160]))
    kind = int(rng.integers(4))
    if kind == 0:
        c = rng.integers(0, 600, G)
    elif kind == 1:
        c = rng.integers(0, 40, G)
    elif kind == 2:
        c = np.where(rng.random(G) < 0.3, 0, rng.integers(200, 3000, G))
    else:
        c = rng.integers(1, 8000 // G + 2, G)
    if c.sum() > 20000:
        c = (c * (20000 / c.sum())).astype(np.int64)
    off = np.zeros(G + 1, dtype=np.int64)
    np.cumsum(c, out=off[1:])
    return G, off


def _per_group(a, off, fn):
    out = None
    for g in range(len(off) - 1):
        s, e = int(off[g]), int(off[g + 1])
        if e > s:
            r = fn(g, a[s:e].float())
            if out is None:
                out = torch.zeros((a.shape[0], r.shape[1]), dtype=torch.float32, device=a.device)
            out[s:e] = r
    return out


def check_every_kind(cuda, off, H, I, gen_seed, name):
    """Every GEMM kind over the copies ``off`` (row offsets) against fp32
    products on the GPU; the top-1 entry points bit for bit against the plain
    GEMM plus the separate row operation."""
    G = len(off) - 1
    A = int(off[-1])
    offd = torch.as_tensor(off, dtype=torch.int32, device=cuda)
    gen = torch.Generator(device=cuda).manual_seed(gen_seed)

    def rn(*shape, scale=1.0):
        return (torch.randn(shape, generator=gen, device=cuda) * scale).to(torch.bfloat16)

    x, dy = rn(A, H), rn(A, H)
    w1, w2 = rn(G, 2 * I, H, scale=0.05), rn(G, H, I, scale=0.05)

    gu, act = kernels.gemm_fc1_swiglu(x, w1, w1.view(-1)[I * H:], 2 * I * H, offd, G, I)
    assert_bf16_close(gu, _per_group(x, off, lambda g, a: a @ w1[g].float().t()), name=f"{name} fc1")
    y = kernels.group_gemm_nt(act, w2, offd)
    assert_bf16_close(y, _per_group(act, off, lambda g, a: a @ w2[g].float().t()), name=f"{name} fc2")
    dact = kernels.group_gemm_nn(dy, w2, offd)
    ref_dact = _per_group(dy, off, lambda g, a: a @ w2[g].float())
    assert_bf16_close(dact, ref_dact, name=f"{name} dgrad")
    dg1 = kernels.gemm_fc2_dgrad_swiglu(dy, w2, gu, offd)
    d = ref_dact.to(torch.bfloat16).float()
    gate, up = gu[:, :I].float(), gu[:, I:].float()
    sg = torch.sigmoid(gate)
    assert_bf16_close(dg1[:, :I], d * up * sg * (1 + gate * (1 - sg)), name=f"{name} d_gate")
    assert_bf16_close(dg1[:, I:], d * (gate * sg).to(torch.bfloat16).float(), name=f"{name} d_up")
    wg = kernels.group_gemm_tn(dy, act, offd)
    for g in range(G):
        s, e = int(off[g]), int(off[g + 1])
        ref = dy[s:e].float().t() @ act[s:e].float() if e > s else torch.zeros((H, I), device=cuda)
        assert_bf16_close(wg[g], ref, name=f"{name} wgrad copy {g}")

    perm = torch.randperm(A, generator=gen, device=cuda).to(torch.int32)
    rw = (0.05 + 0.95 * torch.rand((A,), generator=gen, device=cuda)).to(torch.bfloat16)
    c2, out = kernels.group_gemm_nt_combine_top1(act, w2, offd, perm, rw)
    ref_out = torch.empty_like(out)
    ref_out[perm.long()] = ((y.float() * rw.float()[:, None]).to(torch.bfloat16).float() + 0.0).to(torch.bfloat16)
    assert torch.equal(c2, y) and torch.equal(out, ref_out), f"{name}: fc2 + combine differs from fc2, combine"
    dxp = kernels.group_gemm_nn_unpermute_top1(dy, w2, offd, perm)
    assert torch.equal(dxp[perm.long()], dact), f"{name}: dgrad + unpermute differs from dgrad, unpermute"


@pytest.mark.parametrize("seed", [101, 202, 303, 404])
def test_random_shapes_every_kind(cuda, seed):
    rng = np.random.default_rng(seed)
    for case in range(CASES_PER_SEED):
        G, off = _groups(rng)
        A = int(off[-1])
        H = int(rng.choice([64, 128, 200, 256, 512, 768, 1024]))
        I = int(rng.choice([64, 128, 136, 256, 384]))
        print(f"seed {seed} case {case}: G={G} A={A} H={H} I={I}", flush=True)
        if A == 0:
            continue
        check_every_kind(cuda, off, H, I, seed * 1000 + case, f"seed {seed} case {case}")


def test_top1_outputs_past_2gib(cuda):
    """Top-1 outputs of more than 2 GiB (rows past the 32-bit byte offsets of
    one buffer descriptor) take the 64-bit store path; they must still equal
    the plain GEMM followed by the separate row operation bit for bit."""
    A, K, N = 131200, 64, 8192  # A * N * 2 bytes > 2^31
    off = np.array([0, 70000, A], dtype=np.int64)
    offd = torch.as_tensor(off, dtype=torch.int32, device=cuda)
    gen = torch.Generator(device=cuda).manual_seed(77)
    print(f"top-1 > 2 GiB: A={A} K={K} N={N}", flush=True)
    act = torch.randn((A, K), generator=gen, device=cuda).to(torch.bfloat16)
    w2 = (torch.randn((2, N, K), generator=gen, device=cuda) * 0.1).to(torch.bfloat16)
    perm = torch.randperm(A, generator=gen, device=cuda).to(torch.int32)
    rw = (0.05 + 0.95 * torch.rand((A,), generator=gen, device=cuda)).to(torch.bfloat16)
    y = kernels.group_gemm_nt(act, w2, offd)
    c2, out = kernels.group_gemm_nt_combine_top1(act, w2, offd, perm, rw)
    assert torch.equal(c2, y)
    ref_out = torch.empty_like(out)
    ref_out[perm.long()] = (y * rw[:, None]).float().add_(0.0).to(torch.bfloat16)
    assert torch.equal(out, ref_out), "fc2 + combine past 2 GiB differs from fc2, combine"
    del c2, out, ref_out
    b = w2.transpose(1, 2).contiguous()  # [2, K, N]
    dy = act
    dact = kernels.group_gemm_nn(dy, b, offd)
    dxp = kernels.group_gemm_nn_unpermute_top1(dy, b, offd, perm)
    assert torch.equal(dxp[perm.long()], dact), "dgrad + unpermute past 2 GiB differs from dgrad, unpermute"
