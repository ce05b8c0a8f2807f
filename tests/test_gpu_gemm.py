"""GPU parity of the grouped GEMM kernels (MFMA, persistent tile scheduler)
against the CPU oracle: ragged, tiny and empty groups, every operand layout
and both SwiGLU epilogues.  Tolerance: bf16 max relative error 1e-2."""

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from placemoe_amd import kernels
from tests.helpers import assert_bf16_close

pytestmark = pytest.mark.gpu


def _offsets(counts):
    off = np.zeros(len(counts) + 1, dtype=np.int64)
    np.cumsum(counts, out=off[1:])
    return off


def _dev_offsets(off, cuda):
    return torch.as_tensor(off, dtype=torch.int32).to(cuda)


GROUPS = {
    "ragged": [130, 0, 1, 17, 256, 5, 0, 64],
    "single": [300],
    "tiny": [1, 2, 3, 0, 0, 4],
    "big": [1500, 700, 129],
}


@pytest.mark.parametrize("groups", list(GROUPS))
@pytest.mark.parametrize("H,I", [(256, 128), (1024, 192), (200, 72)])
def test_fc1_swiglu_forward(cuda, groups, H, I):
    counts = GROUPS[groups]
    off = _offsets(counts)
    A, G = int(off[-1]), len(counts)
    g = torch.Generator().manual_seed(A + H + I)
    x = torch.randn((A, H), generator=g).to(torch.bfloat16)
    w1 = (torch.randn((G, 2 * I, H), generator=g) * 0.05).to(torch.bfloat16)
    print(f"fc1 groups={groups} H={H} I={I}", flush=True)
    gu, act = kernels.gemm_fc1_swiglu(x.to(cuda), w1.to(cuda), w1.to(cuda).view(-1)[I * H:], 2 * I * H,
                                      _dev_offsets(off, cuda), G, I)
    gu_ref = O.grouped_gemm_nt(x, w1, off)
    assert_bf16_close(gu, gu_ref, name="gate_up")
    assert_bf16_close(act, O.swiglu_forward(gu_ref[:, :I], gu_ref[:, I:]), name="act")


@pytest.mark.parametrize("groups", list(GROUPS))
@pytest.mark.parametrize("N,K", [(256, 128), (384, 320), (72, 200)])
def test_nt_forward(cuda, groups, N, K):
    counts = GROUPS[groups]
    off = _offsets(counts)
    A, G = int(off[-1]), len(counts)
    g = torch.Generator().manual_seed(A * 3 + N + K)
    a = torch.randn((A, K), generator=g).to(torch.bfloat16)
    b = (torch.randn((G, N, K), generator=g) * 0.05).to(torch.bfloat16)
    c = kernels.group_gemm_nt(a.to(cuda), b.to(cuda), _dev_offsets(off, cuda))
    assert_bf16_close(c, O.grouped_gemm_nt(a, b, off), name="nt")


@pytest.mark.parametrize("groups", list(GROUPS))
@pytest.mark.parametrize("N,K,split", [(256, 128, False), (384, 320, True), (72, 208, True)])
def test_nn_dgrad(cuda, groups, N, K, split):
    counts = GROUPS[groups]
    off = _offsets(counts)
    A, G = int(off[-1]), len(counts)
    g = torch.Generator().manual_seed(A * 5 + N + K)
    a = torch.randn((A, K), generator=g).to(torch.bfloat16)
    b = (torch.randn((G, K, N), generator=g) * 0.05).to(torch.bfloat16)
    if split:
        half = K // 2
        b0, b1 = b[:, :half].contiguous(), b[:, half:].contiguous()
        c = kernels.group_gemm_nn(a.to(cuda), b0.to(cuda), _dev_offsets(off, cuda), b_second=b1.to(cuda))
    else:
        c = kernels.group_gemm_nn(a.to(cuda), b.to(cuda), _dev_offsets(off, cuda))
    assert_bf16_close(c, O.grouped_gemm_nn(a, b, off), name="nn")


@pytest.mark.parametrize("groups", list(GROUPS))
@pytest.mark.parametrize("H,I", [(256, 128), (512, 320), (200, 72)])
def test_fc2_dgrad_swiglu_backward(cuda, groups, H, I):
    counts = GROUPS[groups]
    off = _offsets(counts)
    A, G = int(off[-1]), len(counts)
    g = torch.Generator().manual_seed(A * 7 + H + I)
    dy = torch.randn((A, H), generator=g).to(torch.bfloat16)
    w2 = (torch.randn((G, H, I), generator=g) * 0.05).to(torch.bfloat16)
    gu = torch.randn((A, 2 * I), generator=g).to(torch.bfloat16)
    dg1 = kernels.gemm_fc2_dgrad_swiglu(dy.to(cuda), w2.to(cuda), gu.to(cuda), _dev_offsets(off, cuda))
    dact = O.grouped_gemm_nn(dy, w2, off)
    d_gate, d_up = O.swiglu_backward(dact, gu[:, :I], gu[:, I:])
    assert_bf16_close(dg1[:, :I], d_gate, name="d_gate")
    assert_bf16_close(dg1[:, I:], d_up, name="d_up")


@pytest.mark.parametrize("groups", list(GROUPS))
@pytest.mark.parametrize("M,N,split", [(256, 128, False), (384, 320, True), (72, 200, False)])
def test_tn_wgrad_ragged_k_and_empty_groups(cuda, groups, M, N, split):
    counts = GROUPS[groups]
    off = _offsets(counts)
    A, G = int(off[-1]), len(counts)
    g = torch.Generator().manual_seed(A * 11 + M + N)
    a = torch.randn((A, M), generator=g).to(torch.bfloat16)
    b = torch.randn((A, N), generator=g).to(torch.bfloat16)
    ref = O.grouped_gemm_tn(a, b, off)
    if split:
        c0, c1 = kernels.group_gemm_tn(a.to(cuda), b.to(cuda), _dev_offsets(off, cuda), split=M // 2)
        c = torch.cat([c0, c1], dim=1)
    else:
        c = kernels.group_gemm_tn(a.to(cuda), b.to(cuda), _dev_offsets(off, cuda))
    assert_bf16_close(c, ref, name="tn")
    for gi, cnt in enumerate(counts):
        if cnt == 0:
            assert torch.count_nonzero(c[gi]).item() == 0, "empty group must store zeros"


def test_group_limit_mostly_empty(cuda):
    # G = 2048 (the largest table the tile scheduler's prefix takes), a few
    # hundred rows spread over a handful of groups: every other group is empty.
    G = 2048
    rng = np.random.default_rng(5)
    counts = np.zeros(G, dtype=np.int64)
    for gi, n in zip(rng.choice(G, 12, replace=False), rng.integers(1, 300, 12)):
        counts[gi] = n
    off = _offsets(counts)
    A = int(off[-1])
    g = torch.Generator().manual_seed(77)
    a = torch.randn((A, 64), generator=g).to(torch.bfloat16)
    b = (torch.randn((G, 72, 64), generator=g) * 0.05).to(torch.bfloat16)
    print(f"nt G={G} A={A}", flush=True)
    c = kernels.group_gemm_nt(a.to(cuda), b.to(cuda), _dev_offsets(off, cuda))
    assert_bf16_close(c, O.grouped_gemm_nt(a, b, off), name="nt_g2048")
    y = torch.randn((A, 40), generator=g).to(torch.bfloat16)
    print(f"tn G={G} A={A}", flush=True)
    w = kernels.group_gemm_tn(a.to(cuda), y.to(cuda), _dev_offsets(off, cuda))
    assert_bf16_close(w, O.grouped_gemm_tn(a, y, off), name="tn_g2048")
    assert torch.count_nonzero(w[torch.as_tensor(counts == 0)]).item() == 0


def test_mfma_lane_layout_identity(cuda):
    # X @ I^T = X exactly: pins the MFMA output lane -> (row, col) mapping.
    A, H = 200, 128
    off = _offsets([A])
    x = torch.randn((A, H)).to(torch.bfloat16)
    eye = torch.eye(H).to(torch.bfloat16).reshape(1, H, H)
    c = kernels.group_gemm_nt(x.to(cuda), eye.to(cuda), _dev_offsets(off, cuda))
    assert torch.equal(c.cpu().view(torch.int16), x.view(torch.int16))
