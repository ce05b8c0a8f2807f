"""Seeded random-shape sweep of every grouped-GEMM kind against the CPU
oracle: random group counts (empty, tiny, tile-straddling), random N/K/H/I
(multiples of 8, not of the 256 x 256 x 64 tile), both fc1 weight layouts and
the split variants.  Tolerance: bf16 max relative error 1e-2."""

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from placemoe_amd import kernels
from tests.helpers import assert_bf16_close

pytestmark = pytest.mark.gpu


def case(seed):
    rng = np.random.default_rng(1000 + seed)
    G = int(rng.integers(1, 9))
    counts = rng.choice([0, 1, 7, 63, 64, 65, 255, 256, 257, 513], size=G)
    if counts.sum() == 0:
        counts[0] = 33
    dims = [int(8 * rng.integers(1, 49)) for _ in range(3)]  # 8 .. 384
    return rng, counts, dims


def offsets(counts, cuda):
    off = np.zeros(len(counts) + 1, dtype=np.int64)
    np.cumsum(counts, out=off[1:])
    return off, torch.as_tensor(off, dtype=torch.int32).to(cuda)


@pytest.mark.parametrize("seed", range(24))
def test_sweep_all_kinds(cuda, seed):
    rng, counts, (d0, d1, d2) = case(seed)
    off, doff = offsets(counts, cuda)
    A, G = int(off[-1]), len(counts)
    g = torch.Generator().manual_seed(seed)
    bf = torch.bfloat16
    print(f"sweep seed={seed} counts={counts.tolist()} dims={(d0, d1, d2)}", flush=True)

    # fc1 + SwiGLU, merged [G, 2I, H] weights (H = d0, I = d1)
    H, I = d0, d1
    x = torch.randn((A, H), generator=g).to(bf)
    w1 = (torch.randn((G, 2 * I, H), generator=g) * 0.05).to(bf)
    w1d = w1.to(cuda)
    gu, act = kernels.gemm_fc1_swiglu(x.to(cuda), w1d, w1d.view(-1)[I * H:], 2 * I * H, doff, G, I)
    gu_ref = O.grouped_gemm_nt(x, w1, off)
    assert_bf16_close(gu, gu_ref, name="gu")
    assert_bf16_close(act, O.swiglu_forward(gu_ref[:, :I], gu_ref[:, I:]), name="act")
    # fc1 with split fc1_1 / fc1_2 weights [G, I, H] each
    wg, wu = w1[:, :I].contiguous(), w1[:, I:].contiguous()
    gu2, _ = kernels.gemm_fc1_swiglu(x.to(cuda), wg.to(cuda), wu.to(cuda), I * H, doff, G, I)
    assert torch.equal(gu2.cpu(), gu.cpu()), "split and merged fc1 weights must agree bitwise"

    # NT (N = d2, K = d1)
    a = torch.randn((A, d1), generator=g).to(bf)
    b = (torch.randn((G, d2, d1), generator=g) * 0.05).to(bf)
    assert_bf16_close(kernels.group_gemm_nt(a.to(cuda), b.to(cuda), doff), O.grouped_gemm_nt(a, b, off), name="nt")

    # NN (N = d0, K = 2 * d1 from two halves)
    a2 = torch.randn((A, 2 * d1), generator=g).to(bf)
    b2 = (torch.randn((G, 2 * d1, d0), generator=g) * 0.05).to(bf)
    c2 = kernels.group_gemm_nn(a2.to(cuda), b2[:, :d1].contiguous().to(cuda), doff,
                               b_second=b2[:, d1:].contiguous().to(cuda))
    assert_bf16_close(c2, O.grouped_gemm_nn(a2, b2, off), name="nn_split")

    # fc2 dgrad + SwiGLU backward (H = d0, I = d1)
    dy = torch.randn((A, H), generator=g).to(bf)
    w2 = (torch.randn((G, H, I), generator=g) * 0.05).to(bf)
    dg1 = kernels.gemm_fc2_dgrad_swiglu(dy.to(cuda), w2.to(cuda), gu_ref.to(cuda), doff)
    dgate, dup = O.swiglu_backward(O.grouped_gemm_nn(dy, w2, off), gu_ref[:, :I], gu_ref[:, I:])
    assert_bf16_close(dg1[:, :I], dgate, name="d_gate")
    assert_bf16_close(dg1[:, I:], dup, name="d_up")

    # TN wgrad (M = d2, N = d0), ragged K = group rows, zeros for empty groups
    ta = torch.randn((A, d2), generator=g).to(bf)
    tb = torch.randn((A, d0), generator=g).to(bf)
    wt = kernels.group_gemm_tn(ta.to(cuda), tb.to(cuda), doff)
    assert_bf16_close(wt, O.grouped_gemm_tn(ta, tb, off), name="tn")
    for gi, n in enumerate(counts):
        if n == 0:
            assert torch.count_nonzero(wt[gi]).item() == 0
