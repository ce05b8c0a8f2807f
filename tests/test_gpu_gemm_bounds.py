"""Grouped-GEMM paths that ordinary shapes do not reach.

* The weight gradient's fast path addresses each copy through one buffer
  descriptor over the copy's rows and advances K-tiles in the instruction's
  scalar offset; rows past the copy must fail the descriptor's range check
  (which covers the whole offset, vector plus scalar, on gfx950).  Pinned with
  operands whose rows past the last copy hold NaN and whose copies end off the
  64-row K-tile: every copy's gradient must be finite and equal fp32 products
  of its own rows (a leak of a neighbour's rows would show as a mismatch).
* A block's tiles past its LDS tile table are decoded on the spot.  The test
  build ``libplacemoe_amd_tiletab2.so`` keeps only two table entries, so that
  path runs at small shapes, for every kind and both weight-gradient orders
  (balanced for G <= 512 copies, plain beyond); its outputs must equal the
  shipped library's bit for bit (every tile is computed the same way wherever
  it is decoded) and the fp32 products within the bf16 bar.
* The shipped library runs fc1 + SwiGLU, the fc2 dgrad and the weight
  gradients on the four-wave kernel whenever K is a multiple of 64.  The test
  build ``libplacemoe_amd_w8.so`` runs the eight-wave kernel for every call,
  so its fast-load paths of those kinds stay covered: every kind against the
  fp32 products, and the two builds within the bf16 bar of each other (their
  MFMA shapes sum in different orders, so the bits may differ).
"""

import numpy as np
import pytest
import torch

from placemoe_amd import _capi, build, kernels
from tests.helpers import assert_bf16_close
from tests.test_gpu_gemm_random_layouts import check_every_kind

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M,N", [(256, 192), (1024, 768)])
def test_wgrad_does_not_read_rows_past_its_copy(cuda, M, N):
    counts = np.array([100, 63, 0, 137, 1, 101])  # none a multiple of 64; an empty copy
    off = np.zeros(len(counts) + 1, dtype=np.int64)
    np.cumsum(counts, out=off[1:])
    rows = int(off[-1]) + 93  # rows past the last copy: NaN
    gen = torch.Generator(device=cuda).manual_seed(11)
    a = torch.randn((rows, M), generator=gen, device=cuda).to(torch.bfloat16)
    b = torch.randn((rows, N), generator=gen, device=cuda).to(torch.bfloat16)
    a[int(off[-1]):] = float("nan")
    b[int(off[-1]):] = float("nan")
    print(f"wgrad bounds M={M} N={N} copies {counts.tolist()} rows {rows}", flush=True)
    offd = torch.as_tensor(off, dtype=torch.int32, device=cuda)
    grad = kernels.group_gemm_tn(a, b, offd)
    torch.cuda.synchronize()
    assert torch.isfinite(grad).all(), "rows past the last copy reached a gradient"
    for g in range(len(counts)):
        s, e = int(off[g]), int(off[g + 1])
        ref = a[s:e].float().t() @ b[s:e].float() if e > s else torch.zeros((M, N), device=cuda)
        assert_bf16_close(grad[g], ref, name=f"copy {g} ({e - s} rows)")


def _outputs(cuda, off, H, I, seed):
    """Every kind's outputs over the copies ``off`` with seeded operands."""
    G, A = len(off) - 1, int(off[-1])
    offd = torch.as_tensor(off, dtype=torch.int32, device=cuda)
    gen = torch.Generator(device=cuda).manual_seed(seed)

    def rn(*shape, scale=1.0):
        return (torch.randn(shape, generator=gen, device=cuda) * scale).to(torch.bfloat16)

    x, dy = rn(A, H), rn(A, H)
    w1, w2 = rn(G, 2 * I, H, scale=0.05), rn(G, H, I, scale=0.05)
    perm = torch.randperm(A, generator=gen, device=cuda).to(torch.int32)
    rw = (0.05 + 0.95 * torch.rand((A,), generator=gen, device=cuda)).to(torch.bfloat16)
    gu, act = kernels.gemm_fc1_swiglu(x, w1, w1.view(-1)[I * H:], 2 * I * H, offd, G, I)
    y, out = kernels.group_gemm_nt_combine_top1(act, w2, offd, perm, rw)
    dg1 = kernels.gemm_fc2_dgrad_swiglu(dy, w2, gu, offd)
    dact = kernels.group_gemm_nn(dy, w2, offd)
    dxp = kernels.group_gemm_nn_unpermute_top1(dg1, w1, offd, perm)
    wg2 = kernels.group_gemm_tn(dy, act, offd)
    wg1 = kernels.group_gemm_tn(dg1, x, offd)
    torch.cuda.synchronize()
    return {"gu": gu, "act": act, "y": y, "out": out, "dg1": dg1, "dact": dact, "dxp": dxp, "wg2": wg2,
            "wg1": wg1}


def _copies(G, A, seed, empty=0.2):
    rng = np.random.default_rng(seed)
    c = np.where(rng.random(G) < empty, 0, rng.integers(1, 2 * A // G, G))
    off = np.zeros(G + 1, dtype=np.int64)
    np.cumsum(c, out=off[1:])
    return off


@pytest.mark.parametrize("G,A,H,I", [(160, 60000, 1024, 768), (40, 90000, 512, 384), (600, 30000, 256, 256)],
                         ids=["g160", "g40", "g600_plain_wgrad_order"])
def test_tile_table_overflow_path(cuda, G, A, H, I):
    variant = build.variant_path("tiletab2")
    assert variant.exists(), f"{variant} is not built (python -m placemoe_amd.build)"
    off = _copies(G, A, seed=G)
    print(f"tile table of 2: G={G} A={int(off[-1])} H={H} I={I}", flush=True)
    ref = _outputs(cuda, off, H, I, seed=5)
    with _capi.using(variant):
        got = _outputs(cuda, off, H, I, seed=5)
        for k in ref:
            assert torch.equal(got[k], ref[k]), f"{k}: the two-entry tile table changes the result"
        check_every_kind(cuda, off, H, I, 9, f"tiletab2 G={G}")


@pytest.mark.parametrize("G,A,H,I", [(16, 20000, 1024, 512), (160, 30000, 512, 256), (5, 3000, 256, 192)],
                         ids=["g16", "g160", "g5"])
def test_eight_wave_build_every_kind(cuda, G, A, H, I):
    variant = build.variant_path("w8")
    assert variant.exists(), f"{variant} is not built (python -m placemoe_amd.build)"
    off = _copies(G, A, seed=G + 7)
    print(f"eight-wave build: G={G} A={int(off[-1])} H={H} I={I}", flush=True)
    ref = _outputs(cuda, off, H, I, seed=6)
    with _capi.using(variant):
        got = _outputs(cuda, off, H, I, seed=6)
        check_every_kind(cuda, off, H, I, 10, f"w8 G={G}")
    for k in ref:
        assert_bf16_close(got[k], ref[k], name=f"eight-wave against shipped build: {k}")
