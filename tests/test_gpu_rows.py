"""GPU parity of the bandwidth kernels: weighted combine and its gradient,
unpermute gradient (gather), and the fp32 segment sum."""

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from placemoe_amd import kernels
from tests.helpers import assert_bf16_close, assert_exact

pytestmark = pytest.mark.gpu


def _inputs(T, K, H, C, seed):
    g = torch.Generator().manual_seed(seed)
    sel = torch.randint(0, C, (T, K), generator=g)
    y = torch.randn((T * K, H), generator=g).to(torch.bfloat16)
    w = torch.rand((T, K), generator=g).to(torch.bfloat16)
    dout = torch.randn((T, H), generator=g).to(torch.bfloat16)
    return sel, y, w, dout


@pytest.mark.parametrize("T,K,H", [(1, 1, 8), (257, 2, 1024), (1024, 8, 2048), (96, 1, 7168), (33, 4, 4096),
                                   (19, 3, 33)])
def test_combine_forward_backward(cuda, T, K, H):
    sel, y, w, dout = _inputs(T, K, H, 7, T + K + H)
    r = kernels.route(sel.to(cuda), 7)
    pos = r.pos.cpu().numpy()
    out = kernels.combine_fwd(y.to(cuda), r.pos, w.to(cuda))
    assert_bf16_close(out, O.combine_forward(y, pos, w), name="combine out")
    dy, dw = kernels.combine_bwd(dout.to(cuda), y.to(cuda), r.pos, w.to(cuda))
    dy_ref, dw_ref = O.combine_backward(dout, y, pos, w)
    # dy is one bf16 product per element: bit-exact
    assert_exact(dy, dy_ref, "combine dy")
    assert_bf16_close(dw, dw_ref, name="combine dw")


@pytest.mark.parametrize("T,K,H", [(5, 2, 64), (1000, 8, 2048), (77, 3, 40)])
def test_unpermute_gradient_gather(cuda, T, K, H):
    sel, y, _, _ = _inputs(T, K, H, 5, 3 * T + H)
    r = kernels.route(sel.to(cuda), 5)
    out = kernels.moe_gather(y.to(cuda), r.pos)
    assert_bf16_close(out, O.unpermute_grad(y, r.pos.cpu().numpy()), name="gather")


@pytest.mark.parametrize(("source_rows", "output_rows", "hidden_size"), [(0, 7, 16), (19, 7, 33), (257, 31, 2048),
                                                                         (65536, 32768, 64)])
def test_segment_sum_matches_fp32_index_add(cuda, source_rows, output_rows, hidden_size):
    # Cases of tests/distributed/test_hiermoe_cuda_combine.py:14-51 plus the
    # combine micro-benchmark shape's row counts.
    g = torch.Generator().manual_seed(20260805)
    source = torch.randn((source_rows, hidden_size), generator=g).to(torch.bfloat16)
    index = torch.randint(output_rows, (source_rows,), generator=g)
    actual = kernels.segment_sum(source.to(cuda), index.to(cuda), output_rows)
    expected = torch.zeros((output_rows, hidden_size), dtype=torch.float32)
    expected.index_add_(0, index, source.float())
    assert actual.dtype == torch.bfloat16
    torch.testing.assert_close(actual.cpu().float(), expected.to(torch.bfloat16).float(), atol=2e-2, rtol=2e-2)
    assert_bf16_close(actual, O.segment_sum(source, index.numpy(), output_rows), name="segment sum")


def test_segment_sum_rejects_out_of_range_index(cuda):
    source = torch.randn((2, 8), dtype=torch.bfloat16, device=cuda)
    index = torch.tensor([0, 2], dtype=torch.long, device=cuda)
    with pytest.raises(ValueError, match="outside"):
        kernels.segment_sum(source, index, 2)


def test_combine_of_identity_routing_is_weighted_copy(cuda):
    # K=1 with unit weights: the combine returns y unpermuted, bit for bit.
    T, H = 300, 256
    g = torch.Generator().manual_seed(5)
    sel = torch.randint(0, 4, (T, 1), generator=g)
    y = torch.randn((T, H), generator=g).to(torch.bfloat16)
    w = torch.ones((T, 1), dtype=torch.bfloat16)
    r = kernels.route(sel.to(cuda), 4)
    out = kernels.combine_fwd(y.to(cuda), r.pos, w.to(cuda))
    pos = r.pos.cpu().numpy().reshape(-1)
    assert_exact(out, y[torch.as_tensor(pos)], "identity combine")
    assert np.array_equal(np.sort(pos), np.arange(T))


@pytest.mark.parametrize("seed", range(10))
def test_row_kernels_random_shapes(cuda, seed):
    # Seeded sweep: top-k 1..8 (every K the kernels specialise on plus the
    # generic path), H a multiple of 8 or not, copies 1..300.
    rng = np.random.default_rng(500 + seed)
    T = int(rng.integers(1, 700))
    K = int(rng.integers(1, 9))
    H = int(rng.choice([8, 24, 40, 264, 1000, 2056, 13, 77]))
    C = int(rng.integers(1, 300))
    print(f"rows seed={seed} T={T} K={K} H={H} C={C}", flush=True)
    sel, y, w, dout = _inputs(T, K, H, C, seed)
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16)
    r = kernels.route(sel.to(cuda), C)
    pos = r.pos.cpu().numpy()
    assert_exact(kernels.moe_scatter(x.to(cuda), r.pos), O.permute(x, pos), "scatter")
    assert_bf16_close(kernels.combine_fwd(y.to(cuda), r.pos, w.to(cuda)), O.combine_forward(y, pos, w),
                      name="combine out")
    dy, dw = kernels.combine_bwd(dout.to(cuda), y.to(cuda), r.pos, w.to(cuda))
    dy_ref, dw_ref = O.combine_backward(dout, y, pos, w)
    assert_exact(dy, dy_ref, "combine dy")
    assert_bf16_close(dw, dw_ref, name="combine dw")
    assert_bf16_close(kernels.moe_gather(y.to(cuda), r.pos), O.unpermute_grad(y, pos), name="gather")
