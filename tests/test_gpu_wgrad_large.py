"""Weight gradient of a copy whose rows span more than 4 GiB.

The ragged-K weight-gradient kernel reads a group's rows through buffer
descriptors rebased per 64-row K-tile.  With 300,000 rows of H=7168 bf16
(4.3 GB per operand) the rebase offsets pass 2^32 bytes; a 32-bit rebase
would wrap and the tail of the group would silently load zeros.  Sampled
256 x 256 output tiles are checked against the CPU oracle in float32."""

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from placemoe_amd import kernels
from tests.helpers import assert_bf16_close

pytestmark = pytest.mark.gpu


def test_wgrad_group_past_4gib(cuda):
    counts = [1000, 300_000]
    M = N = 7168
    off = np.array([0, counts[0], counts[0] + counts[1]], dtype=np.int64)
    rows = int(off[-1])
    print(f"wgrad large: rows={rows} M={M} N={N} ({rows * N * 2 / 2**30:.2f} GiB per operand)", flush=True)
    g = torch.Generator(device=cuda).manual_seed(21)
    a = torch.randn((rows, M), generator=g, device=cuda).to(torch.bfloat16)
    b = torch.randn((rows, N), generator=g, device=cuda).to(torch.bfloat16)
    c = kernels.group_gemm_tn(a, b, torch.as_tensor(off, dtype=torch.int32).to(cuda))
    torch.cuda.synchronize()
    print("kernel done", flush=True)
    # group 1: the first tile, the last tile (its rows reach the group's end)
    # and one in between; group 0: one tile.
    checks = [(1, 0, 0), (1, M - 256, N - 256), (1, 3584, 1280), (0, 256, 6912)]
    for grp, m0, n0 in checks:
        s, e = int(off[grp]), int(off[grp + 1])
        a_t = a[s:e, m0:m0 + 256].contiguous().cpu()
        b_t = b[s:e, n0:n0 + 256].contiguous().cpu()
        ref = O.grouped_gemm_tn(a_t, b_t, [0, e - s])[0]
        assert_bf16_close(c[grp, m0:m0 + 256, n0:n0 + 256], ref, name=f"group {grp} tile ({m0},{n0})")
        print(f"group {grp} tile ({m0},{n0}) ok", flush=True)
