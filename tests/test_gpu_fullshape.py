"""Floating-point parity at the full benchmark shapes, stage by stage.

Every kernel of the layer runs at the full shape of a benchmark config
(config 1: T=4096, K=2, H=1024, I=2816, 12 copies of 8 experts; config 2: T=16384, K=8, H=2048, I=768, 160 copies; config 3: 65536 rows over
16 copies of 1.2k-19.4k rows, H=7168, I=2048; config 4: T=32768, K=4, H=4096,
I=1536, 96 copies with empty and tiny ones; config 5: the config-2 shape over
256 copies of 128 experts).  Each
stage is then checked on the CPU with the oracle on a sample, fed with that
stage's own GPU inputs (so a stage is judged on its own rounding):

* fc1 + SwiGLU, fc2, fc2 dgrad + SwiGLU backward, fc1 dgrad: a sample of rows
  of every copy (its first and last row among them);
* both weight gradients: 256 x 256 output tiles of the largest copy (whose K
  is its whole row count), of the smallest non-empty copy, and every empty
  copy (which must be exactly zero);
* permute, combine and their gradients: exact or fp32-summed per token on a
  token sample.

Tolerance: the bf16 bar of ``tests/helpers.py`` (max relative error 1e-2).
"""

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from placemoe_amd import kernels
from placemoe_amd.workloads import make_workload
from tests.helpers import assert_bf16_close, assert_exact

pytestmark = pytest.mark.gpu


def _sample_rows(offsets, per_group, rng):
    """Per non-empty group: up to ``per_group`` row ids, always its first and last row."""
    out = []
    for g in range(offsets.size - 1):
        s, e = int(offsets[g]), int(offsets[g + 1])
        if e == s:
            continue
        n = e - s
        if n <= per_group:
            rows = np.arange(s, e)
        else:
            mid = rng.choice(np.arange(s + 1, e - 1), size=per_group - 2, replace=False)
            rows = np.sort(np.concatenate([[s, e - 1], mid]))
        out.append((g, rows))
    return out


def _rows(t, rows):
    return t[torch.as_tensor(rows, device=t.device)].cpu()


def _tiles(M, N, rng, count):
    """``count`` 256 x 256 tile origins, the first and the last tile among them."""
    mt, nt = (M + 255) // 256, (N + 255) // 256
    picks = {(0, 0), (mt - 1, nt - 1)}
    while len(picks) < min(count, mt * nt):
        picks.add((int(rng.integers(mt)), int(rng.integers(nt))))
    return [(m * 256, n * 256) for m, n in sorted(picks)]


def _check_wgrad(name, grad, a, b, offsets, groups, rng, tiles_per_group=4):
    """grad[g] = a[rows g]^T @ b[rows g], checked on 256 x 256 tiles."""
    G, M, N = grad.shape
    for g in groups:
        s, e = int(offsets[g]), int(offsets[g + 1])
        if e == s:
            assert torch.count_nonzero(grad[g]).item() == 0, f"{name}: empty copy {g} is not zero"
            continue
        for m0, n0 in _tiles(M, N, rng, tiles_per_group):
            a_t = a[s:e, m0:m0 + 256].contiguous().cpu()
            b_t = b[s:e, n0:n0 + 256].contiguous().cpu()
            ref = O.grouped_gemm_tn(a_t, b_t, [0, e - s])[0]
            got = grad[g, m0:m0 + 256, n0:n0 + 256].cpu()
            assert_bf16_close(got, ref, name=f"{name} copy {g} ({e - s} rows) tile ({m0},{n0})")


@pytest.mark.parametrize("config,per_group,tokens_checked",
                         [("toy", 64, 4096), ("qwen3", 24, 2048), ("dsv3", 256, 2048), ("skew", 48, 2048),
                          ("fold", 16, 2048)])
def test_full_shape_stagewise(cuda, config, per_group, tokens_checked):
    torch.set_num_threads(min(16, torch.get_num_threads()))
    wl = make_workload(config, device=cuda)
    T, K, H, I, C = wl.T, wl.K, wl.H, wl.I, wl.C
    print(f"full shape {config}: T={T} K={K} H={H} I={I} C={C}", flush=True)
    rng = np.random.default_rng(17)

    # --- forward, through the same C-ABI wrappers the layer uses
    r = kernels.route(wl.selected, C, mapping=wl.mapping, sources=wl.sources)
    offsets = r.offsets.cpu().numpy().astype(np.int64)
    counts = np.diff(offsets)
    src = wl.sources.cpu().numpy() if wl.sources is not None else np.zeros(T, dtype=np.int64)
    phys = O.map_logical_to_physical(wl.mapping.cpu().numpy(), src, wl.selected.cpu().numpy())
    assert_exact(r.phys, phys, "phys")
    assert_exact(r.offsets, O.group_offsets(O.histogram(phys, C)), "offsets")
    assert_exact(r.pos, O.scatter_index(phys), "pos")
    xp = kernels.moe_scatter(wl.hidden, r.pos)
    assert torch.equal(xp[r.pos.reshape(-1).long()], wl.hidden.repeat_interleave(K, dim=0)), "permute is not a copy"
    w_gate = wl.fc1
    w_up = wl.fc1.view(-1)[I * H:]
    gu, act = kernels.gemm_fc1_swiglu(xp, w_gate, w_up, 2 * I * H, r.offsets, C, I)
    y = kernels.group_gemm_nt(act, wl.fc2, r.offsets)
    w = wl.routing_weights
    out = kernels.combine_fwd(y, r.pos, w)
    # --- backward
    dout = torch.randn((T, H), generator=torch.Generator(device=cuda).manual_seed(5), device=cuda).to(torch.bfloat16)
    dy, dw = kernels.combine_bwd(dout, y, r.pos, w)
    dg1 = kernels.gemm_fc2_dgrad_swiglu(dy, wl.fc2, gu, r.offsets)
    d_fc2 = kernels.group_gemm_tn(dy, act, r.offsets)
    d_fc1 = kernels.group_gemm_tn(dg1, xp, r.offsets)
    dxp = kernels.group_gemm_nn(dg1, wl.fc1, r.offsets)
    dx = kernels.moe_gather(dxp, r.pos)
    torch.cuda.synchronize()
    print(f"kernels done; copy rows min {counts.min()} max {counts.max()} empty {(counts == 0).sum()}", flush=True)

    if K == 1:
        # The top-1 entry points the layer (and bench.py) runs instead: the
        # permute that records each row's token and weight, fc2 with the
        # combine in its epilogue and the fc1 dgrad with the unpermute
        # gradient in its epilogue.  Bit for bit against the unfused kernels
        # above, at this shape.
        xp1, row_src, row_w = kernels.moe_scatter_src(wl.hidden, r.pos, w)
        y1, out1 = kernels.group_gemm_nt_combine_top1(act, wl.fc2, r.offsets, row_src, row_w)
        dx1 = kernels.group_gemm_nn_unpermute_top1(dg1, wl.fc1, r.offsets, row_src)
        torch.cuda.synchronize()
        assert torch.equal(xp1, xp), "moe_scatter_src rows differ from moe_scatter"
        rows = r.pos.reshape(-1).long()
        assert torch.equal(row_src[rows].long(), torch.arange(T, device=cuda)), "row_src is not the row's token"
        assert torch.equal(row_w[rows], w.reshape(-1)), "row_w is not the row's router weight"
        assert torch.equal(y1, y), "fc2 + combine: Y differs from group_gemm_nt"
        assert torch.equal(out1, out), "fc2 + combine: output differs from combine_fwd"
        assert torch.equal(dx1, dx), "fc1 dgrad + unpermute differs from group_gemm_nn + moe_gather"
        del xp1, y1, out1, dx1
        print("top-1 fused entry points bit-identical at full shape", flush=True)

    # --- row-sampled GEMM stages, each fed its own GPU inputs
    w1c, w2c = wl.fc1.cpu(), wl.fc2.cpu()
    for g, rows in _sample_rows(offsets, per_group, rng):
        n = len(rows)
        sub = [0, n]
        xs, gus = _rows(xp, rows), _rows(gu, rows)
        ref_gu = O.grouped_gemm_nt(xs, w1c[g:g + 1], sub)
        assert_bf16_close(_rows(gu, rows), ref_gu, name=f"fc1 copy {g}")
        assert_bf16_close(_rows(act, rows), O.swiglu_forward(gus[:, :I], gus[:, I:]), name=f"swiglu copy {g}")
        ref_y = O.grouped_gemm_nt(_rows(act, rows), w2c[g:g + 1], sub)
        assert_bf16_close(_rows(y, rows), ref_y, name=f"fc2 copy {g}")
        dact = O.grouped_gemm_nn(_rows(dy, rows), w2c[g:g + 1], sub)
        d_gate, d_up = O.swiglu_backward(dact, gus[:, :I], gus[:, I:])
        assert_bf16_close(_rows(dg1, rows), torch.cat([d_gate, d_up], dim=1), name=f"fc2 dgrad+swiglu copy {g}")
        ref_dxp = O.grouped_gemm_nn(_rows(dg1, rows), w1c[g:g + 1], sub)
        assert_bf16_close(_rows(dxp, rows), ref_dxp, name=f"fc1 dgrad copy {g}")
    print("row-sampled GEMM stages ok", flush=True)

    # --- weight gradients: largest copy, smallest non-empty copy, empty copies
    nonempty = np.nonzero(counts)[0]
    groups = sorted({int(np.argmax(counts)), int(nonempty[np.argmin(counts[nonempty])])}
                    | set(np.nonzero(counts == 0)[0].tolist()))
    _check_wgrad("fc2 wgrad", d_fc2, dy, act, offsets, groups, rng)
    _check_wgrad("fc1 wgrad", d_fc1, dg1, xp, offsets, groups, rng)
    print(f"wgrad tiles ok for copies {groups}", flush=True)

    # --- combine, its gradient and the unpermute gradient on a token sample
    toks = np.sort(rng.choice(T, size=min(tokens_checked, T), replace=False))
    tt = torch.as_tensor(toks, device=cuda)
    pos_s = r.pos[tt].cpu().numpy()
    local = np.arange(len(toks) * K, dtype=np.int64).reshape(len(toks), K)
    y_s = y[r.pos[tt].reshape(-1).long()].cpu()
    w_s = w[tt].cpu()
    assert_bf16_close(out[tt].cpu(), O.combine_forward(y_s, local, w_s), name="combine fwd")
    ref_dy, ref_dw = O.combine_backward(dout[tt].cpu(), y_s, local, w_s)
    assert_bf16_close(dy[r.pos[tt].reshape(-1).long()].cpu(), ref_dy, name="combine bwd dy")
    assert_bf16_close(dw[tt].cpu(), ref_dw, name="combine bwd dw")
    dxp_s = dxp[torch.as_tensor(pos_s.reshape(-1), device=cuda).long()].cpu()
    assert_bf16_close(dx[tt].cpu(), O.unpermute_grad(dxp_s, local), name="unpermute grad")
    print("row kernels ok", flush=True)


def test_toy_config_full_forward_matches_oracle(cuda):
    """Config 1, the CPU-runnable case, at its full 4096 tokens: the layer's
    forward (the configuration is forward-only) against the oracle's."""
    from placemoe_amd import experts

    torch.set_num_threads(min(16, torch.get_num_threads()))
    wl = make_workload("toy")
    assert wl.T == 4096 and wl.K == 2 and wl.C == 12
    with torch.no_grad():
        out = experts.expert_layer(wl.hidden.to(cuda), wl.routing_weights.to(cuda), wl.selected.to(cuda),
                                   wl.fc2.to(cuda), fc1_1_2_weight=wl.fc1.to(cuda), mapping=wl.mapping.to(cuda),
                                   sources=wl.sources.to(cuda))
    phys = O.map_logical_to_physical(wl.mapping.numpy(), wl.sources.numpy(), wl.selected.numpy())
    fwd = O.moe_layer_forward(wl.hidden, wl.routing_weights, phys, wl.fc1, wl.fc2)
    assert_bf16_close(out, fwd["out"], name="config-1 layer output")
