"""Pins the CPU oracle before it is trusted as the checker.

Each function of ``oracle/moe_oracle.py`` is checked against something
independent of its own formula: the reference's known-answer tests, brute
force on tiny inputs, closed forms, or a float64 autograd model written as the
reference's own eager loop.  A planted mistake in the oracle (dropped term,
wrong index, transposed operand, wrong rounding point) fails at least one of
these checks.
"""

import itertools

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O

BF = torch.bfloat16


# --------------------------------------------------------------------------- routing


def test_map_known_answer_from_reference():
    # tests/distributed/test_hiermoe_forward_cover_planner.py:1010-1038
    M = np.array([[0, 1, 3, 2], [5, 1, 3, 4]])
    assert O.map_logical_to_physical(M, [0], [[3, 2, 0]]).tolist() == [[2, 3, 0]]
    L = np.array([0, 1, 3, 2, 3, 0])
    # invariant L[M[s, e]] == e for every source row
    assert np.array_equal(L[M], np.tile(np.arange(4), (2, 1)))


def test_map_per_token_source_brute_force():
    g = np.random.default_rng(0)
    M = g.integers(0, 50, size=(5, 9))
    src = g.integers(0, 5, size=40)
    sel = g.integers(0, 9, size=(40, 3))
    phys = O.map_logical_to_physical(M, src, sel)
    for t, k in itertools.product(range(40), range(3)):
        assert phys[t, k] == M[src[t], sel[t, k]]


def test_histogram_brute_force_and_sum():
    g = np.random.default_rng(1)
    phys = g.integers(0, 13, size=(77, 4))
    counts = O.histogram(phys, 13)
    for c in range(13):
        assert counts[c] == sum(1 for v in phys.reshape(-1) if v == c)
    assert counts.sum() == phys.size
    with pytest.raises(ValueError):
        O.histogram(np.array([[0, 13]]), 13)


def _stable_positions_brute(phys):
    flat = list(phys.reshape(-1))
    order = []
    for c in sorted(set(flat)):
        order += [i for i, v in enumerate(flat) if v == c]  # ascending index = stable
    pos = [0] * len(flat)
    for rank, i in enumerate(order):
        pos[i] = rank
    return np.array(pos).reshape(phys.shape)


@pytest.mark.parametrize("seed", range(5))
def test_scatter_index_is_stable_counting_sort(seed):
    g = np.random.default_rng(seed)
    phys = g.integers(0, 6, size=(31, 3))
    pos = O.scatter_index(phys)
    assert np.array_equal(pos, _stable_positions_brute(phys))
    off = O.group_offsets(O.histogram(phys, 6))
    flat, p = phys.reshape(-1), pos.reshape(-1)
    assert np.all((p >= off[flat]) & (p < off[flat + 1]))
    assert np.array_equal(np.sort(p), np.arange(p.size))


def test_group_offsets_closed_form():
    assert O.group_offsets([3, 0, 2]).tolist() == [0, 3, 3, 5]
    assert O.group_offsets([]).tolist() == [0]


def test_permute_places_rows():
    x = torch.arange(12, dtype=torch.float32).reshape(3, 4).to(BF)
    pos = np.array([[2, 0], [5, 1], [3, 4]])
    xp = O.permute(x, pos)
    for t in range(3):
        for k in range(2):
            assert torch.equal(xp[pos[t, k]], x[t])


# --------------------------------------------------------------------------- grouped GEMM


def _brute_gemm(a, b):  # a [m,k] b [k,n] float64 triple loop
    m, k = a.shape
    n = b.shape[1]
    out = np.zeros((m, n))
    for i in range(m):
        for j in range(n):
            out[i, j] = sum(float(a[i, q]) * float(b[q, j]) for q in range(k))
    return out


def test_grouped_gemms_brute_force_tiny():
    g = torch.Generator().manual_seed(2)
    off = np.array([0, 3, 3, 7])
    a = torch.randn((7, 5), generator=g).to(BF)
    bt = torch.randn((3, 4, 5), generator=g).to(BF)  # [G, N, K]
    bn = torch.randn((3, 5, 4), generator=g).to(BF)  # [G, K, N]
    nt, nn = O.grouped_gemm_nt(a, bt, off), O.grouped_gemm_nn(a, bn, off)
    for gi in range(3):
        s, e = off[gi], off[gi + 1]
        if e == s:
            continue
        ref_nt = _brute_gemm(a[s:e].float().numpy(), bt[gi].float().numpy().T)
        ref_nn = _brute_gemm(a[s:e].float().numpy(), bn[gi].float().numpy())
        assert np.allclose(nt[s:e].float().numpy(), ref_nt, rtol=8e-3, atol=1e-2)
        assert np.allclose(nn[s:e].float().numpy(), ref_nn, rtol=8e-3, atol=1e-2)
    b2 = torch.randn((7, 6), generator=g).to(BF)
    tn = O.grouped_gemm_tn(a, b2, off)
    assert torch.count_nonzero(tn[1]) == 0  # empty group stores zeros
    ref = _brute_gemm(a[3:7].float().numpy().T, b2[3:7].float().numpy())
    assert np.allclose(tn[2].float().numpy(), ref, rtol=8e-3, atol=1e-2)


def test_swiglu_closed_forms_and_finite_difference():
    x = torch.tensor([0.0, 20.0, -20.0, 1.0])
    s = O.silu_f32(x)
    assert s[0] == 0 and abs(s[1] - 20.0) < 1e-6 and abs(s[2]) < 1e-6
    assert abs(s[3] - 1.0 / (1.0 + np.exp(-1.0))) < 1e-7
    # silu backward against a central difference of silu in float64
    g = torch.linspace(-4, 4, 33).to(BF)
    u = torch.ones(33).to(BF)
    dact = torch.ones(33).to(BF)
    d_gate, d_up = O.swiglu_backward(dact, g, u)
    gd = g.double()
    h = 1e-6
    fd = ((gd + h) / (1 + torch.exp(-(gd + h))) - (gd - h) / (1 + torch.exp(-(gd - h)))) / (2 * h)
    assert torch.allclose(d_gate.double(), fd, rtol=1e-2, atol=1e-2)
    assert torch.equal(d_up, O.silu_f32(g.float()).to(BF))


def _eager_moe_f64(hidden, w, phys, w1, w2):
    """Per-copy eager loop in float64 (tests/ops/test_fused_moe_split_vs_merged.py:21-44)."""
    I = w1.shape[1] // 2
    out = torch.zeros_like(hidden)
    for c in range(w1.shape[0]):
        tok, kk = np.nonzero(phys == c)
        if tok.size == 0:
            continue
        tok_t, kk_t = torch.as_tensor(tok), torch.as_tensor(kk)
        x = hidden[tok_t]
        gate = x @ w1[c, :I].t()
        up = x @ w1[c, I:].t()
        y = (torch.nn.functional.silu(gate) * up) @ w2[c].t()
        out = out.index_add(0, tok_t, y * w[tok_t, kk_t].unsqueeze(1))
    return out


def test_layer_forward_backward_against_float64_autograd():
    g = torch.Generator().manual_seed(11)
    T, K, H, I, C = 24, 2, 32, 16, 5
    x = torch.randn((T, H), generator=g).to(BF)
    w = torch.rand((T, K), generator=g).to(BF)
    phys = np.random.default_rng(3).integers(0, C, size=(T, K))
    phys[0, :] = [4, 4]  # a token routed twice to the same copy
    w1 = (torch.randn((C, 2 * I, H), generator=g) * 0.2).to(BF)
    w2 = (torch.randn((C, H, I), generator=g) * 0.2).to(BF)
    dout = torch.randn((T, H), generator=g).to(BF)
    fwd = O.moe_layer_forward(x, w, phys, w1, w2)
    bwd = O.moe_layer_backward(dout, fwd, w, w1, w2)

    xd, wd = x.double().requires_grad_(True), w.double().requires_grad_(True)
    w1d, w2d = w1.double().requires_grad_(True), w2.double().requires_grad_(True)
    ref = _eager_moe_f64(xd, wd, phys, w1d, w2d)
    ref.backward(dout.double())

    def close(a, b, tol, name):
        err = (a.double() - b).abs().max().item() / b.abs().max().item()
        assert err < tol, f"{name}: {err}"

    close(fwd["out"], ref.detach(), 2e-2, "out")
    close(bwd["dx"], xd.grad, 3e-2, "dx")
    close(bwd["dw"], wd.grad, 3e-2, "dw")
    close(bwd["dw1"], w1d.grad, 3e-2, "dw1")
    close(bwd["dw2"], w2d.grad, 3e-2, "dw2")


def test_planted_transposed_operand_is_caught():
    # a transposed fc2 (using w2[c] instead of w2[c]^T on a square case) must
    # not pass the float64 model check above
    g = torch.Generator().manual_seed(5)
    T, H, I, C = 16, 8, 8, 2
    x = torch.randn((T, H), generator=g).to(BF)
    w = torch.ones((T, 1)).to(BF)
    phys = np.random.default_rng(0).integers(0, C, size=(T, 1))
    w1 = torch.randn((C, 2 * I, H), generator=g).to(BF)
    w2 = torch.randn((C, H, I), generator=g).to(BF)
    good = O.moe_layer_forward(x, w, phys, w1, w2)["out"]
    bad = O.moe_layer_forward(x, w, phys, w1, w2.transpose(1, 2).contiguous())["out"]
    ref = _eager_moe_f64(x.double(), w.double(), phys, w1.double(), w2.double())
    err_good = (good.double() - ref).abs().max() / ref.abs().max()
    err_bad = (bad.double() - ref).abs().max() / ref.abs().max()
    assert err_good < 2e-2 < err_bad


def _layer_case(seed, T=24, K=2, H=32, I=16, C=5, w=None):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((T, H), generator=g).to(BF)
    if w is None:
        w = torch.rand((T, K), generator=g).to(BF)
    phys = np.random.default_rng(seed).integers(0, C, size=(T, K))
    phys[0, :] = C - 1  # a token routed twice to the same copy
    w1 = (torch.randn((C, 2 * I, H), generator=g) * 0.2).to(BF)
    w2 = (torch.randn((C, H, I), generator=g) * 0.2).to(BF)
    dout = torch.randn((T, H), generator=g).to(BF)
    return x, w, phys, w1, w2, dout


def test_weighted_input_layer_against_float64_autograd():
    """The non-EP branch (router weight on the fc2 input) computes the same
    function as the eager loop, which applies it after fc2: they agree in
    exact arithmetic."""
    x, w, phys, w1, w2, dout = _layer_case(12)
    fwd = O.moe_layer_forward_weighted_input(x, w, phys, w1, w2)
    bwd = O.moe_layer_backward_weighted_input(dout, fwd, w, w1, w2)
    xd, wd = x.double().requires_grad_(True), w.double().requires_grad_(True)
    w1d, w2d = w1.double().requires_grad_(True), w2.double().requires_grad_(True)
    ref = _eager_moe_f64(xd, wd, phys, w1d, w2d)
    ref.backward(dout.double())
    for name, a, b, tol in (("out", fwd["out"], ref.detach(), 2e-2), ("dx", bwd["dx"], xd.grad, 3e-2),
                            ("dw", bwd["dw"], wd.grad, 3e-2), ("dw1", bwd["dw1"], w1d.grad, 3e-2),
                            ("dw2", bwd["dw2"], w2d.grad, 3e-2)):
        err = (a.double() - b).abs().max().item() / b.abs().max().item()
        assert err < tol, f"{name}: {err}"


def test_weighted_input_equals_ep_for_power_of_two_weights():
    """With router weights 2^-j every product with a weight is exact, so the
    two branches round at the same values: output, dx, dw1 and dw2 agree bit
    for bit; dw is summed over different products (dout * y against
    act * d_act_w) and agrees within the bf16 bar."""
    T, K = 24, 2
    j = torch.as_tensor(np.random.default_rng(7).integers(0, 6, size=(T, K)))
    w = torch.pow(2.0, -j.double()).to(BF)
    x, w, phys, w1, w2, dout = _layer_case(13, T=T, K=K, w=w)
    ep = O.moe_layer_forward(x, w, phys, w1, w2)
    ni = O.moe_layer_forward_weighted_input(x, w, phys, w1, w2)
    assert torch.equal(ep["out"], ni["out"])
    bep = O.moe_layer_backward(dout, ep, w, w1, w2)
    bni = O.moe_layer_backward_weighted_input(dout, ni, w, w1, w2)
    for k in ("dx", "dw1", "dw2", "dg1"):
        assert torch.equal(bep[k], bni[k]), k
    err = (bni["dw"].float() - bep["dw"].float()).abs().max() / bep["dw"].float().abs().max()
    assert err < 1e-2
    # and with general weights the two branches do differ (in bf16 rounding)
    x, w, phys, w1, w2, dout = _layer_case(13, T=T, K=K)
    assert not torch.equal(O.moe_layer_forward(x, w, phys, w1, w2)["out"],
                           O.moe_layer_forward_weighted_input(x, w, phys, w1, w2)["out"])


def test_weighted_input_planted_missing_weight_is_caught():
    """A backward that forgets the router weight in dact (planted here, in a
    copy of the oracle's steps) must fail the float64 model check."""
    x, w, phys, w1, w2, dout = _layer_case(14)
    fwd = O.moe_layer_forward_weighted_input(x, w, phys, w1, w2)
    pos, off = fwd["pos"], fwd["offsets"]
    d_act_w = O.grouped_gemm_nn(O.permute(dout, pos), w2, off)
    dg1_bad, _ = O.swiglu_backward_weighted(d_act_w, fwd["gu"], fwd["act"], torch.ones_like(fwd["row_w"]))
    dx_bad = O.unpermute_grad(O.grouped_gemm_nn(dg1_bad, w1, off), pos)
    dx_good = O.moe_layer_backward_weighted_input(dout, fwd, w, w1, w2)["dx"]
    xd = x.double().requires_grad_(True)
    _eager_moe_f64(xd, w.double(), phys, w1.double(), w2.double()).backward(dout.double())
    err = lambda a: ((a.double() - xd.grad).abs().max() / xd.grad.abs().max()).item()  # noqa: E731
    assert err(dx_good) < 3e-2 < err(dx_bad)


# --------------------------------------------------------------------------- combine


def test_combine_matches_fp32_index_add_and_linear_moe_known_answer():
    # fp32 index_add_ formulation of tests/distributed/test_hiermoe_cuda_combine.py:41-51
    g = torch.Generator().manual_seed(20260805)
    T, K, H = 19, 3, 33
    y = torch.randn((T * K, H), generator=g).to(BF)
    w = torch.rand((T, K), generator=g).to(BF)
    phys = np.random.default_rng(1).integers(0, 4, size=(T, K))
    pos = O.scatter_index(phys)
    weighted = torch.empty_like(y)
    token_of_row = torch.empty(T * K, dtype=torch.long)
    for t in range(T):
        for k in range(K):
            weighted[pos[t, k]] = (y[pos[t, k]].float() * w[t, k].float()).to(BF)
            token_of_row[pos[t, k]] = t
    ref = torch.zeros((T, H)).index_add_(0, token_of_row, weighted.float()).to(BF)
    out = O.combine_forward(y, pos, w)
    torch.testing.assert_close(out.float(), ref.float(), atol=2e-2, rtol=2e-2)
    # segment_sum is the same reduction
    torch.testing.assert_close(O.segment_sum(weighted, token_of_row.numpy(), T).float(), ref.float(), atol=2e-2,
                               rtol=2e-2)
    with pytest.raises(ValueError, match="outside"):
        O.segment_sum(weighted[:2], np.array([0, 2]), 2)


def test_combine_linear_moe_known_answer():
    # tests/distributed/test_hiermoe.py:914-921 eager linear MoE in float64 with
    # weights filled expert_id + 1 (:1649-1662): y = x @ W[e], routing 0.5 each.
    hidden = torch.tensor([[1.0, 2.0, 3.0], [0.5, -1.0, 2.0], [0.0, 1.0, 0.0], [2.0, 2.0, 2.0]]).to(BF)
    sel = np.array([[3, 0], [2, 3], [1, 2], [2, 1]])
    w = torch.full((4, 2), 0.5).to(BF)
    W = torch.stack([torch.full((3, 3), float(e + 1)) for e in range(4)])
    pos = O.scatter_index(sel)
    xp = O.permute(hidden, pos)
    off = O.group_offsets(O.histogram(sel, 4))
    y = O.grouped_gemm_nn(xp, W.to(BF), off)
    out = O.combine_forward(y, pos, w)
    expect = torch.zeros((4, 3), dtype=torch.float64)
    for t in range(4):
        for k in range(2):
            expect[t] += hidden[t].double() @ W[sel[t, k]].double() * 0.5
    torch.testing.assert_close(out.double(), expect, rtol=1e-2, atol=1e-2)


def test_combine_backward_against_autograd():
    g = torch.Generator().manual_seed(9)
    T, K, H = 12, 2, 16
    y = torch.randn((T * K, H), generator=g).to(BF)
    w = torch.rand((T, K), generator=g).to(BF)
    dout = torch.randn((T, H), generator=g).to(BF)
    pos = O.scatter_index(np.random.default_rng(2).integers(0, 3, size=(T, K)))
    yd, wd = y.double().requires_grad_(True), w.double().requires_grad_(True)
    pos_t = torch.as_tensor(pos)
    ref = sum(yd[pos_t[:, k]] * wd[:, k : k + 1] for k in range(K))
    ref.backward(dout.double())
    dy, dw = O.combine_backward(dout, y, pos, w)
    torch.testing.assert_close(dy.double(), yd.grad, rtol=1e-2, atol=1e-2)
    torch.testing.assert_close(dw.double(), wd.grad, rtol=2e-2, atol=5e-2)
    dx = O.unpermute_grad(y, pos)
    ref_dx = sum(y[pos_t[:, k]].double() for k in range(K))
    torch.testing.assert_close(dx.double(), ref_dx, rtol=1e-2, atol=1e-2)


# --------------------------------------------------------------------------- replica fold


def test_replica_fold_reference_known_answer():
    # tests/distributed/test_hiermoe.py:3286-3338: the two copies of a logical
    # expert hold 10 and 2 (gate_up) / 20 and 3 (down): totals 12 and 23.
    L = np.array([0, 1, 3, 2, 3, -1])
    gate = torch.zeros((6, 4, 3), dtype=BF)
    down = torch.zeros((6, 3, 3), dtype=BF)
    gate[2], down[2] = 10.0, 20.0
    gate[4], down[4] = 2.0, 3.0
    fg = O.replica_fold(gate, L, 4)
    fd = O.replica_fold(down, L, 4)
    assert torch.all(fg[3] == 12.0) and torch.all(fd[3] == 23.0)
    assert torch.count_nonzero(fg[0]) == 0
    # slot 4 saw no tokens: its contribution is zeroed first
    fz = O.replica_fold(gate, L, 4, slot_counts=[1, 1, 1, 1, 0, 0])
    assert torch.all(fz[3] == 10.0)


def test_replica_fold_equals_logical_gradient_of_eager_model():
    # tests/distributed/test_hiermoe.py:3702-3778: summing the copy gradients
    # of a replicated layer gives the gradient of the unreplicated model.
    g = torch.Generator().manual_seed(4)
    T, K, H, I, E = 20, 2, 16, 8, 3
    L = np.array([0, 1, 2, 0, 2])
    M = np.array([[0, 1, 2], [3, 1, 4]])
    src = np.arange(T) % 2
    sel = np.random.default_rng(5).integers(0, E, size=(T, K))
    x = torch.randn((T, H), generator=g).double()
    w = torch.rand((T, K), generator=g).double()
    w1 = (torch.randn((E, 2 * I, H), generator=g) * 0.3).double()
    w2 = (torch.randn((E, H, I), generator=g) * 0.3).double()
    logical1, logical2 = w1.clone().requires_grad_(True), w2.clone().requires_grad_(True)
    _eager_moe_f64(x, w, sel, logical1, logical2).square().sum().backward()
    copies1 = w1[torch.as_tensor(L)].clone().requires_grad_(True)
    copies2 = w2[torch.as_tensor(L)].clone().requires_grad_(True)
    phys = O.map_logical_to_physical(M, src, sel)
    _eager_moe_f64(x, w, phys, copies1, copies2).square().sum().backward()
    f1 = O.replica_fold(copies1.grad.float(), L, E)
    f2 = O.replica_fold(copies2.grad.float(), L, E)
    torch.testing.assert_close(f1.double(), logical1.grad, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(f2.double(), logical2.grad, rtol=1e-5, atol=1e-5)
