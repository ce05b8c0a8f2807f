"""CPU oracle for the PlaceMoE expert-layer hot path (TEST INFRASTRUCTURE ONLY).

This module restates, on the CPU, what the reference computes on the path
map -> histogram/scan -> permute -> SwiGLU grouped GEMM (fwd, dgrad, wgrad)
-> weighted combine -> replica-gradient fold.  It is the checker for the HIP
library and nothing else: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it.  The product path
(``placemoe_amd``) never imports it and has no CPU fallback.

Integer work is numpy; floating-point work is torch on the CPU in float32
with bf16 rounding at the points where the reference stores bf16 tensors
(fp16 rounding at the same points for fp16 inputs).

Reference citations are paths under the reference repository
(pia7a/PlaceMoE), ``file:line``.

How each function is pinned (the checks live in ``tests/test_oracle_*.py``):

* ``map_logical_to_physical`` - the reference's source-LUT known answer
  (tests/distributed/test_hiermoe_forward_cover_planner.py:1032-1038), the
  ``L[M] == e`` invariant and the mirrored-R2 closed form.
* ``histogram`` / ``group_offsets`` - brute-force counting; sum == A.
* ``scatter_index`` - a pure-Python stable insertion loop on small inputs,
  and the permutation / stability invariants.
* ``grouped_gemm_nt`` / ``grouped_gemm_nn`` / ``grouped_gemm_tn`` -
  brute-force triple loops in float64 on tiny inputs.
* ``expert_layer_forward`` / ``expert_layer_backward`` - an independent
  float64 autograd model (the reference test's per-expert eager loop,
  tests/ops/test_fused_moe_split_vs_merged.py:21-44), forward and gradients.
* ``row_weights`` / ``weight_rows`` / ``swiglu_backward_weighted`` /
  ``moe_layer_forward_weighted_input`` / ``moe_layer_backward_weighted_input``
  (the non-EP branch) - the same float64 autograd model (the router weight
  commutes with fc2 in exact arithmetic); with power-of-two router weights,
  where every product with the weight is exact, the output, dx, dw1 and dw2
  equal the EP branch's bit for bit; a planted backward that drops the
  router weight from dact is caught.
* ``combine_forward`` / ``combine_backward`` / ``unpermute_grad`` - fp32
  ``index_add_`` (tests/distributed/test_hiermoe_cuda_combine.py:41-51),
  autograd of the weighted sum, and the reference's double-precision eager
  linear MoE (tests/distributed/test_hiermoe.py:914-921).
* ``replica_fold`` - the reference's known answer 10+2=12, 20+3=23
  (tests/distributed/test_hiermoe.py:3286-3338) and "sum of copy grads ==
  logical-expert grad of the eager model" (tests/distributed/test_hiermoe.py:3765-3778).
* ``build_local_payload`` / ``aggregate_weighted_outputs`` - the reference's
  known answer for the aggregation (tests/distributed/test_hiermoe.py:1116-1128),
  a dictionary-based pure-Python payload on random inputs, and the
  reference's own end-to-end check (test_hiermoe.py:1009-1011, the rank-dedup
  dispatch + experts + combine equals the eager MoE at 1e-5, :935-996) with ranks simulated in
  one process.
* ``route_statistics`` - the reference's known answer (demand
  [[2,1,1,0],[0,1,1,2]] and the co-selection entries of
  tests/distributed/test_placemoe_optimizer.py:50-73), a pure-Python count
  over token pairs on random samples, and the invariants sum(demand[s]) =
  T_s*K, symmetry, zero diagonal, sum(affinity[s]) = 2 * #distinct pairs.
* ``replica_grad_schedule`` / ``replica_grad_sync`` / ``owner_grad_norm_mask``
  - the reference's three known answers (the 2-rank cover 12 / 23,
  tests/distributed/test_hiermoe.py:3200-3338; the three-copy owner exchange
  6 / 60, :3545-3592; the 4-rank pair graph, :3480-3540) with their
  pairwise / globally-ordered flags, and on random layouts the invariant that
  every copy ends with the exact sum of its expert's copies.
"""

from __future__ import annotations

import numpy as np
import torch

BF16 = torch.bfloat16


# ---------------------------------------------------------------------------
# Integer routing path
# ---------------------------------------------------------------------------


def map_logical_to_physical(M: np.ndarray, src: np.ndarray, sel: np.ndarray) -> np.ndarray:
    """phys[t, k] = M[src[t], sel[t, k]].

    Follows ``ExpertSwapManager._map_logical_to_slot_dedup_aware``
    (veomni/distributed/moe/hiermoe/expert_swap.py:5914-5921), which gathers row
    ``ep_rank`` of ``source_logical_to_physical`` with ``index_select``.  Here the
    source is per token (``src[t]``); the reference is the case ``src[:] = ep_rank``.
    """
    M = np.asarray(M, dtype=np.int64)
    sel = np.asarray(sel, dtype=np.int64)
    src = np.asarray(src, dtype=np.int64).reshape(-1)
    if sel.ndim == 1:
        sel = sel[:, None]
    return M[src[:, None], sel]


def histogram(phys: np.ndarray, num_bins: int) -> np.ndarray:
    """counts[c] = #{(t,k) : phys[t,k] == c}.

    ``expert_histogram`` (veomni/ops/kernels/moe/_kernels/kernel/moe.py:53-82) and
    its EP analogue ``torch.bincount(..., minlength=C)``
    (veomni/distributed/moe/hiermoe/all_to_all.py:827).
    """
    flat = np.asarray(phys, dtype=np.int64).reshape(-1)
    if flat.size and (flat.min() < 0 or flat.max() >= num_bins):
        raise ValueError("phys contains a slot outside [0, num_bins)")
    return np.bincount(flat, minlength=num_bins).astype(np.int64)


def group_offsets(counts: np.ndarray) -> np.ndarray:
    """Exclusive prefix ``offsets[C+1]``; ``offsets[1:]`` is the reference's
    inclusive ``cumsum_M`` (veomni/ops/kernels/moe/group_gemm.py:239,477,770)."""
    counts = np.asarray(counts, dtype=np.int64)
    out = np.zeros(counts.size + 1, dtype=np.int64)
    np.cumsum(counts, out=out[1:])
    return out


def scatter_index(phys: np.ndarray) -> np.ndarray:
    """pos[t,k] = rank of flat index t*K+k in a stable sort of phys.

    ``phys.flatten().argsort(stable=True).argsort()``
    (veomni/ops/kernels/moe/group_gemm.py:474); equivalently
    ``offsets[phys] + #{a' < a : phys[a'] == phys[a]}``.
    """
    phys = np.asarray(phys, dtype=np.int64)
    flat = phys.reshape(-1)
    order = np.argsort(flat, kind="stable")
    pos = np.empty_like(order)
    pos[order] = np.arange(flat.size, dtype=np.int64)
    return pos.reshape(phys.shape)


def permute(X: torch.Tensor, pos: np.ndarray) -> torch.Tensor:
    """Xp[pos[t,k]] = X[t]  (``moe_scatter``, moe.py:251-333)."""
    pos_t = torch.as_tensor(np.asarray(pos, dtype=np.int64))
    T, K = pos_t.shape
    out = torch.empty((T * K, X.shape[1]), dtype=X.dtype)
    out[pos_t.reshape(-1)] = X.repeat_interleave(K, dim=0)
    return out


def route(M, src, sel, num_slots):
    """Convenience: the full integer routing path -> (phys, counts, offsets, pos)."""
    phys = map_logical_to_physical(M, src, sel)
    counts = histogram(phys, num_slots)
    offsets = group_offsets(counts)
    pos = scatter_index(phys)
    return phys, counts, offsets, pos


# ---------------------------------------------------------------------------
# Grouped GEMM (fp32 accumulate, bf16 store)
# ---------------------------------------------------------------------------


def _groups(offsets):
    offsets = np.asarray(offsets, dtype=np.int64)
    for g in range(offsets.size - 1):
        yield g, int(offsets[g]), int(offsets[g + 1])


def grouped_gemm_nt(a: torch.Tensor, b: torch.Tensor, offsets) -> torch.Tensor:
    """C[rows of g] = A[rows of g] @ B[g]^T, B: [G, N, K].

    ``group_gemm_same_nk(..., transpose_b=True)``
    (veomni/ops/kernels/moe/_kernels/kernel/group_gemm.py:67-247): fp32
    accumulation (``tl.dot`` into fp32), stored in the input dtype.
    """
    out = torch.zeros((a.shape[0], b.shape[1]), dtype=torch.float32)
    af = a.float()
    for g, s, e in _groups(offsets):
        if e > s:
            out[s:e] = af[s:e] @ b[g].float().t()
    return out.to(a.dtype)


def grouped_gemm_nn(a: torch.Tensor, b: torch.Tensor, offsets) -> torch.Tensor:
    """C[rows of g] = A[rows of g] @ B[g], B: [G, K, N]  (``same_nk``, transpose_b=False)."""
    out = torch.zeros((a.shape[0], b.shape[2]), dtype=torch.float32)
    af = a.float()
    for g, s, e in _groups(offsets):
        if e > s:
            out[s:e] = af[s:e] @ b[g].float()
    return out.to(a.dtype)


def grouped_gemm_tn(a: torch.Tensor, b: torch.Tensor, offsets, out_dtype=None) -> torch.Tensor:
    """C[g] = A[rows of g]^T @ B[rows of g]; zeros for empty groups.

    ``group_gemm_same_mn(..., transpose_a=True)`` (group_gemm.py:254-410); an
    empty group stores zeros (group_gemm.py:336-350).
    """
    offsets = np.asarray(offsets, dtype=np.int64)
    G = offsets.size - 1
    out = torch.zeros((G, a.shape[1], b.shape[1]), dtype=torch.float32)
    af, bf = a.float(), b.float()
    for g, s, e in _groups(offsets):
        if e > s:
            out[g] = af[s:e].t() @ bf[s:e]
    return out.to(out_dtype or a.dtype)


# ---------------------------------------------------------------------------
# SwiGLU expert MLP over per-copy groups
# ---------------------------------------------------------------------------


def silu_f32(x: torch.Tensor) -> torch.Tensor:
    return x / (1.0 + torch.exp(-x))


def swiglu_forward(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """act = bf16(bf16(silu(gate)) * up) - the two bf16 ops of
    veomni/distributed/moe/moe_layer.py:394-397 (``aten.silu`` then ``*``).
    Every rounding point here and below is the inputs' dtype (bf16, or fp16
    for fp16 tensors, as the reference's ops compute in the input dtype)."""
    dt = gate.dtype
    s = silu_f32(gate.float()).to(dt)
    return (s.float() * up.float()).to(dt)


def swiglu_backward(dact: torch.Tensor, gate: torch.Tensor, up: torch.Tensor):
    """Returns (d_gate, d_up) with the reference's bf16 rounding points
    (veomni/distributed/moe/moe_layer.py:465-482)."""
    dt = dact.dtype
    g = gate.float()
    s = silu_f32(g).to(dt).float()
    d_up = (s * dact.float()).to(dt)
    d_silu = (dact.float() * up.float()).to(dt).float()
    sig = torch.sigmoid(g)
    d_gate = (d_silu * (sig * (1.0 + g * (1.0 - sig)))).to(dt)
    return d_gate, d_up


def expert_layer_forward(xp: torch.Tensor, offsets, w1: torch.Tensor, w2: torch.Tensor):
    """``EPMergedFc1GroupGemm.forward`` (veomni/distributed/moe/moe_layer.py:358-429).

    xp [A,H] bf16, w1 = gate_up [C,2I,H], w2 = down [C,H,I].
    Returns (gate_up [A,2I], act [A,I], y [A,H]).
    """
    gu = grouped_gemm_nt(xp, w1, offsets)
    I = w1.shape[1] // 2
    act = swiglu_forward(gu[:, :I], gu[:, I:])
    y = grouped_gemm_nt(act, w2, offsets)
    return gu, act, y


def expert_layer_backward(dy, xp, gu, offsets, w1, w2):
    """``EPMergedFc1GroupGemm.backward`` (veomni/distributed/moe/moe_layer.py:431-547).

    Returns (dxp [A,H], dw1 [C,2I,H], dw2 [C,H,I], dg1 [A,2I]).
    """
    I = w1.shape[1] // 2
    act = swiglu_forward(gu[:, :I], gu[:, I:])
    dact = grouped_gemm_nn(dy, w2, offsets)
    dw2 = grouped_gemm_tn(dy, act, offsets)
    d_gate, d_up = swiglu_backward(dact, gu[:, :I], gu[:, I:])
    dg1 = torch.cat([d_gate, d_up], dim=1)
    dxp = grouped_gemm_nn(dg1, w1, offsets)
    dw1 = grouped_gemm_tn(dg1, xp, offsets)
    return dxp, dw1, dw2, dg1


# ---------------------------------------------------------------------------
# Combine (EP semantics) and its gradients
# ---------------------------------------------------------------------------


def combine_forward(y: torch.Tensor, pos, w: torch.Tensor) -> torch.Tensor:
    """out[t] = bf16( sum_k fp32( bf16(y[pos[t,k]] * w[t,k]) ) ).

    ``rank_dedup_combine`` (veomni/distributed/moe/hiermoe/all_to_all.py:2539-2564):
    bf16 product with the router weight, then the fp32 segment sum of
    ``_aggregate_weighted_outputs`` (:2266-2294) /
    ``segment_sum_dim0_fp32_to_source_dtype``
    (veomni/distributed/moe/hiermoe/triton_segment_sum.py:52-103).
    """
    pos_t = torch.as_tensor(np.asarray(pos, dtype=np.int64))
    T, K = pos_t.shape
    acc = torch.zeros((T, y.shape[1]), dtype=torch.float32)
    for k in range(K):
        rows = y[pos_t[:, k]].float()
        acc += (rows * w[:, k : k + 1].float()).to(y.dtype).float()
    return acc.to(y.dtype)


def combine_backward(dout: torch.Tensor, y: torch.Tensor, pos, w: torch.Tensor):
    """Gradients of ``combine_forward``: dy[pos[t,k]] = bf16(dout[t] * w[t,k]) and
    dw[t,k] = bf16( sum_h fp32( bf16(dout[t,h] * y[pos[t,k],h]) ) ).

    Autograd of the bf16 multiply in ``rank_dedup_combine`` (all_to_all.py:2552)
    and the exact ``index_select`` backward of the segment sum (all_to_all.py:930-933).
    """
    pos_t = torch.as_tensor(np.asarray(pos, dtype=np.int64))
    T, K = pos_t.shape
    dy = torch.empty_like(y)
    dw = torch.empty((T, K), dtype=w.dtype)
    d = dout.float()
    for k in range(K):
        rows = y[pos_t[:, k]].float()
        dy[pos_t[:, k]] = (d * w[:, k : k + 1].float()).to(y.dtype)
        dw[:, k] = (d * rows).to(y.dtype).float().sum(dim=1).to(w.dtype)
    return dy, dw


def unpermute_grad(dxp: torch.Tensor, pos) -> torch.Tensor:
    """dx[t] = bf16( sum_k fp32(dxp[pos[t,k]]) )  (``moe_gather``, moe.py:85-159)."""
    pos_t = torch.as_tensor(np.asarray(pos, dtype=np.int64))
    T, K = pos_t.shape
    acc = torch.zeros((T, dxp.shape[1]), dtype=torch.float32)
    for k in range(K):
        acc += dxp[pos_t[:, k]].float()
    return acc.to(dxp.dtype)


def segment_sum(source: torch.Tensor, index, num_rows: int) -> torch.Tensor:
    """out[r] = sum_{i: index[i]==r} source[i] in fp32, stored in source dtype
    (triton_segment_sum.py:52-103)."""
    index_t = torch.as_tensor(np.asarray(index, dtype=np.int64))
    if index_t.numel() and (int(index_t.min()) < 0 or int(index_t.max()) >= num_rows):
        raise ValueError("index contains a row outside [0, num_rows).")
    out = torch.zeros((num_rows, source.shape[1]), dtype=torch.float32)
    out.index_add_(0, index_t, source.float())
    return out.to(source.dtype)


# ---------------------------------------------------------------------------
# Replica-gradient fold
# ---------------------------------------------------------------------------


def copy_groups(slot_to_logical, num_experts):
    """Copies of each logical expert in slot order (``redundant_copy_groups``,
    expert_swap.py:552-572; ``copy_slots_for_device`` :520-550)."""
    L = np.asarray(slot_to_logical, dtype=np.int64)
    return [[int(c) for c in np.nonzero(L == e)[0]] for e in range(num_experts)]


def replica_fold(grads: torch.Tensor, slot_to_logical, num_experts: int, slot_counts=None) -> torch.Tensor:
    """dW_logical[e] = sum_{c : L[c]==e} dW[c] in fp32.

    ``_replica_grad_contributions`` (expert_swap.py:6839-6876) sums the copies of
    each expert; slots with no accumulated tokens are zeroed first
    (``_zero_inactive_slot_grads_for_layer``, expert_swap.py:6250-6262).  The sum
    here is in fp32 (the reference sums in the gradient dtype).
    """
    C = grads.shape[0]
    flat = grads.reshape(C, -1).float()
    active = np.ones(C, dtype=bool) if slot_counts is None else (np.asarray(slot_counts) > 0)
    out = torch.zeros((num_experts, flat.shape[1]), dtype=torch.float32)
    for e, slots in enumerate(copy_groups(slot_to_logical, num_experts)):
        for c in slots:
            if active[c]:
                out[e] += flat[c]
    return out.reshape((num_experts,) + tuple(grads.shape[1:]))


# ---------------------------------------------------------------------------
# Whole layer (one GPU's share)
# ---------------------------------------------------------------------------


def moe_layer_forward(x, w, phys, w1, w2):
    """Forward of the full path for already-mapped ``phys``; returns a dict of
    every intermediate the backward needs."""
    C = w1.shape[0]
    counts = histogram(phys, C)
    offsets = group_offsets(counts)
    pos = scatter_index(phys)
    xp = permute(x, pos)
    gu, act, y = expert_layer_forward(xp, offsets, w1, w2)
    out = combine_forward(y, pos, w)
    return dict(counts=counts, offsets=offsets, pos=pos, xp=xp, gu=gu, act=act, y=y, out=out)


def moe_layer_backward(dout, fwd, w, w1, w2):
    dy, dw = combine_backward(dout, fwd["y"], fwd["pos"], w)
    dxp, dw1, dw2, dg1 = expert_layer_backward(dy, fwd["xp"], fwd["gu"], fwd["offsets"], w1, w2)
    dx = unpermute_grad(dxp, fwd["pos"])
    return dict(dy=dy, dw=dw, dxp=dxp, dw1=dw1, dw2=dw2, dg1=dg1, dx=dx)


# ---------------------------------------------------------------------------
# Router weight on the fc2 input (the reference's non-EP branch)
# ---------------------------------------------------------------------------


def row_weights(w: torch.Tensor, pos) -> torch.Tensor:
    """scattered_gate_weight[scatter_index.flatten()] = gate_weights.reshape(-1)
    (veomni/ops/kernels/moe/group_gemm.py:269-272, :494-497): each permuted
    row's router weight."""
    pos_t = torch.as_tensor(np.asarray(pos, dtype=np.int64)).reshape(-1)
    out = torch.empty(pos_t.numel(), dtype=w.dtype)
    out[pos_t] = w.reshape(-1)
    return out


def weight_rows(act: torch.Tensor, row_w: torch.Tensor) -> torch.Tensor:
    """fc1_weighted_output = fc1_activation * scattered_gate_weight, a bf16
    product (group_gemm.py:276, :499)."""
    return (act.float() * row_w.float()[:, None]).to(act.dtype)


def swiglu_backward_weighted(d_act_w: torch.Tensor, gu: torch.Tensor, act: torch.Tensor, row_w: torch.Tensor):
    """The router weight's backward and the SwiGLU backward of the non-EP
    branch (group_gemm.py:577-592; split :365-406), returning (dg1 [R,2I],
    dw_row [R]):
    grad_fc1_activation = bf16(d_act_w * w), grad_scattered_gate_weight =
    bf16(sum_j fp32(bf16(act * d_act_w))) (``torch.sum`` of a bf16 product),
    then silu_backward and the up-projection product as in the EP branch."""
    I = act.shape[1]
    dt = d_act_w.dtype
    dact = (d_act_w.float() * row_w.float()[:, None]).to(dt)
    dw_row = (act.float() * d_act_w.float()).to(dt).float().sum(dim=1).to(row_w.dtype)
    d_gate, d_up = swiglu_backward(dact, gu[:, :I], gu[:, I:])
    return torch.cat([d_gate, d_up], dim=1), dw_row


def moe_layer_forward_weighted_input(x, w, phys, w1, w2):
    """``MergedFc1TritonFusedMoeExpertFunction.forward`` (group_gemm.py:458-531)
    for already-mapped ``phys``: the router weight multiplies the fc2 input and
    ``moe_gather`` sums a token's rows unweighted."""
    C = w1.shape[0]
    counts = histogram(phys, C)
    offsets = group_offsets(counts)
    pos = scatter_index(phys)
    xp = permute(x, pos)
    gu = grouped_gemm_nt(xp, w1, offsets)
    I = w1.shape[1] // 2
    act = swiglu_forward(gu[:, :I], gu[:, I:])
    row_w = row_weights(w, pos)
    act_w = weight_rows(act, row_w)
    y = grouped_gemm_nt(act_w, w2, offsets)
    out = unpermute_grad(y, pos)
    return dict(counts=counts, offsets=offsets, pos=pos, xp=xp, gu=gu, act=act, row_w=row_w, act_w=act_w, y=y,
                out=out)


def moe_layer_backward_weighted_input(dout, fwd, w, w1, w2):
    """``MergedFc1TritonFusedMoeExpertFunction.backward`` (group_gemm.py:533-629):
    grad_fc2_output = moe_scatter(grad_output), its dgrad through fc2, the
    router weight's backward, fc1 as in the EP branch, ``moe_gather``."""
    pos, offsets = fwd["pos"], fwd["offsets"]
    dyp = permute(dout, pos)
    d_act_w = grouped_gemm_nn(dyp, w2, offsets)
    dw2 = grouped_gemm_tn(dyp, fwd["act_w"], offsets)
    dg1, dw_row = swiglu_backward_weighted(d_act_w, fwd["gu"], fwd["act"], fwd["row_w"])
    pos_t = torch.as_tensor(np.asarray(pos, dtype=np.int64)).reshape(-1)
    dw = dw_row[pos_t].reshape(w.shape)
    dxp = grouped_gemm_nn(dg1, w1, offsets)
    dw1 = grouped_gemm_tn(dg1, fwd["xp"], offsets)
    dx = unpermute_grad(dxp, pos)
    return dict(dyp=dyp, d_act_w=d_act_w, dg1=dg1, dw_row=dw_row, dw=dw, dxp=dxp, dw1=dw1, dw2=dw2, dx=dx)


# ---------------------------------------------------------------------------
# Route statistics for the placement planner
# ---------------------------------------------------------------------------


def route_statistics(samples, num_experts: int):
    """Source-conditioned demand [S, E] and co-selection affinity [S, E, E]
    (float64) of routing samples, ``profile_route_statistics``
    (veomni/distributed/moe/hiermoe/placemoe/statistics.py:30-64): demand is
    the bincount of each source's routes; every unordered pair of top-k
    positions adds one to (a, b) and to (b, a); the diagonal is zeroed.

    ``samples``: a list of samples, each a list (one per source rank) of
    integer arrays [tokens, top_k]."""
    S = len(samples[0])
    demand = np.zeros((S, num_experts), dtype=np.float64)
    affinity = np.zeros((S, num_experts, num_experts), dtype=np.float64)
    for sample in samples:
        for s, route in enumerate(sample):
            route = np.asarray(route, dtype=np.int64)
            demand[s] += np.bincount(route.reshape(-1), minlength=num_experts)
            K = route.shape[1]
            for a in range(K):
                for b in range(a + 1, K):
                    pair = route[:, a] * num_experts + route[:, b]
                    counts = np.bincount(pair, minlength=num_experts * num_experts).reshape(num_experts, num_experts)
                    affinity[s] += counts + counts.T
    for m in affinity:
        np.fill_diagonal(m, 0.0)
    return demand, affinity


# ---------------------------------------------------------------------------
# Expert-parallel payloads (per-rank halves around the all-to-all)
# ---------------------------------------------------------------------------


def build_local_payload(hidden: torch.Tensor, phys, weights: torch.Tensor, num_slots: int, ep_size: int) -> dict:
    """``_build_local_payload`` (veomni/distributed/moe/hiermoe/all_to_all.py:979-1055):
    assignments keyed by (target rank, token), sorted, deduplicated with
    ``unique_consecutive``; one hidden row per key, one metadata row
    (ordinal of the key within its rank, local slot, token) and weight per
    assignment.  The reference sorts with an unstable argsort; here the sort
    is stable (ties keep k order), one of the orders it may produce."""
    phys = np.asarray(phys, dtype=np.int64)
    T, K = phys.shape
    L = num_slots // ep_size
    flat = phys.reshape(-1)
    ranks = flat // L
    tokens = np.repeat(np.arange(T, dtype=np.int64), K)
    stride = max(1, T)
    keys = ranks * stride + tokens
    order = np.argsort(keys, kind="stable")
    skeys = keys[order]
    change = np.ones(skeys.size, dtype=bool)
    change[1:] = skeys[1:] != skeys[:-1]
    inverse = np.cumsum(change) - 1
    ukeys = skeys[change]
    uranks = ukeys // stride
    utokens = ukeys - uranks * stride
    usplits = np.bincount(uranks, minlength=ep_size)
    uoffsets = np.concatenate([[0], np.cumsum(usplits)[:-1]])
    ordinal = (np.arange(ukeys.size) - uoffsets[uranks])[inverse]
    meta = np.stack([ordinal, flat[order] - ranks[order] * L, tokens[order]], axis=1).astype(np.int32)
    w = weights.reshape(-1)[torch.as_tensor(order)]
    return {
        "send_hidden": hidden[torch.as_tensor(utokens)],
        "send_meta": meta,
        "send_weights": w.reshape(-1, 1),
        "unique_tokens": utokens,
        "unique_send_splits": usplits.tolist(),
        "assignment_send_splits": np.bincount(ranks, minlength=ep_size).tolist(),
        "target_ranks": ranks.reshape(T, K),
    }


def aggregate_weighted_outputs(weighted: torch.Tensor, source_tokens, split_sizes, key_stride=None):
    """``_aggregate_weighted_outputs`` (all_to_all.py:2266-2294): rows keyed by
    (source rank, token) in receive order, ``unique_consecutive`` runs summed
    with an fp32 ``index_add`` and cast back; returns (sums, runs per rank)."""
    if weighted.numel() == 0:
        return weighted[:0], []
    src_ranks = np.repeat(np.arange(len(split_sizes)), split_sizes)
    tokens = np.asarray(source_tokens, dtype=np.int64)
    stride = max(1, int(key_stride) if key_stride is not None else tokens.size + 1)
    keys = src_ranks * stride + tokens
    change = np.ones(keys.size, dtype=bool)
    change[1:] = keys[1:] != keys[:-1]
    inverse = torch.as_tensor(np.cumsum(change) - 1)
    ukeys = keys[change]
    acc = torch.zeros((ukeys.size, weighted.shape[1]), dtype=torch.float32)
    acc.index_add_(0, inverse, weighted.float())
    return acc.to(weighted.dtype), np.bincount(ukeys // stride, minlength=len(split_sizes)).tolist()


# ---------------------------------------------------------------------------
# Cross-rank replica-gradient exchange (all ranks simulated in one process)
# ---------------------------------------------------------------------------


def replica_grad_schedule(slot_to_logical, logical_to_physical, num_local: int, ep_rank: int, ep_size: int):
    """``_replica_grad_schedule_for_layer`` (expert_swap.py:6797-6837) over
    ``redundant_copy_groups`` (:552-572), owners from
    ``_owner_rank_for_copy_group`` (:6541-6555).  Returns a dict with
    ``groups`` = [(logical, owner_rank, copy_ranks, local_slots)], ``pairwise``
    and ``globally_ordered_pairs``."""
    L = np.asarray(slot_to_logical, dtype=np.int64)
    owners = np.asarray(logical_to_physical, dtype=np.int64)
    active = L[L >= 0]
    counts = np.bincount(active, minlength=owners.size) if active.size else np.zeros(owners.size, np.int64)
    groups = []
    for e in np.nonzero(counts > 1)[0]:
        slots = [int(s) for s in np.nonzero(L == e)[0]]
        owner_slot = int(owners[e])
        if owner_slot not in slots:
            raise RuntimeError(f"HierMoE owner slot {owner_slot} for logical expert {int(e)} is not in its copy group.")
        copy_ranks = tuple(sorted({s // num_local for s in slots}))
        local = tuple(s % num_local for s in slots if s // num_local == ep_rank)
        groups.append((int(e), owner_slot // num_local, copy_ranks, local))
    pairwise = all(len(g[2]) <= 2 for g in groups)
    neighbors = [set() for _ in range(ep_size)]
    if pairwise:
        for _, _, ranks, _ in groups:
            if len(ranks) == 2:
                a, b = ranks
                neighbors[a].add(b)
                neighbors[b].add(a)
    ordered = pairwise and any(len(n) > 1 for n in neighbors)
    return {"groups": groups, "pairwise": pairwise, "globally_ordered_pairs": ordered}


def replica_grad_sync(rank_grads, slot_to_logical, logical_to_physical, num_local: int):
    """``sync_redundant_gradients`` (expert_swap.py:7220-7252) of every rank at
    once.  ``rank_grads[r]`` is the tuple of rank r's copy gradients (one
    tensor [num_local, ...] per parameter, gate_up then down); returns new
    tuples.  Arithmetic follows the reference in the gradient dtype: local
    sums by ``clone`` + ``add_`` in slot order (:6839-6876); pairwise totals
    ``local_sum + remote`` (:7038-7107); owner totals ``local_sum`` plus each
    source's part in the order the owner's receive list first meets the
    source ranks (:7109-7217); every local copy then takes the total
    (``_unpack_replica_grad``, :6886-6889)."""
    R = len(rank_grads)
    out = [tuple(g.clone() for g in grads) for grads in rank_grads]
    scheds = [replica_grad_schedule(slot_to_logical, logical_to_physical, num_local, r, R) for r in range(R)]
    pairwise = scheds[0]["pairwise"]
    # The owner's receive dict meets source ranks group by group, in rank order.
    peer_order = {r: [] for r in range(R)}
    for _, owner, ranks, _ in scheds[0]["groups"]:
        for q in ranks:
            if q != owner and q not in peer_order[owner]:
                peer_order[owner].append(q)

    def local_sum(r, slots, p):
        s = rank_grads[r][p][slots[0]].clone()
        for c in slots[1:]:
            s.add_(rank_grads[r][p][c])
        return s

    for gi, (e, owner, ranks, _) in enumerate(scheds[0]["groups"]):
        local = {r: scheds[r]["groups"][gi][3] for r in ranks}
        for p in range(len(rank_grads[0])):
            sums = {r: local_sum(r, local[r], p) for r in ranks}
            if pairwise:
                totals = {r: sums[r] + sums[q] for r in ranks for q in ranks if q != r} if len(ranks) == 2 \
                    else {r: sums[r] for r in ranks}
            else:
                total = sums[owner].clone()
                for src in sorted((q for q in ranks if q != owner), key=peer_order[owner].index):
                    total.add_(sums[src])
                totals = {r: total for r in ranks}
            for r in ranks:
                for c in local[r]:
                    out[r][p][c].copy_(totals[r])
    return out


def owner_grad_norm_mask(logical_to_physical, num_local: int, ep_rank: int):
    """``redundant_grad_norm_masks`` (expert_swap.py:7254-7266): True at the
    local slots of this rank that are the runtime owner of their expert."""
    mask = np.zeros(num_local, dtype=bool)
    for s in np.asarray(logical_to_physical, dtype=np.int64):
        if s // num_local == ep_rank:
            mask[s % num_local] = True
    return mask
