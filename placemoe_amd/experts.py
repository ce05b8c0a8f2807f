"""Autograd functions for one GPU's share of the PlaceMoE expert layer.

Forward:  route (M table -> histogram -> scan -> stable scatter index) ->
permute -> fc1 + SwiGLU -> fc2 -> router-weighted combine.
Backward: combine gradient -> fc2 dgrad + SwiGLU backward -> fc2 wgrad ->
fc1 dgrad -> fc1 wgrad -> unpermute gradient.
With top-1 routing the combine runs in fc2's epilogue and the unpermute
gradient in the fc1 dgrad's (bit-identical; ``set_top1_fusion``).

Every step is a gfx950 kernel of ``libplacemoe_amd.so``; no step has a torch
or CPU fallback.  The composition follows the reference's EP + PlaceMoE
branch of ``group_gemm_fused_moe_forward``
(veomni/ops/kernels/moe/group_gemm.py:669-857): ``M`` gather
(``map_logical_to_physical``, veomni/distributed/moe/hiermoe/expert_swap.py:5831-5879),
per-copy contiguous rows, ``EPMergedFc1GroupGemm`` / ``EPGroupGemm``
(veomni/distributed/moe/moe_layer.py:147-547), router weights applied in the
combine (``rank_dedup_combine``, veomni/distributed/moe/hiermoe/all_to_all.py:2539-2564).

``weighted_input=True`` gives the arithmetic of the reference's non-EP
branch instead (``TritonFusedMoeExpertFunction`` /
``MergedFc1TritonFusedMoeExpertFunction``, group_gemm.py:210-631): each row's
SwiGLU output is multiplied by its router weight before fc2, the top-k rows
of a token are summed unweighted (``moe_gather``), and the backward takes the
router-weight gradient from the fc2 input side.  The two agree in exact
arithmetic and differ in bf16 rounding.
"""

from __future__ import annotations

import os

import torch

from . import kernels

# Route checks whose status copy has not been looked at yet.  The op never
# waits for one: each forward and backward polls them (an event query) and
# raises for the first that has landed and reports an invalid id; a check
# whose copy is still in flight stays here for the next poll.
_PENDING_CHECKS: list = []


def _sync_route_checks() -> bool:
    """PLACEMOE_AMD_CHECK_ROUTES=1: check every forward's routing on the spot
    (one stream synchronisation per call)."""
    return os.environ.get("PLACEMOE_AMD_CHECK_ROUTES", "0") not in ("", "0")


def check_pending_routes(block: bool = False) -> None:
    """Raise ``ValueError`` if a routing call whose status has landed flagged
    an invalid expert or source id.  ``block=True`` first waits for every
    pending status copy (a host synchronisation: for the end of a step or a
    test); the default only looks at copies that have already landed."""
    if block:
        for check in _PENDING_CHECKS:
            if not check.checked:
                check.raise_if_failed()
    _poll_pending_checks()


# Backward GEMM pairs that do not depend on each other (fc2 dgrad and fc2
# wgrad; fc1 dgrad and fc1 wgrad) can run on two streams, so that the tail of
# one persistent GEMM (its last, partly filled round of tiles) runs beside
# the other's blocks.  That pays off for short GEMMs and costs for long ones,
# whose weight gradient deals its tiles to blocks assuming they all start
# together (measured, layer fwd+bwd: Qwen3-30B-A3B shape, A*H*I = 2.1e11,
# 4.80 -> 4.73 ms and with the replica fold 6.57 -> 6.49 ms; DeepSeek-V3
# shape, 9.6e11, 15.70 -> 16.26 ms; skewed 96-copy shape, 8.3e11, 15.33 ->
# 15.62 ms).  By default (None) the two streams are used when
# rows * H * I < _OVERLAP_MAX_WORK.  Streams keep the default priority.
_OVERLAP = None
_OVERLAP_MAX_WORK = 4e11
_SIDE_STREAMS: dict = {}


def set_backward_overlap(enabled: bool | None) -> bool | None:
    """Run the backward's independent GEMM pairs on two streams (True), all
    on the caller's stream (False), or choose by GEMM size (None, the
    default); returns the previous setting."""
    global _OVERLAP
    prev, _OVERLAP = _OVERLAP, (None if enabled is None else bool(enabled))
    return prev


def uses_backward_overlap(rows: int, hidden: int, inter: int) -> bool:
    """Whether the backward of a layer with `rows` received rows, hidden size
    and intermediate size runs its independent GEMM pairs on two streams."""
    if _OVERLAP is not None:
        return _OVERLAP
    return rows * hidden * inter < _OVERLAP_MAX_WORK


# Top-1 layers (every token routed to one copy) fold two row kernels into
# GEMM epilogues: the router-weighted combine into fc2 (which then writes the
# layer output beside Y) and the unpermute gradient into the fc1 dgrad (which
# writes each row straight to its token); the combine gradient walks the rows
# in their storage order.  Results are bit-identical to the separate kernels.
_TOP1_FUSION = True


def set_top1_fusion(enabled: bool) -> bool:
    """Fold the combine and the unpermute gradient of top-1 layers into the
    fc2 and fc1-dgrad GEMMs (default) or run them as separate kernels;
    returns the previous setting."""
    global _TOP1_FUSION
    prev, _TOP1_FUSION = _TOP1_FUSION, bool(enabled)
    return prev


def _side_stream(device: torch.device) -> torch.cuda.Stream:
    s = _SIDE_STREAMS.get(device)
    if s is None:
        s = torch.cuda.Stream(device=device)
        _SIDE_STREAMS[device] = s
    return s


def _poll_pending_checks() -> None:
    """Look at every pending check whose copy has landed (no waiting); the
    first that failed raises.  Checks still in flight are kept."""
    keep = []
    failed = None
    for check in _PENDING_CHECKS:
        if check.checked:
            continue
        if check.ready():
            check.checked = True
            if failed is None and check.failed():
                failed = check
        else:
            keep.append(check)
    _PENDING_CHECKS[:] = keep
    if failed is not None:
        failed.raise_if_failed()


class _ExpertLayerBase(torch.autograd.Function):
    """Shared forward/backward; subclasses fix how fc1 weights are passed."""

    @staticmethod
    def _forward(ctx, hidden, routing_weights, selected, mapping, sources, source, w_gate, w_up, copy_stride,
                 fc2_weight, split, recorder, weighted_input):
        T, H = hidden.shape
        C, H2, inter = fc2_weight.shape
        assert H2 == H, f"down_proj hidden size {H2} != hidden size {H}"
        # fc1 must describe the same C copies, hidden size and intermediate size as fc2.
        # bf16 or fp16 throughout: the weights in the hidden states' dtype
        assert hidden.dtype in (torch.bfloat16, torch.float16), (
            f"hidden states must be bfloat16 or float16, got {hidden.dtype}"
        )
        assert w_gate.dtype == hidden.dtype and w_up.dtype == hidden.dtype, (
            f"fc1 weights must be {hidden.dtype} like the hidden states, got {w_gate.dtype}/{w_up.dtype}"
        )
        assert fc2_weight.dtype == hidden.dtype, f"fc2 weight must be {hidden.dtype}, got {fc2_weight.dtype}"
        fc1_shape = (C, inter, H) if split else (C, 2 * inter, H)
        assert tuple(w_gate.shape) == fc1_shape, (
            f"fc1 weight shape {tuple(w_gate.shape)} does not match fc2 {tuple(fc2_weight.shape)} "
            f"and hidden size {H} (expected {fc1_shape})"
        )
        _poll_pending_checks()
        r = kernels.route(selected, C, mapping=mapping, sources=sources, source=source)
        # Invalid expert or source ids are clamped on the device and flagged in
        # the routing status word.  Its copy is checked without a host sync:
        # by the backward if it has landed by then, else by a later forward or
        # backward (or check_pending_routes).
        check = kernels.RouteCheck(r)
        if _sync_route_checks():
            check.raise_if_failed()
        else:
            _PENDING_CHECKS.append(check)
        if recorder is not None:
            recorder(r.counts)
        ctx.split = split
        ctx.inter = inter
        ctx.routing = r
        ctx.weighted_input = weighted_input
        if weighted_input:
            # group_gemm.py:473-511: fc1_weighted_output = fc1_activation *
            # scattered_gate_weight feeds fc2; moe_gather sums a token's rows.
            xp, row_src, row_w = kernels.moe_scatter_src(hidden, r.pos, routing_weights)
            gu, act = kernels.gemm_fc1_swiglu(xp, w_gate, w_up, copy_stride, r.offsets, C, inter)
            act_w = kernels.weight_rows(act, row_w)
            y = kernels.group_gemm_nt(act_w, fc2_weight, r.offsets)
            out = kernels.moe_gather(y, r.pos)
            ctx.save_for_backward(xp, gu, act, act_w, r.pos, r.offsets, routing_weights, w_gate, w_up, fc2_weight,
                                  row_src, row_w)
            return out
        row_src = None
        if r.pos.shape[1] == 1 and _TOP1_FUSION:
            xp, row_src, row_w = kernels.moe_scatter_src(hidden, r.pos, routing_weights)
        else:
            xp = kernels.moe_scatter(hidden, r.pos)
        gu, act = kernels.gemm_fc1_swiglu(xp, w_gate, w_up, copy_stride, r.offsets, C, inter)
        if row_src is not None:
            y, out = kernels.group_gemm_nt_combine_top1(act, fc2_weight, r.offsets, row_src, row_w)
        else:
            y = kernels.group_gemm_nt(act, fc2_weight, r.offsets)
            out = kernels.combine_fwd(y, r.pos, routing_weights)
        ctx.save_for_backward(xp, gu, act, y, r.pos, r.offsets, routing_weights, w_gate, w_up, fc2_weight, row_src)
        return out

    @staticmethod
    def _backward(ctx, grad_out):
        _poll_pending_checks()
        if ctx.weighted_input:
            return _ExpertLayerBase._backward_weighted_input(ctx, grad_out)
        xp, gu, act, y, pos, offsets, w, w_gate, w_up, fc2_weight, row_src = ctx.saved_tensors
        grad_out = grad_out.contiguous()
        need_w, need_x = ctx.needs_input_grad[1], ctx.needs_input_grad[0]
        if row_src is not None and y.shape[1] % 8 == 0 and grad_out.data_ptr() % 16 == 0 and y.data_ptr() % 16 == 0:
            # top-1: the combine gradient walked in the rows' storage order
            # (bit-identical to combine_bwd, faster: Y read and dY written in order)
            dy, dw = kernels.combine_bwd_top1_rows(grad_out, y, row_src, w)
        else:
            dy, dw = kernels.combine_bwd(grad_out, y, pos, w)
        main = torch.cuda.current_stream(dy.device)
        side = _side_stream(dy.device) if uses_backward_overlap(dy.shape[0], dy.shape[1], ctx.inter) else main
        # The weight gradients go to the side stream, each after the main
        # stream has produced its inputs; the dgrads stay on the main stream.
        d_fc2 = d_fc1 = None
        if ctx.fc2_needs_grad:
            side.wait_stream(main)
            with torch.cuda.stream(side):
                d_fc2 = kernels.group_gemm_tn(dy, act, offsets)
        dg1 = kernels.gemm_fc2_dgrad_swiglu(dy, fc2_weight, gu, offsets)
        if ctx.fc1_needs_grad:
            side.wait_stream(main)
            with torch.cuda.stream(side):
                d_fc1 = kernels.group_gemm_tn(dg1, xp, offsets, split=ctx.inter if ctx.split else None)
        dx = None
        if need_x:
            # Merged weights: w_gate is the whole [C, 2I, H] gate_up_proj.
            b_second = w_up if ctx.split else None
            if row_src is not None:
                dx = kernels.group_gemm_nn_unpermute_top1(dg1, w_gate, offsets, row_src, b_second=b_second)
            else:
                dxp = kernels.group_gemm_nn(dg1, w_gate, offsets, b_second=b_second)
                dx = kernels.moe_gather(dxp, pos)
        if side is not main:
            # The caller's stream waits for the weight gradients, which were
            # allocated on the side stream and are used on the caller's.
            main.wait_stream(side)
            for t in (d_fc2, *(d_fc1 if isinstance(d_fc1, tuple) else (d_fc1,))):
                if t is not None:
                    t.record_stream(main)
        return dx, (dw if need_w else None), d_fc1, d_fc2

    @staticmethod
    def _backward_weighted_input(ctx, grad_out):
        """group_gemm.py:533-629: grad_fc2_output = moe_scatter(grad_output);
        its dgrad through fc2, then the router weight's backward with the
        SwiGLU backward in one row kernel; fc1 as in the EP branch."""
        xp, gu, act, act_w, pos, offsets, w, w_gate, w_up, fc2_weight, row_src, row_w = ctx.saved_tensors
        grad_out = grad_out.contiguous()
        need_w, need_x = ctx.needs_input_grad[1], ctx.needs_input_grad[0]
        dyp = kernels.moe_scatter(grad_out, pos)
        main = torch.cuda.current_stream(dyp.device)
        side = _side_stream(dyp.device) if uses_backward_overlap(dyp.shape[0], dyp.shape[1], ctx.inter) else main
        d_fc2 = d_fc1 = None
        if ctx.fc2_needs_grad:
            side.wait_stream(main)
            with torch.cuda.stream(side):
                d_fc2 = kernels.group_gemm_tn(dyp, act_w, offsets)
        d_act_w = kernels.group_gemm_nn(dyp, fc2_weight, offsets)
        dg1, dw = kernels.swiglu_bwd_weighted(d_act_w, gu, act, row_w, row_src, pos.numel())
        if ctx.fc1_needs_grad:
            side.wait_stream(main)
            with torch.cuda.stream(side):
                d_fc1 = kernels.group_gemm_tn(dg1, xp, offsets, split=ctx.inter if ctx.split else None)
        dx = None
        if need_x:
            b_second = w_up if ctx.split else None
            if pos.shape[1] == 1 and _TOP1_FUSION:
                # top-1: row_src[r] is row r's token
                dx = kernels.group_gemm_nn_unpermute_top1(dg1, w_gate, offsets, row_src, b_second=b_second)
            else:
                dxp = kernels.group_gemm_nn(dg1, w_gate, offsets, b_second=b_second)
                dx = kernels.moe_gather(dxp, pos)
        if side is not main:
            main.wait_stream(side)
            for t in (d_fc2, *(d_fc1 if isinstance(d_fc1, tuple) else (d_fc1,))):
                if t is not None:
                    t.record_stream(main)
        return dx, (dw.view(w.shape) if need_w else None), d_fc1, d_fc2


class HipMergedFc1ExpertLayer(_ExpertLayerBase):
    """Merged ``gate_up_proj`` [C, 2I, H] (``EPMergedFc1GroupGemm`` layout)."""

    @staticmethod
    def forward(ctx, hidden, routing_weights, selected, mapping, sources, source, fc1_1_2_weight, fc2_weight,
                recorder=None, weighted_input=False):
        C, two_i, H = fc1_1_2_weight.shape
        assert two_i % 2 == 0, f"Merged fc1_1_2_weight dim 1 must be even, got {two_i}"
        inter = two_i // 2
        assert fc1_1_2_weight.is_contiguous() and fc2_weight.is_contiguous(), "Noncontiguous weights"
        w_up = fc1_1_2_weight.view(-1)[inter * H:]
        ctx.fc1_needs_grad = ctx.needs_input_grad[6]
        ctx.fc2_needs_grad = ctx.needs_input_grad[7]
        return _ExpertLayerBase._forward(
            ctx, hidden, routing_weights, selected, mapping, sources, source, fc1_1_2_weight, w_up,
            2 * inter * H, fc2_weight, False, recorder, weighted_input,
        )

    @staticmethod
    def backward(ctx, grad_out):
        dx, dw, d_fc1, d_fc2 = _ExpertLayerBase._backward(ctx, grad_out)
        return dx, dw, None, None, None, None, d_fc1, d_fc2, None, None


class HipSplitFc1ExpertLayer(_ExpertLayerBase):
    """Split ``fc1_1`` (gate) and ``fc1_2`` (up) [C, I, H] (``EPGroupGemm`` layout)."""

    @staticmethod
    def forward(ctx, hidden, routing_weights, selected, mapping, sources, source, fc1_1_weight, fc1_2_weight,
                fc2_weight, recorder=None, weighted_input=False):
        C, inter, H = fc1_1_weight.shape
        assert fc1_2_weight.shape == fc1_1_weight.shape, "fc1_1 and fc1_2 shapes differ"
        assert fc1_1_weight.is_contiguous() and fc1_2_weight.is_contiguous() and fc2_weight.is_contiguous(), (
            "Noncontiguous weights"
        )
        ctx.fc1_needs_grad = ctx.needs_input_grad[6] or ctx.needs_input_grad[7]
        ctx.fc2_needs_grad = ctx.needs_input_grad[8]
        return _ExpertLayerBase._forward(
            ctx, hidden, routing_weights, selected, mapping, sources, source, fc1_1_weight, fc1_2_weight,
            inter * H, fc2_weight, True, recorder, weighted_input,
        )

    @staticmethod
    def backward(ctx, grad_out):
        dx, dw, d_fc1, d_fc2 = _ExpertLayerBase._backward(ctx, grad_out)
        d_gate, d_up = d_fc1 if d_fc1 is not None else (None, None)
        return dx, dw, None, None, None, None, d_gate, d_up, d_fc2, None, None


def expert_layer(
    hidden: torch.Tensor,
    routing_weights: torch.Tensor,
    selected_experts: torch.Tensor,
    fc2_weight: torch.Tensor,
    fc1_1_2_weight: torch.Tensor | None = None,
    fc1_1_weight: torch.Tensor | None = None,
    fc1_2_weight: torch.Tensor | None = None,
    mapping: torch.Tensor | None = None,
    sources: torch.Tensor | None = None,
    source: int = 0,
    recorder=None,
    weighted_input: bool = False,
) -> torch.Tensor:
    """The full layer on one GPU: [T, H] -> [T, H], differentiable in hidden,
    routing weights and the expert weights.

    ``mapping`` [S, E] maps (source, logical expert) to a physical copy (slot)
    of ``fc2_weight.shape[0]`` copies; None means slot == logical expert.
    ``recorder(counts)`` receives the int32 per-copy token counts (on the device).
    ``weighted_input``: apply the router weights to the fc2 input (the
    reference's non-EP arithmetic) instead of in the combine (EP).
    """
    if fc1_1_2_weight is not None:
        if fc1_1_weight is not None or fc1_2_weight is not None:
            raise ValueError("Provide either split fc1 weights or merged fc1_1_2_weight, not both.")
        return HipMergedFc1ExpertLayer.apply(
            hidden, routing_weights, selected_experts, mapping, sources, source, fc1_1_2_weight, fc2_weight,
            recorder, bool(weighted_input),
        )
    if fc1_1_weight is None or fc1_2_weight is None:
        raise ValueError("Split fc1 mode requires both fc1_1_weight and fc1_2_weight.")
    return HipSplitFc1ExpertLayer.apply(
        hidden, routing_weights, selected_experts, mapping, sources, source, fc1_1_weight, fc1_2_weight, fc2_weight,
        recorder, bool(weighted_input),
    )
