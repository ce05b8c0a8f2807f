"""Rank-deduplicated expert-parallel payloads: the per-rank halves of
PlaceMoE's dispatch and combine around the all-to-all, on the GPU.

``build_local_payload`` mirrors ``_build_local_payload``
(veomni/distributed/moe/hiermoe/all_to_all.py:979-1055): it returns the same
seven values - ``(send_hidden, send_meta, send_weights, unique_tokens,
unique_send_splits, assignment_send_splits, target_ranks)`` - computed by
``pmx_ep_dispatch_payload``.  ``aggregate_weighted_outputs`` mirrors
``_aggregate_weighted_outputs`` (:2266-2294) and ``combine_aggregate`` fuses
it with the unsort and weighting of ``rank_dedup_combine`` (:2553-2556),
both through ``pmx_ep_combine_aggregate``.  The split lists are host lists,
as in the reference (one device-to-host copy of the counts per call); the
all-to-all between ranks is outside this module.
"""

from __future__ import annotations

import ctypes

import torch

from . import _capi

BF16 = torch.bfloat16
HALF = (torch.bfloat16, torch.float16)


def _stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def build_local_payload(hidden_states: torch.Tensor, selected_experts: torch.Tensor, routing_weights: torch.Tensor,
                        num_experts: int, ep_size: int, physical_experts: torch.Tensor | None = None):
    """Dispatch payload of this rank for ``ep_size`` ranks holding
    ``num_experts // ep_size`` slots each; ``physical_experts`` (copy slots)
    replace ``selected_experts`` for the routing when given."""
    assert hidden_states.is_cuda, "placemoe_amd kernels need GPU tensors"
    assert hidden_states.dtype in HALF, f"hidden_states must be bfloat16 or float16, got {hidden_states.dtype}"
    dt = hidden_states.dtype  # the payload copies 16-bit patterns: either type
    device = hidden_states.device
    num_local = num_experts // ep_size
    if num_local <= 0:
        raise ValueError("num_experts must be at least ep_size")
    if selected_experts.ndim == 1:
        selected_experts = selected_experts.unsqueeze(-1)
        routing_weights = routing_weights.unsqueeze(-1)
    routed = selected_experts if physical_experts is None else physical_experts
    if routed.ndim == 1:
        routed = routed.unsqueeze(-1)
    T, K = int(routed.shape[0]), int(routed.shape[1])
    H = int(hidden_states.shape[-1])
    A = T * K
    phys = routed.to(device=device, dtype=torch.int32).contiguous()
    weights = routing_weights.to(device=device, dtype=dt).contiguous()
    hidden = hidden_states.contiguous()
    pad = (-H) % 8
    if pad:
        hidden = torch.nn.functional.pad(hidden, (0, pad))
    Hp = H + pad

    i32 = dict(dtype=torch.int32, device=device)
    assign_counts = torch.empty(ep_size, **i32)
    assign_offsets = torch.empty(ep_size + 1, **i32)
    unique_counts = torch.empty(ep_size, **i32)
    unique_offsets = torch.empty(ep_size + 1, **i32)
    send_hidden = torch.empty((A, Hp), dtype=dt, device=device)
    unique_tokens = torch.empty(A, **i32)
    send_meta = torch.empty((A, 3), **i32)
    send_weights = torch.empty(A, dtype=dt, device=device)
    target_rank = torch.empty(A, **i32)
    status = torch.zeros(1, **i32)
    ws = _workspace(_capi.load().pmx_ep_payload_workspace_bytes(A, ep_size), device)
    _capi.call(
        "pmx_ep_dispatch_payload", phys.data_ptr() if A else None, hidden.data_ptr() if T else None,
        weights.data_ptr() if A else None, T, K, Hp, ep_size, num_local, assign_counts.data_ptr(),
        assign_offsets.data_ptr(), unique_counts.data_ptr(), unique_offsets.data_ptr(),
        send_hidden.data_ptr() if A else None, unique_tokens.data_ptr() if A else None,
        send_meta.data_ptr() if A else None, send_weights.data_ptr() if A else None,
        target_rank.data_ptr() if A else None, status.data_ptr(), ws.data_ptr(), ws.numel(), _stream(device),
    )
    counts = torch.cat([assign_counts, unique_counts, status]).cpu().tolist()
    if counts[-1]:
        raise ValueError("physical expert id outside [0, num_experts)")
    assignment_send_splits = [int(c) for c in counts[:ep_size]]
    unique_send_splits = [int(c) for c in counts[ep_size:2 * ep_size]]
    U = sum(unique_send_splits)
    return (
        send_hidden[:U, :H].to(hidden_states.dtype),
        send_meta,
        send_weights.to(routing_weights.dtype).unsqueeze(1),
        unique_tokens[:U].to(torch.long),
        unique_send_splits,
        assignment_send_splits,
        target_rank.reshape(T, K).to(torch.long),
    )


def combine_aggregate(expert_outputs: torch.Tensor, pos: torch.Tensor, recv_weights: torch.Tensor,
                      source_ranks: torch.Tensor, source_token_indices: torch.Tensor, ep_size: int):
    """Per (source rank, source token) fp32 sums of ``bf16(expert_outputs[pos[a]] * w[a])``
    over the received assignments ``a`` in receive order; returns the partial
    rows [U, H] (in the outputs' dtype, bf16 or fp16, which also rounds the
    products) and the rows per source rank (a host list)."""
    assert expert_outputs.is_cuda, "placemoe_amd kernels need GPU tensors"
    assert expert_outputs.dtype in HALF, f"expert_outputs must be bfloat16 or float16, got {expert_outputs.dtype}"
    dt = expert_outputs.dtype
    device = expert_outputs.device
    N = int(pos.numel())
    H = int(expert_outputs.shape[-1])
    y = expert_outputs.contiguous()
    pad = (-H) % 8
    if pad:
        y = torch.nn.functional.pad(y, (0, pad))
    Hp = H + pad
    i32 = dict(dtype=torch.int32, device=device)
    pos32 = pos.to(**i32).contiguous()
    w = recv_weights.reshape(-1).to(device=device, dtype=dt).contiguous()
    ranks = source_ranks.to(**i32).contiguous()
    tokens = source_token_indices.to(**i32).contiguous()
    out = torch.empty((max(N, 1), Hp), dtype=dt, device=device)
    run_offsets = torch.empty(N + 1, **i32)
    rank_runs = torch.empty(ep_size, **i32)
    num_runs = torch.empty(1, **i32)
    status = torch.zeros(1, **i32)
    ws = _workspace(_capi.load().pmx_ep_combine_workspace_bytes(N), device)
    name = "pmx_ep_combine_aggregate_f16" if dt == torch.float16 else "pmx_ep_combine_aggregate"
    _capi.call(
        name, y.data_ptr(), pos32.data_ptr() if N else None, w.data_ptr() if N else None,
        ranks.data_ptr() if N else None, tokens.data_ptr() if N else None, N, Hp, ep_size, out.data_ptr(),
        run_offsets.data_ptr(), rank_runs.data_ptr(), num_runs.data_ptr(), status.data_ptr(), ws.data_ptr(),
        ws.numel(), _stream(device),
    )
    host = torch.cat([rank_runs, num_runs, status]).cpu().tolist()
    if host[-1]:
        raise ValueError("source rank outside [0, ep_size)")
    U = int(host[ep_size])
    return out[:U, :H], [int(c) for c in host[:ep_size]]


def aggregate_weighted_outputs(weighted_outputs: torch.Tensor, source_token_indices: torch.Tensor,
                               split_sizes: list[int], key_stride: int | None = None):
    """``_aggregate_weighted_outputs``: rows already weighted and in receive
    order (``split_sizes`` rows per source rank), summed in fp32 per (source
    rank, token) run; returns the sums and the runs per source rank.
    ``key_stride`` is accepted for signature parity: runs are compared on
    (rank, token) directly, which is what distinct keys encode."""
    del key_stride
    device = weighted_outputs.device
    if weighted_outputs.numel() == 0:
        return torch.empty((0, weighted_outputs.shape[-1]), dtype=weighted_outputs.dtype, device=device), []
    R = len(split_sizes)
    ranks = torch.repeat_interleave(torch.arange(R, device=device),
                                    torch.as_tensor(split_sizes, device=device, dtype=torch.long))
    N = int(weighted_outputs.shape[0])
    dt = weighted_outputs.dtype if weighted_outputs.dtype in HALF else BF16
    ones = torch.ones(N, dtype=dt, device=device)
    sums, splits = combine_aggregate(weighted_outputs.to(dt), torch.arange(N, device=device), ones, ranks,
                                     source_token_indices, R)
    return sums.to(weighted_outputs.dtype), splits
