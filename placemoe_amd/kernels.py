"""Torch-tensor wrappers around the gfx950 C ABI.

Each wrapper checks device, dtype and contiguity (``AssertionError``, as the
reference's Triton wrappers do), allocates outputs with ``torch.empty`` on the
input's device, and enqueues the kernels on torch's current stream.  Nothing
here synchronises the host except ``route_status``.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _capi

BF16 = torch.bfloat16
F16 = torch.float16
HALF = (BF16, F16)


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _check_dev(*tensors: torch.Tensor | None) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        assert t.is_cuda, "placemoe_amd kernels need GPU tensors"
        if dev is None:
            dev = t.device
        assert t.device == dev, f"tensors on different devices: {t.device} vs {dev}"
    return dev


def _half(name: str, t: torch.Tensor, like: torch.dtype | None = None) -> torch.dtype:
    """A 16-bit float operand: bfloat16 or float16, contiguous, and of the
    dtype ``like`` of the call's other operands; returns its dtype."""
    assert t.dtype in HALF, f"{name} must be bfloat16 or float16, got {t.dtype}"
    if like is not None:
        assert t.dtype == like, f"{name} must be {like} like the other operands, got {t.dtype}"
    assert t.is_contiguous(), f"{name} must be contiguous"
    return t.dtype


def _sym(name: str, dtype: torch.dtype) -> str:
    """The entry point for the dtype: fp16 tensors go to the *_f16 twin."""
    return name + "_f16" if dtype == F16 else name


# ---------------------------------------------------------------------------
# Routing
# ---------------------------------------------------------------------------


@dataclass
class Routing:
    """Integer routing of one batch: every tensor is int32 on the device."""

    phys: torch.Tensor  # [T, K] physical copy of each assignment
    counts: torch.Tensor  # [C]
    offsets: torch.Tensor  # [C+1] exclusive prefix; offsets[1:] is cumsum_M
    pos: torch.Tensor  # [T, K] row of each assignment in the permuted buffer
    workspace: torch.Tensor  # holds the routing status word

    @property
    def num_slots(self) -> int:
        return int(self.counts.numel())


def route(
    selected: torch.Tensor,
    num_slots: int,
    mapping: torch.Tensor | None = None,
    sources: torch.Tensor | None = None,
    source: int = 0,
) -> Routing:
    """phys = mapping[source(t), selected]; counts; offsets; stable scatter index.

    ``mapping`` is the source-aware ``M`` table [S, E] (int64 on the device),
    or None for the identity map.  ``sources`` is an int64 [T] per-token source
    id; without it every token uses ``source`` (the reference's ``ep_rank``).
    """
    dev = _check_dev(selected, mapping, sources)
    sel = selected if selected.dim() == 2 else selected.reshape(-1, 1)
    sel = sel.to(torch.int64).contiguous()
    T, K = sel.shape
    C = int(num_slots)
    if mapping is not None:
        mapping = mapping.to(torch.int64).contiguous()
        assert mapping.dim() == 2, "mapping must be [num_sources, num_experts]"
        S, E = mapping.shape
    else:
        S, E = 1, C
    if sources is not None:
        assert mapping is not None, "per-token sources need a mapping table"
        sources = sources.to(torch.int64).contiguous().reshape(-1)
        assert sources.numel() == T, "sources must have one entry per token"
    A = T * K
    ws_bytes = _capi.load().pmx_route_workspace_bytes(A, C)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    phys = torch.empty((T, K), dtype=torch.int32, device=dev)
    pos = torch.empty((T, K), dtype=torch.int32, device=dev)
    counts = torch.empty(C, dtype=torch.int32, device=dev)
    offsets = torch.empty(C + 1, dtype=torch.int32, device=dev)
    _capi.call(
        "pmx_route", _ptr(sel), _ptr(mapping), _ptr(sources), int(source), S, E, T, K, C,
        _ptr(phys), _ptr(counts), _ptr(offsets), _ptr(pos), _ptr(ws), ws_bytes, _stream(dev),
    )
    return Routing(phys=phys, counts=counts, offsets=offsets, pos=pos, workspace=ws)


def route_status(r: Routing) -> int:
    """0 if every id was inside its table (synchronises the stream)."""
    out = ctypes.c_int32(-1)
    _capi.call("pmx_route_status", _ptr(r.workspace), ctypes.byref(out), _stream(r.workspace.device))
    return int(out.value)


class RouteCheck:
    """The routing status word, copied to pinned host memory behind the
    routing kernels on the same stream.  ``ready()`` asks (without waiting)
    whether the copy has landed; ``failed()`` waits for it."""

    def __init__(self, r: Routing):
        dev = r.workspace.device
        self._host = torch.empty(1, dtype=torch.int32, pin_memory=True)
        self._host.copy_(r.workspace[:4].view(torch.int32), non_blocking=True)
        self._event = torch.cuda.Event()
        self._event.record(torch.cuda.current_stream(dev))
        self.checked = False

    def ready(self) -> bool:
        return self._event.query()

    def failed(self) -> bool:
        self._event.synchronize()
        return int(self._host[0]) != 0

    def raise_if_failed(self) -> None:
        self.checked = True
        if self.failed():
            raise ValueError(
                "selected_experts holds an expert id outside [0, num_experts) (or a source id outside the "
                "mapping's rows); the routing kernels clamped it, so this step's outputs are not valid."
            )


# ---------------------------------------------------------------------------
# Row movement
# ---------------------------------------------------------------------------


def moe_scatter(x: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
    """Xp[pos[t,k]] = x[t]  ->  [T*K, H]."""
    dev = _check_dev(x, pos)
    dt = _half("x", x)
    assert pos.dtype == torch.int32 and pos.is_contiguous()
    T, H = x.shape
    K = pos.shape[1]
    out = torch.empty((T * K, H), dtype=x.dtype, device=dev)
    _capi.call("pmx_moe_scatter", _ptr(x), _ptr(pos), T, K, H, _ptr(out), _stream(dev))
    return out


def moe_scatter_src(x: torch.Tensor, pos: torch.Tensor, w: torch.Tensor | None = None):
    """moe_scatter that also returns each row's source: row_src[pos[t,k]] =
    t*K + k (int32 [T*K]), and with the router weights ``w`` [T, K] each row's
    weight row_w[pos[t,k]] = w[t,k] -> (Xp, row_src, row_w or None)."""
    dev = _check_dev(x, pos, w)
    dt = _half("x", x)
    assert pos.dtype == torch.int32 and pos.is_contiguous()
    T, H = x.shape
    K = pos.shape[1]
    out = torch.empty((T * K, H), dtype=x.dtype, device=dev)
    src = torch.empty(T * K, dtype=torch.int32, device=dev)
    row_w = None
    if w is not None:
        _half("routing weights", w, dt)
        assert w.numel() == T * K, "routing weights: one per (token, k)"
        row_w = torch.empty(T * K, dtype=w.dtype, device=dev)
    _capi.call("pmx_moe_scatter_src", _ptr(x), _ptr(pos), _ptr(w), T, K, H, _ptr(out), _ptr(src), _ptr(row_w),
               _stream(dev))
    return out, src, row_w


def moe_gather(y: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
    """out[t] = bf16(sum_k fp32(y[pos[t,k]]))  ->  [T, H]."""
    dev = _check_dev(y, pos)
    dt = _half("y", y)
    assert pos.dtype == torch.int32 and pos.is_contiguous()
    T, K = pos.shape
    H = y.shape[1]
    out = torch.empty((T, H), dtype=y.dtype, device=dev)
    _capi.call(_sym("pmx_moe_gather", dt), _ptr(y), _ptr(pos), T, K, H, _ptr(out), _stream(dev))
    return out


def combine_fwd(y: torch.Tensor, pos: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """out[t] = bf16(sum_k fp32(bf16(y[pos[t,k]] * w[t,k])))."""
    dev = _check_dev(y, pos, w)
    dt = _half("y", y)
    _half("routing weights", w, dt)
    T, K = pos.shape
    H = y.shape[1]
    out = torch.empty((T, H), dtype=y.dtype, device=dev)
    _capi.call(_sym("pmx_combine_fwd", dt), _ptr(y), _ptr(pos), _ptr(w), T, K, H, _ptr(out), _stream(dev))
    return out


def combine_bwd(dout: torch.Tensor, y: torch.Tensor, pos: torch.Tensor, w: torch.Tensor):
    """(dy [T*K,H], dw [T,K]) - the gradients of ``combine_fwd``."""
    dev = _check_dev(dout, y, pos, w)
    dt = _half("grad_output", dout)
    _half("y", y, dt)
    _half("routing weights", w, dt)
    T, K = pos.shape
    H = y.shape[1]
    dy = torch.empty_like(y)
    dw = torch.empty((T, K), dtype=w.dtype, device=dev)
    _capi.call(
        _sym("pmx_combine_bwd", dt), _ptr(dout), _ptr(y), _ptr(pos), _ptr(w), T, K, H, _ptr(dy), _ptr(dw),
        _stream(dev)
    )
    return dy, dw


def combine_bwd_top1_rows(dout: torch.Tensor, y: torch.Tensor, row_token: torch.Tensor, w: torch.Tensor):
    """Top-1 combine gradient walked in the rows' storage order (row_token:
    the row map of moe_scatter_src) -> (dY [T, H], dw [T, 1]); bit-identical
    to combine_bwd with the matching pos."""
    dev = _check_dev(dout, y, row_token, w)
    dt = _half("dout", dout)
    _half("y", y, dt)
    _half("routing weights", w, dt)
    T, H = dout.shape
    assert y.shape == (T, H), "top-1: one row of Y per token"
    assert row_token.dtype == torch.int32 and row_token.is_contiguous() and row_token.numel() == T
    assert w.numel() == T, "top-1 routing weights: one per token"
    dy = torch.empty((T, H), dtype=y.dtype, device=dev)
    dw = torch.empty((T, 1), dtype=w.dtype, device=dev)
    _capi.call(_sym("pmx_combine_bwd_top1_rows", dt), _ptr(dout), _ptr(y), _ptr(row_token), _ptr(w), T, H,
               _ptr(dy), _ptr(dw), _stream(dev))
    return dy, dw


def segment_sum(source: torch.Tensor, index: torch.Tensor, num_rows: int) -> torch.Tensor:
    """out[r] = sum_{i: index[i]==r} source[i] in fp32, stored as bf16.

    Mirrors ``segment_sum_dim0_fp32_to_source_dtype``: raises ``ValueError`` for
    an index outside [0, num_rows) (this check synchronises the stream).
    """
    if source.ndim != 2 or index.ndim != 1:
        raise ValueError("source must be 2D and index must be 1D.")
    if int(source.shape[0]) != int(index.numel()):
        raise ValueError("index length must match source rows.")
    num_rows = int(num_rows)
    if num_rows < 0:
        raise ValueError(f"num_rows must be non-negative, got {num_rows}.")
    dev = _check_dev(source)
    dt = _half("source", source)
    N, H = source.shape
    out = torch.empty((num_rows, H), dtype=source.dtype, device=dev)
    if num_rows == 0:
        if N != 0:
            raise ValueError("non-empty source cannot be reduced into zero rows.")
        return out
    idx = index.to(device=dev, dtype=torch.int64).contiguous()
    ws_bytes = _capi.load().pmx_segment_sum_workspace_bytes(N, num_rows)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    _capi.call(
        _sym("pmx_segment_sum", dt), _ptr(source), _ptr(idx), N, H, num_rows, _ptr(out), _ptr(ws), ws_bytes,
        _stream(dev)
    )
    status = ctypes.c_int32(-1)
    _capi.call("pmx_route_status", _ptr(ws), ctypes.byref(status), _stream(dev))
    if status.value != 0:
        raise ValueError("index contains a row outside [0, num_rows).")
    return out


# ---------------------------------------------------------------------------
# Grouped GEMM
# ---------------------------------------------------------------------------


def gemm_fc1_swiglu(x: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor, copy_stride: int,
                    offsets: torch.Tensor, num_groups: int, inter: int):
    """(gu [A,2I], act [A,I]) = SwiGLU fc1 over per-copy row groups."""
    dev = _check_dev(x, w_gate, w_up, offsets)
    dt = _half("hidden", x)
    _half("fc1 gate weight", w_gate, dt)
    _half("fc1 up weight", w_up, dt)
    A, H = x.shape
    G, inter, copy_stride = int(num_groups), int(inter), int(copy_stride)
    assert offsets.dtype == torch.int32 and offsets.numel() == G + 1, "offsets must be int32 [num_groups + 1]"
    # The kernel reads I*H elements of gate (and of up) rows at g*copy_stride for every group g.
    need = (G - 1) * copy_stride + inter * H
    assert copy_stride >= inter * H and w_gate.numel() >= need and w_up.numel() >= need, (
        f"fc1 weights hold {w_gate.numel()}/{w_up.numel()} elements; {G} copies of [{inter}, {H}] "
        f"at stride {copy_stride} need {need}"
    )
    gu = torch.empty((A, 2 * inter), dtype=x.dtype, device=dev)
    act = torch.empty((A, inter), dtype=x.dtype, device=dev)
    _capi.call(
        _sym("pmx_gemm_fc1_swiglu_fwd", dt), _ptr(x), _ptr(w_gate), _ptr(w_up), int(copy_stride), _ptr(offsets),
        int(num_groups), A, H, int(inter), _ptr(gu), _ptr(act), _stream(dev),
    )
    return gu, act


def group_gemm_nt(a: torch.Tensor, b: torch.Tensor, offsets: torch.Tensor) -> torch.Tensor:
    """C[rows of g] = a[rows of g] @ b[g]^T, b: [G, N, K]."""
    dev = _check_dev(a, b, offsets)
    dt = _half("a", a)
    _half("b", b, dt)
    G, N, K = b.shape
    assert a.shape[1] == K, "a and b disagree on K"
    assert offsets.numel() == G + 1
    M = a.shape[0]
    c = torch.empty((M, N), dtype=a.dtype, device=dev)
    _capi.call(_sym("pmx_group_gemm_nt", dt), _ptr(a), _ptr(b), _ptr(offsets), G, M, N, K, _ptr(c), _stream(dev))
    return c


def group_gemm_nt_combine_top1(a: torch.Tensor, b: torch.Tensor, offsets: torch.Tensor, row_token: torch.Tensor,
                               row_weight: torch.Tensor):
    """Top-1 layers: C = group_gemm_nt(a, b, offsets) and, in the same kernel,
    out[row_token[r]] = bf16(C[r] * row_weight[r]) (the combine) -> (C, out)."""
    dev = _check_dev(a, b, offsets, row_token, row_weight)
    dt = _half("a", a)
    _half("b", b, dt)
    _half("row weights", row_weight, dt)
    G, N, K = b.shape
    M = a.shape[0]
    assert a.shape[1] == K, "a and b disagree on K"
    assert offsets.numel() == G + 1
    assert row_token.dtype == torch.int32 and row_token.is_contiguous() and row_token.numel() == M
    assert row_weight.numel() == M, "top-1 routing weights: one per row"
    c = torch.empty((M, N), dtype=a.dtype, device=dev)
    out = torch.empty((M, N), dtype=a.dtype, device=dev)
    _capi.call(_sym("pmx_group_gemm_nt_combine_top1", dt), _ptr(a), _ptr(b), _ptr(offsets), G, M, N, K, _ptr(c),
               _ptr(row_token), _ptr(row_weight), _ptr(out), _stream(dev))
    return c, out


def group_gemm_nn_unpermute_top1(a: torch.Tensor, b: torch.Tensor, offsets: torch.Tensor, row_token: torch.Tensor,
                                 b_second: torch.Tensor | None = None) -> torch.Tensor:
    """Top-1 layers: group_gemm_nn whose row r is written to row row_token[r]
    (the unpermute gradient in the same kernel)."""
    assert row_token.dtype == torch.int32 and row_token.is_contiguous() and row_token.numel() == a.shape[0]
    return group_gemm_nn(a, b, offsets, b_second=b_second, row_token=row_token)


def group_gemm_nn(a: torch.Tensor, b: torch.Tensor, offsets: torch.Tensor,
                  b_second: torch.Tensor | None = None, row_token: torch.Tensor | None = None) -> torch.Tensor:
    """C[rows of g] = a[rows of g] @ cat(b, b_second, dim=1)[g], b: [G, K(, +K2), N];
    with ``row_token`` (top-1 layers) row r goes to row row_token[r] of C."""
    dev = _check_dev(a, b, offsets, b_second, row_token)
    dt = _half("a", a)
    _half("b", b, dt)
    G, K0, N = b.shape
    K = K0 + (b_second.shape[1] if b_second is not None else 0)
    if b_second is not None:
        _half("b_second", b_second, dt)
        assert b_second.shape[0] == G and b_second.shape[2] == N and b_second.shape[1] == K0
    assert a.shape[1] == K, "a and b disagree on K"
    assert offsets.numel() == G + 1
    M = a.shape[0]
    c = torch.empty((M, N), dtype=a.dtype, device=dev)
    split = K0 if b_second is not None else 0
    if row_token is None:
        _capi.call(_sym("pmx_group_gemm_nn", dt), _ptr(a), _ptr(b), _ptr(b_second), K0 * N, split, _ptr(offsets),
                   G, M, N, K, _ptr(c), _stream(dev))
    else:
        _capi.call(_sym("pmx_group_gemm_nn_unpermute_top1", dt), _ptr(a), _ptr(b), _ptr(b_second), K0 * N, split,
                   _ptr(offsets), G, M, N, K, _ptr(row_token), _ptr(c), _stream(dev))
    return c


def gemm_fc2_dgrad_swiglu(dy: torch.Tensor, w_down: torch.Tensor, gu: torch.Tensor,
                          offsets: torch.Tensor) -> torch.Tensor:
    """dG1 [A,2I] = SwiGLU backward of (dy @ w_down[g]) given the saved gate/up."""
    dev = _check_dev(dy, w_down, gu, offsets)
    dt = _half("dy", dy)
    _half("w_down", w_down, dt)
    _half("gu", gu, dt)
    G, H, I = w_down.shape
    A = dy.shape[0]
    assert dy.shape[1] == H and gu.shape == (A, 2 * I)
    dg1 = torch.empty((A, 2 * I), dtype=dy.dtype, device=dev)
    _capi.call(
        _sym("pmx_gemm_fc2_dgrad_swiglu_bwd", dt), _ptr(dy), _ptr(w_down), _ptr(gu), _ptr(offsets), G, A, H, I,
        _ptr(dg1), _stream(dev),
    )
    return dg1


def weight_rows(act: torch.Tensor, row_w: torch.Tensor) -> torch.Tensor:
    """out[r] = bf16(act[r] * row_w[r]) -> [R, N]: the router weight applied
    to the fc2 input (the reference's non-EP path)."""
    dev = _check_dev(act, row_w)
    dt = _half("act", act)
    _half("row weights", row_w, dt)
    R, N = act.shape
    assert row_w.numel() == R and row_w.is_contiguous(), "one router weight per row"
    out = torch.empty_like(act)
    _capi.call(_sym("pmx_weight_rows", dt), _ptr(act), _ptr(row_w), R, N, _ptr(out), _stream(dev))
    return out


def swiglu_bwd_weighted(d_act_w: torch.Tensor, gu: torch.Tensor, act: torch.Tensor, row_w: torch.Tensor,
                        row_src: torch.Tensor, num_assign: int):
    """Backward of ``weight_rows`` and the SwiGLU forward, per row:
    dG1 [R, 2I] from dact = bf16(d_act_w * row_w), and the router-weight
    gradient dw[row_src[r]] = bf16(sum_j bf16(act[r,j] * d_act_w[r,j]))
    -> (dG1, dw [num_assign] bf16; entries no row names are not written)."""
    dev = _check_dev(d_act_w, gu, act, row_w, row_src)
    dt = _half("act", act)
    for name, t in (("d_act_w", d_act_w), ("gu", gu), ("row weights", row_w)):
        _half(name, t, dt)
    R, I = act.shape
    assert d_act_w.shape == (R, I) and gu.shape == (R, 2 * I), "d_act_w [R, I], gu [R, 2I]"
    assert row_w.numel() == R and row_w.is_contiguous()
    assert row_src.dtype == torch.int32 and row_src.is_contiguous() and row_src.numel() == R
    dg1 = torch.empty((R, 2 * I), dtype=act.dtype, device=dev)
    dw = torch.empty(num_assign, dtype=row_w.dtype, device=dev)
    _capi.call(_sym("pmx_swiglu_bwd_weighted", dt), _ptr(d_act_w), _ptr(gu), _ptr(act), _ptr(row_w), _ptr(row_src),
               R, I, num_assign, _ptr(dg1), _ptr(dw), _stream(dev))
    return dg1, dw


def group_gemm_tn(a: torch.Tensor, b: torch.Tensor, offsets: torch.Tensor, split: int | None = None):
    """C[g] = a[rows g]^T @ b[rows g] -> [G, M, N] (zeros for empty groups).

    With ``split`` the result is returned as two tensors [G, split, N] and
    [G, M - split, N] (split fc1 weight gradients).
    """
    dev = _check_dev(a, b, offsets)
    dt = _half("a", a)
    _half("b", b, dt)
    M, N = a.shape[1], b.shape[1]
    K = a.shape[0]
    assert b.shape[0] == K, "a and b must have the same rows"
    G = offsets.numel() - 1
    if a.shape[0] == 0:
        # No rows at all (an empty micro-batch): every group is empty, so every C[g] is zero.
        # The entry point takes non-null A and B, which an empty tensor does not have.
        c = torch.zeros((G, M, N), dtype=a.dtype, device=dev)
        return c if split is None else (c[:, :split].clone(), c[:, split:].clone())
    if split is None:
        c0 = torch.empty((G, M, N), dtype=a.dtype, device=dev)
        _capi.call(
            _sym("pmx_group_gemm_tn", dt), _ptr(a), _ptr(b), _ptr(offsets), G, K, M, N, _ptr(c0), None, M * N,
            0, _stream(dev)
        )
        return c0
    assert M - split == split, "split gradients must have equal halves"
    c0 = torch.empty((G, split, N), dtype=a.dtype, device=dev)
    c1 = torch.empty((G, split, N), dtype=a.dtype, device=dev)
    _capi.call(
        _sym("pmx_group_gemm_tn", dt), _ptr(a), _ptr(b), _ptr(offsets), G, K, M, N, _ptr(c0), _ptr(c1), split * N,
        split, _stream(dev),
    )
    return c0, c1


# ---------------------------------------------------------------------------
# Replica fold
# ---------------------------------------------------------------------------


def replica_fold(grads: torch.Tensor, copy_offsets: torch.Tensor, copy_slots: torch.Tensor, num_experts: int,
                 slot_tokens: torch.Tensor | None = None, writeback: bool = False,
                 status: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 [E, ...] = sum over the active copies of each expert of ``grads`` [C, ...].

    A ``copy_slots`` entry outside [0, C) is skipped by the kernel and sets
    ``status`` (a caller-zeroed int32 device tensor, if given) to 1; nothing
    here reads it back, so the call never synchronises the host.
    """
    dev = _check_dev(grads, copy_offsets, copy_slots, slot_tokens, status)
    dt = _half("grads", grads)
    assert copy_offsets.dtype == torch.int32 and copy_slots.dtype == torch.int32
    assert copy_offsets.numel() == int(num_experts) + 1, "copy_offsets must have num_experts + 1 entries"
    if status is not None:
        assert status.dtype == torch.int32 and status.numel() >= 1
    C = grads.shape[0]
    P = grads[0].numel() if C else 0
    out = torch.empty((num_experts,) + tuple(grads.shape[1:]), dtype=torch.float32, device=dev)
    if slot_tokens is not None:
        slot_tokens = slot_tokens.to(torch.int64).contiguous()
        assert slot_tokens.numel() == C
    _capi.call(
        _sym("pmx_replica_fold", dt), _ptr(grads), _ptr(copy_offsets), _ptr(copy_slots), _ptr(slot_tokens),
        int(num_experts), C, P, ctypes.cast(out.data_ptr(), ctypes.POINTER(ctypes.c_float)),
        1 if writeback else 0, _ptr(status), _stream(dev),
    )
    return out
