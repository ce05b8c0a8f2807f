"""Replica-gradient fold for the copies held by one GPU.

``fold_replica_gradients`` is the single-GPU share of
``ExpertSwapManager.sync_redundant_gradients``
(veomni/distributed/moe/hiermoe/expert_swap.py:7220-7252): slots that saw no
tokens are treated as zero (``_zero_inactive_slot_grads_for_layer``,
:6250-6262), copies of each logical expert are summed (here in fp32;
``_replica_grad_contributions``, :6839-6876), and, with ``writeback``, every
copy receives the total (``_unpack_replica_grad``, :6886-6889).

``replica_grad_schedule`` / ``ReplicaGradExchange`` are one rank's side of
the cross-rank exchange for experts whose copies live on several EP ranks
(``_replica_grad_schedule_for_layer`` :6797-6837,
``_sync_pairwise_replica_gradients`` :7038-7107,
``_sync_owner_replica_gradients`` :7109-7217): the send buffers are packed
and the received parts folded into every local copy on the GPU
(``pmx_replica_exchange_pack`` / ``_unpack``), with the reference's buffer
layout, so that any transport (RCCL send/recv, all-to-all) can move them.
The transport itself is the caller's.  ``redundant_grad_norm_mask`` mirrors
``redundant_grad_norm_masks`` (:7254-7266).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Sequence

import numpy as np
import torch

from . import _capi, experts, kernels
from .placement import PLACEMENTS, LayerPlacement


def fold_replica_gradients(placement: LayerPlacement, grads: torch.Tensor, *, writeback: bool = True,
                           use_slot_tokens: bool = True) -> torch.Tensor:
    """fp32 [E, ...] logical gradients from copy gradients ``grads`` [C, ...] (bf16)."""
    if int(grads.shape[0]) != placement.num_slots:
        raise ValueError(f"expected {placement.num_slots} copy gradients, got {int(grads.shape[0])}")
    off, slots = placement.copy_tables_for_device(grads.device)
    tokens = placement.accumulated_slot_tokens if use_slot_tokens else None
    return kernels.replica_fold(grads.contiguous(), off, slots, placement.num_experts, slot_tokens=tokens,
                                writeback=writeback)


@torch.no_grad()
def sync_redundant_gradients(modules: dict[str, torch.nn.Module]) -> dict[str, tuple[torch.Tensor, torch.Tensor]]:
    """Fold ``gate_up_proj.grad`` and ``down_proj.grad`` of every registered
    layer in place; returns the fp32 logical gradients per layer and clears
    the accumulated token counts."""
    out = {}
    for key, module in modules.items():
        placement = PLACEMENTS.get(key)
        if placement is None:
            continue
        results = []
        for param in (module.gate_up_proj, module.down_proj):
            if param.grad is None:
                param.grad = torch.zeros_like(param)
            results.append(fold_replica_gradients(placement, param.grad))
        placement.clear_slot_tokens()
        out[key] = (results[0], results[1])
    return out


class OverlappedReplicaSync:
    """The fold of ``sync_redundant_gradients``, layer by layer, overlapped
    with the rest of the backward.

    As soon as both expert gradients of a registered layer have been
    accumulated (a post-accumulate-grad hook on ``gate_up_proj`` and
    ``down_proj``), that layer's fold is enqueued on a side stream that
    waits for the caller's stream at that point; the backward of the layers
    before it goes on on the caller's stream meanwhile.  The reference does
    the same per layer on a separate stream ordered by ready events
    (veomni/distributed/moe/hiermoe/expert_swap.py:5259-5262, :5318-5336).
    ``finish()`` makes the caller's stream wait for every fold and returns the
    fp32 logical gradients per layer, as ``sync_redundant_gradients`` does.

    One fold per backward while ``enabled``; with gradient accumulation,
    disable it for all but the last micro-batch.  The side stream keeps the
    default priority.
    """

    def __init__(self, modules: dict[str, torch.nn.Module], *, writeback: bool = True):
        self.enabled = True
        self._modules = dict(modules)
        self._writeback = writeback
        self._arrived: dict[str, set] = {}
        self._results: dict[str, tuple[torch.Tensor, torch.Tensor]] = {}
        self._streams: dict[torch.device, torch.cuda.Stream] = {}
        self._handles = []
        for key, module in self._modules.items():
            for param in (module.gate_up_proj, module.down_proj):
                self._handles.append(param.register_post_accumulate_grad_hook(self._hook(key)))

    def _hook(self, key: str):
        def on_grad(param: torch.Tensor) -> None:
            if not self.enabled:
                return
            arrived = self._arrived.setdefault(key, set())
            arrived.add(id(param))
            if len(arrived) == 2:
                arrived.clear()
                self._enqueue(key)

        return on_grad

    def _stream(self, device: torch.device) -> torch.cuda.Stream:
        s = self._streams.get(device)
        if s is None:
            s = torch.cuda.Stream(device=device)
            self._streams[device] = s
        return s

    @torch.no_grad()
    def _enqueue(self, key: str) -> None:
        placement = PLACEMENTS.get(key)
        if placement is None:
            return
        module = self._modules[key]
        grads = (module.gate_up_proj.grad, module.down_proj.grad)
        device = grads[0].device
        main = torch.cuda.current_stream(device)
        side = self._stream(device)
        side.wait_stream(main)
        with torch.cuda.stream(side):
            folded = tuple(fold_replica_gradients(placement, g, writeback=self._writeback) for g in grads)
        for g in grads:
            g.record_stream(side)
        self._results[key] = folded

    def finish(self) -> dict[str, tuple[torch.Tensor, torch.Tensor]]:
        """The caller's stream waits for every enqueued fold; returns the fp32
        logical gradients of the layers folded since the last call and clears
        their accumulated token counts.  Routing checks of the step whose
        status has landed are looked at (no waiting): an invalid expert id
        raises ``ValueError`` here at the latest."""
        experts.check_pending_routes()
        for device, side in self._streams.items():
            main = torch.cuda.current_stream(device)
            main.wait_stream(side)
        out, self._results = self._results, {}
        for key, folded in out.items():
            for t in folded:
                t.record_stream(torch.cuda.current_stream(t.device))
            placement = PLACEMENTS.get(key)
            if placement is not None:
                placement.clear_slot_tokens()
        return out

    def remove(self) -> None:
        for h in self._handles:
            h.remove()
        self._handles = []


# ---------------------------------------------------------------------------
# Cross-rank replica-gradient exchange: one rank's side
# ---------------------------------------------------------------------------

PMX_DTYPE = {torch.bfloat16: 0, torch.float32: 1, torch.float16: 2}


@dataclass(frozen=True)
class ReplicaGradGroup:
    """``_ReplicaGradGroup`` (expert_swap.py:829-834)."""

    logical_expert: int
    owner_rank: int
    copy_ranks: tuple[int, ...]
    local_slots: tuple[int, ...]


@dataclass(frozen=True)
class ReplicaGradSchedule:
    """``_ReplicaGradSchedule`` (expert_swap.py:837-841)."""

    groups: tuple[ReplicaGradGroup, ...]
    pairwise: bool
    globally_ordered_pairs: bool


def replica_grad_schedule(slot_to_logical, logical_to_physical, num_local_experts: int, ep_rank: int,
                          ep_size: int) -> ReplicaGradSchedule:
    """Copy groups of the experts with more than one copy (in expert order),
    their owner rank (the rank of the expert's runtime owner slot), the ranks
    holding copies and this rank's local slots; ``pairwise`` when no expert has
    copies on more than two ranks, ``globally_ordered_pairs`` when some rank
    then pairs with more than one peer.  Mirrors
    ``_replica_grad_schedule_for_layer`` (expert_swap.py:6797-6837) over
    ``redundant_copy_groups`` (:552-572) and ``_owner_rank_for_copy_group``
    (:6541-6555), including its errors."""
    L = np.asarray(torch.as_tensor(slot_to_logical).cpu(), dtype=np.int64).reshape(-1)
    owners = np.asarray(torch.as_tensor(logical_to_physical).cpu(), dtype=np.int64).reshape(-1)
    E = int(owners.size)
    active = L[L >= 0]
    counts = np.bincount(active, minlength=E) if active.size else np.zeros(E, dtype=np.int64)
    groups = []
    for e in np.nonzero(counts > 1)[0].tolist():
        if not 0 <= e < E:
            raise RuntimeError(f"HierMoE redundant gradient sync received invalid logical expert {e}.")
        slots = np.nonzero(L == e)[0].tolist()
        owner_slot = int(owners[e])
        if owner_slot not in slots:
            raise RuntimeError(f"HierMoE owner slot {owner_slot} for logical expert {e} is not in its copy group.")
        copy_ranks = tuple(sorted({s // num_local_experts for s in slots}))
        local = tuple(s % num_local_experts for s in slots if s // num_local_experts == ep_rank)
        groups.append(ReplicaGradGroup(int(e), owner_slot // num_local_experts, copy_ranks, local))
    pairwise = all(len(g.copy_ranks) <= 2 for g in groups)
    neighbors = [set() for _ in range(int(ep_size))]
    if pairwise:
        for g in groups:
            if len(g.copy_ranks) == 2:
                a, b = g.copy_ranks
                neighbors[a].add(b)
                neighbors[b].add(a)
    return ReplicaGradSchedule(tuple(groups), pairwise, pairwise and any(len(n) > 1 for n in neighbors))


def redundant_grad_norm_mask(slot_to_logical, logical_to_physical, num_local_experts: int,
                             ep_rank: int) -> torch.Tensor | None:
    """Bool [num_local_experts]: the local slots that hold their expert's
    runtime owner copy, so that a gradient norm counts every expert once
    (``redundant_grad_norm_masks``, expert_swap.py:7254-7266).  None when the
    layer has no expert with more than one copy (the reference adds no mask)."""
    L = np.asarray(torch.as_tensor(slot_to_logical).cpu(), dtype=np.int64).reshape(-1)
    active = L[L >= 0]
    if active.size == 0 or np.bincount(active).max() <= 1:
        return None
    mask = torch.zeros(num_local_experts, dtype=torch.bool)
    for slot in np.asarray(torch.as_tensor(logical_to_physical).cpu(), dtype=np.int64).reshape(-1).tolist():
        rank, local = divmod(int(slot), num_local_experts)
        if rank == ep_rank:
            mask[local] = True
    return mask


@dataclass
class _ItemTable:
    """Device tables of one launch: items of one parameter."""

    param: int
    n: int
    slot_offsets: torch.Tensor
    slots: torch.Tensor
    part_offsets: torch.Tensor | None
    part_ptrs: torch.Tensor | None
    out_offsets: torch.Tensor | None
    out_ptrs: torch.Tensor | None


class ReplicaGradExchange:
    """One rank's side of the replica-gradient exchange of one layer.

    ``grads`` are this rank's copy gradients, one contiguous tensor
    [num_local_experts, ...] per parameter (gate_up, then down).  Buffers are
    keyed by dtype (the reference's buckets) and peer rank; each holds the
    flattened items (expert-major, parameter-minor, schedule order) exactly as
    ``_pack_replica_grad_items`` lays them out, so received buffers from the
    reference or from this class are interchangeable.

    Pairwise schedules: ``pairwise_send()`` -> transport -> ``pairwise_finish(recv)``.
    Owner schedules: ``owner_reduce_send()`` -> transport ->
    ``owner_reduce_finish(recv)`` (returns the broadcast buffers) -> transport
    -> ``owner_broadcast_finish(recv)``.  Sums are fp32 on the GPU, stored in
    the gradient dtype; every local copy ends with the expert's total."""

    def __init__(self, schedule: ReplicaGradSchedule, ep_rank: int, grads: Sequence[torch.Tensor],
                 slot_tokens: torch.Tensor | None = None):
        """``slot_tokens`` (tokens each local slot saw since the last sync):
        slots with none are zeroed first, as ``_zero_inactive_slot_grads_for_layer``
        (expert_swap.py:6250-6262) does; a count vector of the wrong length is
        ignored, as there."""
        self.schedule = schedule
        self.ep_rank = int(ep_rank)
        self.grads = list(grads)
        for g in self.grads:
            if not g.is_cuda or not g.is_contiguous():
                raise ValueError("replica exchange gradients must be contiguous GPU tensors")
            if g.dtype not in PMX_DTYPE:
                raise ValueError(f"replica exchange supports bf16 and fp32 gradients, got {g.dtype}")
        self.device = self.grads[0].device
        if slot_tokens is not None:
            counts = torch.as_tensor(slot_tokens)
            if counts.ndim == 1 and int(counts.numel()) == int(self.grads[0].shape[0]):
                idle = torch.nonzero(counts.to(self.device) <= 0).flatten()
                if idle.numel():
                    for g in self.grads:
                        g.index_fill_(0, idle, 0)
        self.numel = [int(g[0].numel()) if g.shape[0] else 0 for g in self.grads]
        self._status = torch.zeros(1, dtype=torch.int32, device=self.device)
        # Bytes the launched kernels must read and write (local copies, parts,
        # outputs), accumulated on the host for bandwidth reports.
        self.bytes_moved = 0

    # -- helpers ------------------------------------------------------------

    def _buckets(self):
        out = {}
        for p, g in enumerate(self.grads):
            out.setdefault(g.dtype, []).append(p)
        return out

    def _layout(self, peer_groups: dict[int, list[ReplicaGradGroup]], params: list[int]):
        """Element offset of every (peer, group, param) item and each peer's total."""
        offsets, sizes = {}, {}
        for peer, groups in peer_groups.items():
            off = 0
            for g in groups:
                for p in params:
                    offsets[(peer, g.logical_expert, p)] = off
                    off += self.numel[p]
            sizes[peer] = off
        return offsets, sizes

    def _table(self, p: int, items: list[tuple[ReplicaGradGroup, list[int], list[int]]], *, pack: bool = False,
               with_local: bool = True) -> _ItemTable:
        """items: (group, part addresses, out addresses)."""
        es = self.grads[p].element_size() * self.numel[p]
        for g, pa, oa in items:
            reads = (len(g.local_slots) if with_local else 0) + len(pa)
            writes = len(oa) + (0 if pack else len(g.local_slots))
            self.bytes_moved += (reads + writes) * es
        dev = self.device
        i32 = dict(dtype=torch.int32)
        slot_off = np.zeros(len(items) + 1, dtype=np.int64)
        part_off = np.zeros(len(items) + 1, dtype=np.int64)
        out_off = np.zeros(len(items) + 1, dtype=np.int64)
        slots, parts, outs = [], [], []
        for i, (g, pa, oa) in enumerate(items):
            slots.extend(g.local_slots)
            parts.extend(pa)
            outs.extend(oa)
            slot_off[i + 1], part_off[i + 1], out_off[i + 1] = len(slots), len(parts), len(outs)

        def dev_i32(a):
            return torch.as_tensor(np.asarray(a, dtype=np.int32), **i32).to(dev)

        def dev_i64(a):
            return torch.as_tensor(np.asarray(a, dtype=np.int64)).to(dev)

        return _ItemTable(
            p, len(items), dev_i32(slot_off), dev_i32(slots if slots else [0]),
            dev_i32(part_off) if parts else None, dev_i64(parts) if parts else None,
            dev_i32(out_off) if outs else None, dev_i64(outs) if outs else None)

    def _launch(self, t: _ItemTable, *, pack: bool, with_local: bool = True) -> None:
        if t.n == 0 or self.numel[t.param] == 0:
            return
        g = self.grads[t.param]
        stream = ctypes.c_void_p(torch.cuda.current_stream(self.device).cuda_stream)
        ptr = lambda x: x.data_ptr() if x is not None else None  # noqa: E731
        if pack:
            _capi.call("pmx_replica_exchange_pack", g.data_ptr(), PMX_DTYPE[g.dtype], self.numel[t.param],
                       int(g.shape[0]), t.n, ptr(t.slot_offsets), ptr(t.slots), ptr(t.out_offsets), ptr(t.out_ptrs),
                       self._status.data_ptr(), stream)
        else:
            _capi.call("pmx_replica_exchange_unpack", g.data_ptr(), PMX_DTYPE[g.dtype], self.numel[t.param],
                       int(g.shape[0]), t.n, ptr(t.slot_offsets), ptr(t.slots), int(with_local),
                       ptr(t.part_offsets), ptr(t.part_ptrs), ptr(t.out_offsets), ptr(t.out_ptrs),
                       self._status.data_ptr(), stream)

    def _check_status(self) -> None:
        if int(self._status.item()):
            self._status.zero_()
            raise ValueError("replica exchange: a local slot lies outside the gradient tensor")

    def _pack(self, peer_groups: dict[int, list[ReplicaGradGroup]]) -> dict[torch.dtype, dict[int, torch.Tensor]]:
        out = {}
        for dtype, params in self._buckets().items():
            offsets, sizes = self._layout(peer_groups, params)
            bufs = {peer: torch.empty(sizes[peer], dtype=dtype, device=self.device) for peer in peer_groups}
            es = torch.empty((), dtype=dtype).element_size()
            for p in params:
                items = [(g, [], [bufs[peer].data_ptr() + offsets[(peer, g.logical_expert, p)] * es])
                         for peer, groups in peer_groups.items() for g in groups]
                self._launch(self._table(p, items, pack=True), pack=True)
            out[dtype] = bufs
        return out

    def _finish(self, peer_groups: dict[int, list[ReplicaGradGroup]], received, local_only: list[ReplicaGradGroup],
                *, with_local: bool, out_groups: dict[int, list[ReplicaGradGroup]] | None = None):
        """Fold received parts (and the local copies) into every local copy;
        with ``out_groups`` also write the totals into fresh send buffers."""
        sent = {}
        for dtype, params in self._buckets().items():
            offsets, _ = self._layout(peer_groups, params)
            recv = received.get(dtype, {})
            for peer, groups in peer_groups.items():
                need = sum(self.numel[p] for _ in groups for p in params)
                if peer not in recv or int(recv[peer].numel()) < need:
                    raise ValueError(f"replica exchange: buffer from rank {peer} is missing or too short")
                if recv[peer].dtype != dtype or recv[peer].device != self.device or not recv[peer].is_contiguous():
                    raise ValueError("replica exchange: received buffer has the wrong dtype or device, "
                                     "or is not contiguous")
            es = torch.empty((), dtype=dtype).element_size()
            if out_groups is not None:
                o_off, o_sizes = self._layout(out_groups, params)
                obufs = {peer: torch.empty(o_sizes[peer], dtype=dtype, device=self.device) for peer in out_groups}
                sent[dtype] = obufs
            for p in params:
                by_group: dict[int, tuple[ReplicaGradGroup, list[int], list[int]]] = {}
                for g in local_only:
                    by_group.setdefault(g.logical_expert, (g, [], []))
                for peer, groups in peer_groups.items():
                    for g in groups:
                        entry = by_group.setdefault(g.logical_expert, (g, [], []))
                        entry[1].append(recv[peer].data_ptr() + offsets[(peer, g.logical_expert, p)] * es)
                if out_groups is not None:
                    for peer, groups in out_groups.items():
                        for g in groups:
                            entry = by_group.setdefault(g.logical_expert, (g, [], []))
                            entry[2].append(obufs[peer].data_ptr() + o_off[(peer, g.logical_expert, p)] * es)
                items = [by_group[e] for e in sorted(by_group)]
                self._launch(self._table(p, items, with_local=with_local), pack=False, with_local=with_local)
        self._check_status()
        return sent

    # -- pairwise schedules (:7038-7107) --------------------------------------

    def _pairwise_peers(self):
        peers: dict[int, list[ReplicaGradGroup]] = {}
        local_only = []
        for g in self.schedule.groups:
            if not g.local_slots:
                continue
            remote = [r for r in g.copy_ranks if r != self.ep_rank]
            if not remote:
                local_only.append(g)
                continue
            if len(remote) != 1:
                raise RuntimeError("Pairwise redundant gradient schedule contains more than one remote copy.")
            peers.setdefault(remote[0], []).append(g)
        return peers, local_only

    def pairwise_send(self) -> dict[torch.dtype, dict[int, torch.Tensor]]:
        """Send buffer per peer: this rank's local sums of the items shared with it."""
        if not self.schedule.pairwise:
            raise RuntimeError("pairwise_send needs a pairwise schedule")
        peers, _ = self._pairwise_peers()
        return self._pack(peers)

    def pairwise_finish(self, received: dict[torch.dtype, dict[int, torch.Tensor]]) -> None:
        """Every local copy := local sum + the peer's sum (or the local sum for
        experts whose copies are all on this rank)."""
        peers, local_only = self._pairwise_peers()
        self._finish(peers, received, local_only, with_local=True)

    # -- owner schedules (:7109-7217) -----------------------------------------

    def _owner_roles(self):
        to_owner: dict[int, list[ReplicaGradGroup]] = {}
        from_sources: dict[int, list[ReplicaGradGroup]] = {}
        to_dest: dict[int, list[ReplicaGradGroup]] = {}
        owned = []
        for g in self.schedule.groups:
            if self.ep_rank not in g.copy_ranks:
                continue
            if self.ep_rank == g.owner_rank:
                owned.append(g)
                for r in g.copy_ranks:
                    if r != g.owner_rank:
                        from_sources.setdefault(r, []).append(g)
                        to_dest.setdefault(r, []).append(g)
            else:
                to_owner.setdefault(g.owner_rank, []).append(g)
        return to_owner, from_sources, to_dest, owned

    def owner_reduce_send(self) -> dict[torch.dtype, dict[int, torch.Tensor]]:
        """Send buffer per owner rank: this rank's local sums of the experts it owns a copy of."""
        to_owner, _, _, _ = self._owner_roles()
        return self._pack(to_owner)

    def owner_reduce_finish(self, received) -> dict[torch.dtype, dict[int, torch.Tensor]]:
        """Owner totals = local sum + every source's part, written into the
        local copies; returns the broadcast buffer per destination rank."""
        _, from_sources, to_dest, owned = self._owner_roles()
        return self._finish(from_sources, received, owned, with_local=True, out_groups=to_dest)

    def owner_broadcast_finish(self, received) -> None:
        """Every local copy of an expert owned elsewhere := the owner's total."""
        to_owner, _, _, _ = self._owner_roles()
        self._finish(to_owner, received, [], with_local=False)
