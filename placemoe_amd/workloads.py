"""Seeded synthetic workloads for the five benchmark configurations.

Every tensor is drawn from a ``torch.Generator`` seeded per configuration, on
the requested device.  Token counts can be scaled down (``tokens=``) for
parity tests while the layer shape (H, I, E, C, K, sources) stays the
configuration's.

1. ``toy``   T=4096, H=1024, E=8 -> C=12 (experts 0-3 duplicated), K=2, I=2816,
             4 sources, round-robin M.  Forward only.
2. ``qwen3`` T=16384, H=2048, E=128 -> C=160 (the 32 most-routed experts of
             the batch replicated at slots 128..159), K=8, I=768, 8 sources,
             round-robin M; router logits N(0,1) + per-expert bias N(0,0.5).
3. ``dsv3``  one EP rank's share: 65536 received rows, H=7168, I=2048, 16
             slots (8 experts + 8 hot replicas holding other ranks' experts,
             so 16 distinct weight sets); per-slot counts multinomial over
             Zipf(1.0); rows arrive mapped (K=1, identity M); router weights
             U(0.05, 1).
4. ``skew``  T=32768, H=4096, E=64 -> C=96 (32 highest-demand experts
             replicated), K=4, I=1536; expert demand Zipf(1.4) over the 45
             head experts and an expected 0-16 rows for each of the 19 tail
             experts (~20% of the copies), K distinct experts per token drawn
             without replacement; 16 sources with a uniformly random copy per
             (source, expert).
5. ``fold``  Qwen3 shape (E=128, H=2048, I=768, K=8, T=16384) with 1-4 copies
             per expert, 256 in total, allocated by largest remainder in
             proportion to Zipf(1.0) demand; round-robin M over 8 sources.

Router weights of configs 1, 2 and 5: softmax over the logits (fp32), top-K,
renormalised, bf16.  Config 4: softmax of N(0,1) logits over the K chosen
experts.  Hidden ~ N(0,1); weights ~ N(0, 0.02) (0.006 for dsv3), bf16.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

CONFIG_SEEDS = {"toy": 1001, "qwen3": 1002, "dsv3": 1003, "skew": 1004, "fold": 1005}
CONFIG_INDEX = {"toy": 0, "qwen3": 1, "dsv3": 2, "skew": 3, "fold": 4}


@dataclass
class Workload:
    name: str
    hidden: torch.Tensor  # [T, H] bf16
    routing_weights: torch.Tensor  # [T, K] bf16
    selected: torch.Tensor  # [T, K] int64 logical experts
    sources: torch.Tensor | None  # [T] int64
    mapping: torch.Tensor  # [S, E] int64 (M)
    slot_to_logical: np.ndarray  # [C] (L)
    fc1: torch.Tensor | None  # [C, 2I, H] bf16 copy weights (gate rows, then up rows)
    fc2: torch.Tensor | None  # [C, H, I] bf16
    num_experts: int
    seed: int
    inter: int
    meta: dict = field(default_factory=dict)

    @property
    def T(self) -> int:
        return int(self.hidden.shape[0])

    @property
    def K(self) -> int:
        return int(self.selected.shape[1])

    @property
    def H(self) -> int:
        return int(self.hidden.shape[1])

    @property
    def I(self) -> int:  # noqa: E743
        return int(self.inter)

    @property
    def C(self) -> int:
        return int(self.slot_to_logical.shape[0])

    def owner_slots(self) -> np.ndarray:
        L = self.slot_to_logical
        return np.array([int(np.nonzero(L == e)[0][0]) for e in range(self.num_experts)], dtype=np.int64)


def _round_robin_mapping(slot_to_logical: np.ndarray, num_experts: int, num_sources: int) -> np.ndarray:
    copies = [np.nonzero(slot_to_logical == e)[0] for e in range(num_experts)]
    M = np.empty((num_sources, num_experts), dtype=np.int64)
    for e, c in enumerate(copies):
        for s in range(num_sources):
            M[s, e] = c[s % len(c)]
    return M


def _zipf(n: int, s: float) -> np.ndarray:
    p = np.arange(1, n + 1, dtype=np.float64) ** (-s)
    return p / p.sum()


def zipf_copy_counts(demand: np.ndarray, total: int, lo: int = 1, hi: int = 4) -> np.ndarray:
    """Copies per expert in proportion to demand, clamped to [lo, hi], summing to
    ``total`` (largest-remainder rounding, then clamping with redistribution)."""
    n = demand.size
    if not n * lo <= total <= n * hi:
        raise ValueError("total copies outside [n*lo, n*hi]")
    target = demand / demand.sum() * total
    counts = np.clip(np.floor(target).astype(np.int64), lo, hi)
    remainder = target - np.floor(target)
    order = np.lexsort((np.arange(n), -remainder))  # largest remainder first, ties by index
    while counts.sum() < total:
        for e in order:
            if counts.sum() == total:
                break
            if counts[e] < hi:
                counts[e] += 1
    while counts.sum() > total:
        for e in order[::-1]:
            if counts.sum() == total:
                break
            if counts[e] > lo:
                counts[e] -= 1
    return counts


def _randn(shape, gen, device, std=1.0, dtype=torch.bfloat16):
    return (torch.randn(shape, generator=gen, device=device, dtype=torch.float32) * std).to(dtype)


def _topk_router(logits: torch.Tensor, k: int) -> tuple[torch.Tensor, torch.Tensor]:
    probs = torch.softmax(logits.float(), dim=-1)
    w, sel = torch.topk(probs, k, dim=-1)
    w = w / w.sum(dim=-1, keepdim=True)
    return w.to(torch.bfloat16).contiguous(), sel.to(torch.int64).contiguous()


def _logical_then_copies(enabled, slot_to_logical, E, H, I, gen, dev, std):
    """Logical expert weights [E, 2I, H] and [E, H, I], then one copy per slot."""
    if not enabled:
        return None, None
    f1 = _randn((E, 2 * I, H), gen, dev, std)
    f2 = _randn((E, H, I), gen, dev, std)
    L = torch.as_tensor(slot_to_logical, device=dev)
    return f1.index_select(0, L).contiguous(), f2.index_select(0, L).contiguous()


def make_workload(name: str, device="cpu", tokens: int | None = None, num_slots: int | None = None,
                  seed: int | None = None, weights: bool = True) -> Workload:
    """Build configuration ``name`` on ``device``.  ``tokens`` scales T (rows for
    dsv3); ``num_slots`` (dsv3 only) reduces the slot count for CPU-sized tests;
    ``weights=False`` skips the expert weights (routing-only studies)."""
    seed = CONFIG_SEEDS[name] if seed is None else seed
    gen = torch.Generator(device=device).manual_seed(seed)
    rng = np.random.default_rng(seed)
    dev = torch.device(device)
    if name == "toy":
        T, H, E, K, I, S = tokens or 4096, 1024, 8, 2, 2816, 4
        L = np.array(list(range(8)) + [0, 1, 2, 3], dtype=np.int64)
        hidden = _randn((T, H), gen, dev)
        w, sel = _topk_router(torch.randn((T, E), generator=gen, device=dev), K)
        src = torch.randint(0, S, (T,), generator=gen, device=dev)
        M = _round_robin_mapping(L, E, S)
        fc1, fc2 = _logical_then_copies(weights, L, E, H, I, gen, dev, 0.02)
        meta = {"forward_only": True}
    elif name in ("qwen3", "fold"):
        T, H, E, K, I, S = tokens or 16384, 2048, 128, 8, 768, 8
        hidden = _randn((T, H), gen, dev)
        if name == "qwen3":
            logits = torch.randn((T, E), generator=gen, device=dev) + 0.5 * torch.randn((E,), generator=gen, device=dev)
            w, sel = _topk_router(logits, K)
            counts = torch.bincount(sel.reshape(-1), minlength=E).cpu().numpy()
            hot = np.lexsort((np.arange(E), -counts))[:32]  # most-routed first, ties by id
            L = np.concatenate([np.arange(E), hot]).astype(np.int64)
        else:
            demand = _zipf(E, 1.0)
            probs = torch.as_tensor(demand, dtype=torch.float32, device=dev).expand(T, E)
            sel = torch.multinomial(probs, K, replacement=False, generator=gen).to(torch.int64)
            logits = torch.randn((T, K), generator=gen, device=dev)
            w = torch.softmax(logits, dim=-1).to(torch.bfloat16).contiguous()
            copies = zipf_copy_counts(demand, 256)
            L = np.concatenate([np.arange(E)] + [np.full(c - 1, e) for e, c in enumerate(copies) if c > 1]).astype(
                np.int64
            )
        src = torch.randint(0, S, (T,), generator=gen, device=dev)
        M = _round_robin_mapping(L, E, S)
        fc1, fc2 = _logical_then_copies(weights, L, E, H, I, gen, dev, 0.02)
        meta = {}
    elif name == "dsv3":
        C = num_slots or 16
        T, H, I, K = tokens or 65536, 7168, 2048, 1
        E = C  # replicas of other ranks' experts: every slot has its own weights here
        L = np.arange(C, dtype=np.int64)
        p = torch.as_tensor(_zipf(C, 1.0), dtype=torch.float32, device=dev)
        slots = torch.multinomial(p, T, replacement=True, generator=gen)
        sel = slots.to(torch.int64).reshape(T, 1).contiguous()
        hidden = _randn((T, H), gen, dev)
        w = (0.05 + 0.95 * torch.rand((T, 1), generator=gen, device=dev)).to(torch.bfloat16)
        src = None
        M = np.arange(C, dtype=np.int64).reshape(1, C)
        fc1, fc2 = _logical_then_copies(weights, L, C, H, I, gen, dev, 0.006)
        meta = {"mapped_rows": True}
    elif name == "skew":
        T, H, E, K, I, S = tokens or 32768, 4096, 64, 4, 1536, 16
        # Zipf(1.4) over the 45 head experts; the 19 tail experts (~20% of the
        # 96 copies) get an expected 0-16 rows each, so the tiny/empty-group
        # paths are exercised (Zipf(1.4) alone gives every copy > 100 rows).
        demand = np.empty(E)
        demand[:45] = _zipf(45, 1.4)
        # without-replacement draws roughly double a tiny weight's share
        tail = rng.integers(0, 17, size=E - 45) / float(2 * T * K)
        demand[45:] = tail
        demand[:45] *= 1.0 - tail.sum()
        probs = torch.as_tensor(demand, dtype=torch.float32, device=dev).expand(T, E)
        sel = torch.multinomial(probs, K, replacement=False, generator=gen).to(torch.int64).contiguous()
        w = torch.softmax(torch.randn((T, K), generator=gen, device=dev), dim=-1).to(torch.bfloat16).contiguous()
        L = np.concatenate([np.arange(E), np.arange(32)]).astype(np.int64)
        copies = [np.nonzero(L == e)[0] for e in range(E)]
        M = np.array([[c[rng.integers(len(c))] for c in copies] for _ in range(S)], dtype=np.int64)
        src = torch.randint(0, S, (T,), generator=gen, device=dev)
        hidden = _randn((T, H), gen, dev)
        fc1, fc2 = _logical_then_copies(weights, L, E, H, I, gen, dev, 0.02)
        meta = {}
    else:
        raise KeyError(f"unknown workload {name!r}; expected one of {sorted(CONFIG_SEEDS)}")
    return Workload(
        name=name, hidden=hidden.contiguous(), routing_weights=w.contiguous(), selected=sel.contiguous(),
        sources=None if src is None else src.to(torch.int64).contiguous(),
        mapping=torch.as_tensor(M, dtype=torch.int64, device=dev), slot_to_logical=L, fc1=fc1, fc2=fc2,
        num_experts=E, seed=seed, inter=I, meta=meta,
    )


def algorithmic_work(T: int, K: int, H: int, I: int, C: int) -> dict:
    """Flops and bytes per layer step (the roofline numerators)."""
    A = T * K
    return {
        "gemm_fwd_flops": 6 * A * H * I,
        "gemm_bwd_flops": 12 * A * H * I,
        "fc1_fwd_flops": 4 * A * H * I,
        "fc2_fwd_flops": 2 * A * H * I,
        "fc2_dgrad_flops": 2 * A * H * I,
        "fc2_wgrad_flops": 2 * A * H * I,
        "fc1_dgrad_flops": 4 * A * H * I,
        "fc1_wgrad_flops": 4 * A * H * I,
        "route_bytes": 4 * T + 8 * A,
        "permute_bytes": 2 * T * H + 2 * A * H + 4 * A,
        "combine_fwd_bytes": 2 * A * H + 2 * T * H + 4 * A,
        "combine_bwd_bytes": 2 * T * H + 4 * A * H + 4 * A,
        "unpermute_grad_bytes": 2 * A * H + 2 * T * H + 4 * A,
    }
