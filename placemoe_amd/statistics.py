"""Route statistics for the PlaceMoE placement planner, captured on the GPU.

``profile_route_statistics`` mirrors the reference's function of the same name
(veomni/distributed/moe/hiermoe/placemoe/statistics.py:30-64): the
source-conditioned demand ``demand[s, e]`` (assignments of expert ``e`` from
source rank ``s``) and the co-selection affinity ``affinity[s, a, b]`` (token
pairs of source ``s`` that chose both ``a`` and ``b``; symmetric, zero
diagonal), with the same argument checks and error messages.  The counting
runs in ``pmx_route_statistics``; ``RouteStatisticsRecorder`` keeps the
tables on the device across a profiling window, so recording a batch costs
one kernel and no host copy of the routes.
"""

from __future__ import annotations

import ctypes
from collections.abc import Sequence
from dataclasses import dataclass

import numpy as np
import torch

from . import _capi


def _readonly_float64(value) -> np.ndarray:
    array = np.array(value, dtype=np.float64, copy=True)
    array.setflags(write=False)
    return array


@dataclass(frozen=True)
class ProfileStatistics:
    """Source-conditioned assignment demand and expert co-selection affinity
    (``ProfileStatistics``, veomni/distributed/moe/hiermoe/placemoe/types.py:73-103)."""

    demand: np.ndarray
    affinity: np.ndarray

    def __post_init__(self) -> None:
        demand = _readonly_float64(self.demand)
        affinity = _readonly_float64(self.affinity)
        if demand.ndim != 2:
            raise ValueError("demand must have shape [source_rank, expert].")
        ep_size, num_experts = demand.shape
        if affinity.shape != (ep_size, num_experts, num_experts):
            raise ValueError("affinity must have shape [source_rank, expert, expert].")
        if bool((demand < 0).any()) or bool((affinity < 0).any()):
            raise ValueError("Profile statistics must be non-negative.")
        if not np.allclose(affinity, affinity.transpose(0, 2, 1)):
            raise ValueError("Expert affinity must be symmetric for every source rank.")
        if not np.allclose(np.diagonal(affinity, axis1=1, axis2=2), 0.0):
            raise ValueError("Expert affinity diagonal must be zero.")
        object.__setattr__(self, "demand", demand)
        object.__setattr__(self, "affinity", affinity)

    @property
    def ep_size(self) -> int:
        return int(self.demand.shape[0])

    @property
    def num_experts(self) -> int:
        return int(self.demand.shape[1])


def _device() -> torch.device:
    if not torch.cuda.is_available():
        raise RuntimeError("route statistics are computed on the GPU; no GPU is visible (there is no CPU fallback)")
    return torch.device("cuda", torch.cuda.current_device())


class RouteStatisticsRecorder:
    """Device-resident demand/affinity tables for ``ep_size`` sources and
    ``num_experts`` experts.  ``record`` enqueues one kernel on the current
    stream; ``invalid`` and ``statistics`` synchronise."""

    def __init__(self, ep_size: int, num_experts: int, device: torch.device | None = None):
        if ep_size <= 0:
            raise ValueError("ep_size must be positive.")
        if num_experts <= 0:
            raise ValueError("num_experts must be positive.")
        self.ep_size = int(ep_size)
        self.num_experts = int(num_experts)
        self.device = torch.device(device) if device is not None else _device()
        self.demand = torch.zeros((self.ep_size, self.num_experts), dtype=torch.int64, device=self.device)
        self.affinity = torch.zeros((self.ep_size, self.num_experts, self.num_experts), dtype=torch.int64,
                                    device=self.device)
        self._status = torch.zeros(1, dtype=torch.int32, device=self.device)

    def record(self, route: torch.Tensor, source_rank: int | torch.Tensor) -> None:
        """Add one route tensor [tokens, top_k] of logical expert ids; the
        source is one rank for every token or an int64 tensor [tokens]."""
        if route.ndim != 2 or route.shape[1] <= 0:
            raise ValueError("Each route tensor must have shape [tokens, top_k].")
        sel = route.to(device=self.device, dtype=torch.int64).contiguous()
        src_ptr, src_const = None, 0
        if isinstance(source_rank, torch.Tensor):
            src = source_rank.to(device=self.device, dtype=torch.int64).contiguous()
            assert src.numel() == sel.shape[0], "one source rank per token"
            src_ptr = src.data_ptr()
        else:
            src_const = int(source_rank)
            if not 0 <= src_const < self.ep_size:
                raise ValueError(f"source rank {src_const} outside [0, {self.ep_size}).")
        T, K = int(sel.shape[0]), int(sel.shape[1])
        _capi.call(
            "pmx_route_statistics", sel.data_ptr() if T else None, src_ptr, src_const, self.ep_size,
            self.num_experts, T, K, self.demand.data_ptr(), self.affinity.data_ptr(), self._status.data_ptr(),
            ctypes.c_void_p(torch.cuda.current_stream(self.device).cuda_stream),
        )
        # keep the inputs alive until the kernel has read them
        self._keep = (sel, source_rank)

    def invalid(self) -> bool:
        """True once a recorded token held an expert id outside [0, E) or a
        source outside [0, S) (such tokens are not counted)."""
        return bool(self._status.item())

    def reset(self) -> None:
        self.demand.zero_()
        self.affinity.zero_()
        self._status.zero_()

    def statistics(self) -> ProfileStatistics:
        return ProfileStatistics(demand=self.demand.cpu().numpy(), affinity=self.affinity.cpu().numpy())


RouteSamples = Sequence[Sequence[torch.Tensor]]


def profile_route_statistics(samples: RouteSamples, *, num_experts: int) -> ProfileStatistics:
    """Compute the source-conditioned demand and co-selection affinity of
    ``samples`` (a sequence of samples, each one route tensor per source
    rank), as ``profile_route_statistics`` (statistics.py:30-64) does, on the
    GPU."""
    if not samples or not samples[0]:
        raise ValueError("At least one routing sample and source rank are required.")
    if num_experts <= 0:
        raise ValueError("num_experts must be positive.")
    ep_size = len(samples[0])
    for sample in samples:
        if len(sample) != ep_size:
            raise ValueError("All routing samples must contain the same source ranks.")
        for route in sample:
            if route.ndim != 2 or route.shape[1] <= 0:
                raise ValueError("Each route tensor must have shape [tokens, top_k].")
    recorder = RouteStatisticsRecorder(ep_size, num_experts)
    for sample in samples:
        for source_rank, route in enumerate(sample):
            recorder.record(route, source_rank)
            if recorder.invalid():
                raise ValueError("Routing sample contains an invalid logical expert ID.")
    return recorder.statistics()
