"""Benchmark: one GPU's share of the PlaceMoE expert layer, forward + backward.

A step is one pass of the hot path over one batch of synthetic input:
route (M table, histogram, scan, stable scatter index) -> permute -> fc1 +
SwiGLU -> fc2 -> weighted combine, then the backward (combine gradient, fc2
dgrad + SwiGLU backward, fc2 and fc1 wgrad, fc1 dgrad, unpermute gradient).
Inputs and weights are resident in HBM before the timed region starts.

Default workload: the DeepSeek-V3-shape share of one EP rank (65536 received
rows, H=7168, I=2048, 16 physical slots with Zipf(1.0) row counts, fwd+bwd):
the configuration the grouped-GEMM target is quoted on and the largest that
fits one GPU.  ``--config`` picks another; ``--config fold`` adds the
replica-gradient fold of both copy gradients (fp32 logical sums, written back
to every copy) to each step.

Prints ONE JSON line.  ``value`` is the layer fwd+bwd time in ms (lower is
better); the grouped-GEMM TFLOP/s and permute GB/s of the same run, the
roofline of the dominant kernel (HIP-event durations on the kernels' stream)
and a CPU baseline (the oracle on a bounded token sample, on the host cores)
ride along.
"""

from __future__ import annotations

import argparse
import contextlib
import json
import os
import sys
import time
from collections import defaultdict

import numpy as np
import torch

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBPS = 8000.0  # MI355X HBM3E

# HBM bytes per launch of the candidate dominant kernels of the default
# workload and of the Qwen3-shape workload, measured on this build in separate
# rocprofv3 runs of this benchmark (FETCH_SIZE, then WRITE_SIZE, each scaled by
# what the counter reads for a 1 GiB device copy: x2.00 and x1.00;
# profiles/hbm_traffic_dsv3.md, profiles/hbm_traffic_qwen3.md).  Counters
# cannot be read from inside a timed run, so the figure is carried here; other
# workloads report traffic null.
MEASURED_TRAFFIC_BYTES = {
    ("dsv3", "fc1_fwd"): (7384 + 769) * 2**20,
    ("dsv3", "fc1_wgrad"): (8868 + 896) * 2**20,
    ("dsv3", "fc1_dgrad"): (6765 + 896) * 2**20,
    ("qwen3", "fc1_fwd"): (2444 + 576) * 2**20,
    ("qwen3", "fc1_wgrad"): (1349 + 961) * 2**20,
    ("qwen3", "fc1_dgrad"): (2083 + 512) * 2**20,
}

# Entry-point call order inside one step; repeated names are told apart by
# their occurrence index.
STAGES = [
    ("pmx_route", 0, "route"),
    ("pmx_moe_scatter", 0, "permute"),
    ("pmx_moe_scatter_src", 0, "permute"),
    ("pmx_gemm_fc1_swiglu_fwd", 0, "fc1_fwd"),
    ("pmx_group_gemm_nt", 0, "fc2_fwd"),
    ("pmx_group_gemm_nt_combine_top1", 0, "fc2_fwd"),
    ("pmx_combine_fwd", 0, "combine_fwd"),
    ("pmx_combine_bwd", 0, "combine_bwd"),
    ("pmx_combine_bwd_top1_rows", 0, "combine_bwd"),
    ("pmx_gemm_fc2_dgrad_swiglu_bwd", 0, "fc2_dgrad"),
    ("pmx_group_gemm_tn", 0, "fc2_wgrad"),
    ("pmx_group_gemm_tn", 1, "fc1_wgrad"),
    ("pmx_group_gemm_nn", 0, "fc1_dgrad"),
    ("pmx_group_gemm_nn_unpermute_top1", 0, "fc1_dgrad"),
    ("pmx_moe_gather", 0, "unpermute_grad"),
    ("pmx_replica_fold", 0, "fold_gate_up"),
    ("pmx_replica_fold", 1, "fold_down"),
]


class EventTimer:
    """Brackets every C-ABI call with HIP events on torch's current stream (the
    stream the kernels are launched on)."""

    def __init__(self):
        self.records = []
        self._seen = defaultdict(int)

    def new_step(self):
        self._seen.clear()

    @contextlib.contextmanager
    def __call__(self, name):
        name = name[:-4] if name.endswith("_f16") else name  # fp16 twins count as their stage
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        idx = self._seen[name]
        self._seen[name] += 1
        s.record()
        yield
        e.record()
        self.records.append((name, idx, s, e))

    def averages(self):
        torch.cuda.synchronize()
        acc = defaultdict(list)
        for name, idx, s, e in self.records:
            acc[(name, idx)].append(s.elapsed_time(e))
        return {k: float(np.mean(v)) for k, v in acc.items()}


def parse():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--config", default="dsv3", choices=["toy", "qwen3", "dsv3", "skew", "fold"])
    p.add_argument("--cpu-sample-tokens", type=int, default=None,
                   help="tokens of the CPU baseline's sample (default: 1/16 of the batch, at least 1024)")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--profile-steps", type=int, default=20, help="extra steps timed per kernel with HIP events")
    p.add_argument("--calibrate-copy", action="store_true",
                   help="first run a plain 1 GiB device copy (reference kernel for HBM-traffic counters)")
    p.add_argument("--vendor-gemm", action="store_true",
                   help="also time the six GEMMs through hipBLASLt, one call per copy, on the same groups")
    p.add_argument("--no-top1-fusion", action="store_true",
                   help="top-1 workloads: run the combine and the unpermute gradient as separate kernels "
                        "instead of in the fc2 and fc1-dgrad epilogues")
    p.add_argument("--no-backward-overlap", action="store_true",
                   help="run the backward's independent GEMM pairs one after the other on one stream")
    p.add_argument("--dtype", default="bf16", choices=["bf16", "fp16"],
                   help="tensor dtype of the layer (the metric is quoted on bf16; fp16 runs the *_f16 "
                        "entry points on the same workload cast to fp16)")
    p.add_argument("--layers", type=int, default=1,
                   help="stack this many layers (own copy weights and placement each) per step; with --config "
                        "fold, each layer's replica fold runs on a side stream beside the backward of the "
                        "layers before it; prints the step time only")
    return p.parse_args()


def layer_stack(wl, dev, layers: int, steps: int, warmup: int, fold: bool):
    """`layers` expert layers in a row through the op boundary (each with its
    own copy weights and registered placement), forward + backward, and with
    `fold` the replica fold of every layer overlapped with the backward
    (``OverlappedReplicaSync``).  Returns ms per step."""
    import placemoe_amd
    from placemoe_amd.fused_moe import hip_fused_moe_forward
    from placemoe_amd.placement import PLACEMENTS, LayerPlacement, LayerPlan

    class Experts(torch.nn.Module):
        def __init__(self, fc1, fc2):
            super().__init__()
            self.gate_up_proj = torch.nn.Parameter(fc1)
            self.down_proj = torch.nn.Parameter(fc2)

    plan = LayerPlan(slot_to_logical=wl.slot_to_logical, source_logical_to_physical=wl.mapping.cpu().numpy(),
                     owner_slots=wl.owner_slots())
    mods = {}
    for i in range(layers):
        key = f"layers.{i}.mlp.experts"
        m = Experts(wl.fc1.detach().clone(), wl.fc2.detach().clone())
        pl = LayerPlacement.from_plan(key, plan, wl.num_experts)
        pl.token_sources = wl.sources
        PLACEMENTS.register(pl, m.gate_up_proj, m.down_proj)
        mods[key] = m
    sync = placemoe_amd.OverlappedReplicaSync(mods) if fold else None
    x = wl.hidden.detach().requires_grad_(True)
    w = wl.routing_weights.detach()
    dout = torch.randn_like(wl.hidden, dtype=torch.float32).to(wl.hidden.dtype)

    def step():
        h = x
        for key, m in mods.items():
            m.zero_grad(set_to_none=True)
            h = hip_fused_moe_forward(wl.num_experts, w, wl.selected, h, None, None, m.down_proj, m.gate_up_proj,
                                      layer_key=key)
        h.backward(dout)
        if sync is not None:
            sync.finish()

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    if sync is not None:
        sync.remove()
    PLACEMENTS.clear()
    return ms


def host_cpu() -> dict:
    """The host's CPU model, its logical CPU count, the CPUs this process may
    run on, and the CPU threads the job is given (OMP_NUM_THREADS, which the
    GPU pool sets to its per-GPU share of the host)."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = os.cpu_count() or 1
    share = os.environ.get("OMP_NUM_THREADS")
    threads = int(share) if share and share.isdigit() and int(share) > 0 else affinity
    return {"model": model, "cpu_count": os.cpu_count(), "affinity": affinity,
            "threads": min(threads, affinity)}


def cpu_baseline(wl, sample_tokens: int | None, backward: bool):
    """The CPU oracle (torch on the host cores) on the first ``sample_tokens``
    tokens of the same workload, scaled linearly to the full token count.
    Runs on every CPU thread the job is given (``host_cpu()['threads']``)."""
    from oracle import moe_oracle as O

    host = host_cpu()
    threads = host["threads"]
    torch.set_num_threads(threads)
    if sample_tokens is None:
        sample_tokens = max(1024, wl.T // 16)
    Ts = min(sample_tokens, wl.T)
    x = wl.hidden[:Ts].cpu()
    w = wl.routing_weights[:Ts].cpu()
    sel = wl.selected[:Ts].cpu().numpy()
    src = wl.sources[:Ts].cpu().numpy() if wl.sources is not None else np.zeros(Ts, dtype=np.int64)
    M = wl.mapping.cpu().numpy()
    fc1, fc2 = wl.fc1.cpu(), wl.fc2.cpu()
    dout = torch.randn((Ts, wl.H), generator=torch.Generator().manual_seed(0)).to(torch.bfloat16)

    def run():
        phys = O.map_logical_to_physical(M, src, sel)
        fwd = O.moe_layer_forward(x, w, phys, fc1, fc2)
        if backward:
            O.moe_layer_backward(dout, fwd, w, fc1, fc2)

    def median_ms(fn):
        fn()  # warm-up
        times = []
        for _ in range(3):
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
        return float(np.median(times)) * 1e3

    ms = median_ms(run)
    value = ms * wl.T / Ts
    sample = (f"oracle layer {'fwd+bwd' if backward else 'fwd'} on {Ts} of {wl.T} tokens, median of 3 "
              f"({ms:.1f} ms), scaled x{wl.T / Ts:g} to the full batch")
    if wl.name == "fold":
        # Replica fold of both copy gradients over the copies of the first
        # `fold_experts` logical experts, scaled by the copy count.
        fold_experts = 4
        L = np.asarray(wl.slot_to_logical)
        picked = np.nonzero(L < fold_experts)[0]
        gsub = [torch.randn((picked.size,) + tuple(t.shape[1:]), generator=torch.Generator().manual_seed(2))
                .to(torch.bfloat16) for t in (fc1, fc2)]
        fold_ms = median_ms(lambda: [O.replica_fold(g, L[picked], fold_experts) for g in gsub])
        value += fold_ms * L.size / picked.size
        sample += (f"; plus the oracle replica fold of both copy gradients over the {picked.size} copies of "
                   f"{fold_experts} experts ({fold_ms:.1f} ms), scaled x{L.size / picked.size:g} to all "
                   f"{L.size} copies")
    sample += (f"; {threads} torch threads on {host['model']} (host: {host['cpu_count']} logical CPUs, "
               f"{host['affinity']} in this process's affinity set)")
    return {"value": value, "unit": "ms", "cores": threads, "kind": "port", "sample": sample,
            "cpu_model": host["model"], "host_cpu_count": host["cpu_count"], "affinity_cpus": host["affinity"]}


def dense_gemm_tflops(dev, n: int = 8192, reps: int = 10) -> float:
    """bf16 TFLOP/s of the vendor library (hipBLASLt through torch.matmul) on
    one dense n x n x n product of random data, x @ w^T with w stored [N, K]
    as the layer's weights are (the vendor's fastest layout here: its plain
    row-major x @ w ran ~12% slower): the measured MFMA reference beside the
    2.5 PFLOP/s spec (random operands keep the part at its power limit, as the
    layer's GEMMs do)."""
    g = torch.Generator(device=dev).manual_seed(9)
    a = torch.randn((n, n), generator=g, device=dev).to(torch.bfloat16)
    w = torch.randn((n, n), generator=g, device=dev).to(torch.bfloat16)
    for _ in range(2):
        c = torch.matmul(a, w.t())
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        c = torch.matmul(a, w.t())
    e.record()
    torch.cuda.synchronize()
    ms = s.elapsed_time(e) / reps
    del a, w, c
    return round(2 * n**3 / (ms * 1e-3) / 1e12, 1)


def device_copy_gbps(dev, reps: int = 10) -> float:
    """Read+write rate of a plain 1 GiB device-to-device copy (torch `copy_`,
    ROCm's blit kernel) on this box, timed with HIP events: a reference point
    for the box's streaming rate beside the 8 TB/s peak."""
    x = torch.empty(2**29, dtype=torch.bfloat16, device=dev)
    y = torch.empty_like(x)
    y.copy_(x)
    torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        y.copy_(x)
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / reps
    del x, y
    return round(2 * 2**30 / (ms * 1e-3) / 1e9, 1)


def aux_measurements(wl, dev, reps: int = 10):
    """Kernels beside the layer step, timed with HIP events around direct
    C-ABI calls (preallocated buffers, no host synchronisation inside):
    route-statistics capture, and the expert-parallel dispatch payload and
    combine aggregation of this rank's routing split over 8 ranks."""
    import ctypes

    from placemoe_amd import _capi, kernels

    lib = _capi.load()
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    i32 = dict(dtype=torch.int32, device=dev)

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(reps):
            fn()
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e) / reps

    T, K, H, C = wl.T, wl.K, wl.H, wl.C
    A = T * K
    ms, gbps = {}, {}
    # route statistics: demand [S,E] and co-selection [S,E,E] counts
    S = int(wl.mapping.shape[0]) if wl.sources is not None else 1
    E = wl.num_experts
    demand = torch.zeros((S, E), dtype=torch.int64, device=dev)
    aff = torch.zeros((S, E, E), dtype=torch.int64, device=dev)
    status = torch.zeros(1, **i32)
    src = wl.sources.data_ptr() if wl.sources is not None else None
    ms["route_statistics"] = timed(lambda: lib.pmx_route_statistics(
        wl.selected.data_ptr(), src, 0, S, E, T, K, demand.data_ptr(), aff.data_ptr(), status.data_ptr(), stream))
    # EP dispatch payload over R ranks of C/R slots
    R = 8 if C % 8 == 0 else 4
    r = kernels.route(wl.selected, C, mapping=wl.mapping, sources=wl.sources)
    w = wl.routing_weights.contiguous()
    outs = dict(ac=torch.empty(R, **i32), ao=torch.empty(R + 1, **i32), uc=torch.empty(R, **i32),
                uo=torch.empty(R + 1, **i32), sh=torch.empty((A, H), dtype=torch.bfloat16, device=dev),
                ut=torch.empty(A, **i32), meta=torch.empty((A, 3), **i32),
                sw=torch.empty(A, dtype=torch.bfloat16, device=dev), tr=torch.empty(A, **i32))
    ws = torch.empty(lib.pmx_ep_payload_workspace_bytes(A, R), dtype=torch.uint8, device=dev)
    o = outs
    ms["ep_dispatch_payload"] = timed(lambda: lib.pmx_ep_dispatch_payload(
        r.phys.data_ptr(), wl.hidden.data_ptr(), w.data_ptr(), T, K, H, R, C // R, o["ac"].data_ptr(),
        o["ao"].data_ptr(), o["uc"].data_ptr(), o["uo"].data_ptr(), o["sh"].data_ptr(), o["ut"].data_ptr(),
        o["meta"].data_ptr(), o["sw"].data_ptr(), o["tr"].data_ptr(), status.data_ptr(), ws.data_ptr(),
        ws.numel(), stream))
    U = int(o["uc"].sum().item())
    gbps["ep_dispatch_payload"] = (4 * U * H + 22 * A + 4 * U) / (ms["ep_dispatch_payload"] * 1e-3) / 1e9
    # combine aggregation: this rank's assignments in send order as a receive buffer
    src_rank = torch.repeat_interleave(torch.arange(R, device=dev, dtype=torch.int32), o["ac"].long())
    src_tok = o["meta"][:, 2].contiguous()
    y = torch.randn((A, H), device=dev).to(torch.bfloat16)
    pos = r.pos.reshape(-1).contiguous()
    out = torch.empty((A, H), dtype=torch.bfloat16, device=dev)
    run_off = torch.empty(A + 1, **i32)
    rank_runs = torch.empty(R, **i32)
    nruns = torch.empty(1, **i32)
    cws = torch.empty(lib.pmx_ep_combine_workspace_bytes(A), dtype=torch.uint8, device=dev)
    ms["ep_combine_aggregate"] = timed(lambda: lib.pmx_ep_combine_aggregate(
        y.data_ptr(), pos.data_ptr(), o["sw"].data_ptr(), src_rank.data_ptr(), src_tok.data_ptr(), A, H, R,
        out.data_ptr(), run_off.data_ptr(), rank_runs.data_ptr(), nruns.data_ptr(), status.data_ptr(),
        cws.data_ptr(), cws.numel(), stream))
    Ur = int(nruns.item())
    gbps["ep_combine_aggregate"] = (2 * A * H + 2 * Ur * H + 14 * A) / (ms["ep_combine_aggregate"] * 1e-3) / 1e9
    cfg = {"ep_ranks": R, "unique_rank_token_pairs": U}
    del outs, o, ws, y, out, cws
    cfg.update(replica_exchange_measurement(wl, dev, R, ms, gbps))
    return ({k: round(v, 4) for k, v in ms.items()}, {k: round(v, 1) for k, v in gbps.items()}, cfg)


def replica_exchange_measurement(wl, dev, R, ms, gbps):
    """Rank 0's side of the cross-rank replica-gradient exchange with the
    workload's copies split over R ranks (C/R slots each): its pack and its
    finish (the received buffers are the other ranks' real packs), bf16 copy
    gradients of the layer's shapes."""
    from placemoe_amd.replica import ReplicaGradExchange, replica_grad_schedule

    C, H, I = wl.C, wl.H, wl.I
    nl = C // R
    L = np.asarray(wl.slot_to_logical)
    owners = np.asarray(wl.owner_slots())
    sched = [replica_grad_schedule(L, owners, nl, r, R) for r in range(R)]
    g = torch.Generator(device=dev).manual_seed(11)
    grads = [(torch.randn((nl, 2 * I, H), generator=g, device=dev).to(torch.bfloat16),
              torch.randn((nl, H, I), generator=g, device=dev).to(torch.bfloat16)) for _ in range(R)]
    ex = [ReplicaGradExchange(sched[r], r, grads[r]) for r in range(R)]
    pairwise = sched[0].pairwise
    sends = [e.pairwise_send() if pairwise else e.owner_reduce_send() for e in ex]
    recv0 = {}
    for src, per_dtype in enumerate(sends):
        for dtype, bufs in per_dtype.items():
            if 0 in bufs:
                recv0.setdefault(dtype, {})[src] = bufs[0]
    pack = ex[0].pairwise_send if pairwise else ex[0].owner_reduce_send
    finish = ex[0].pairwise_finish if pairwise else ex[0].owner_reduce_finish

    def kernel_ms(fn, entry, reps=5):
        # HIP events around each launch only: the host builds the item tables
        # between launches, which is not kernel time.
        from placemoe_amd import _capi

        fn()
        timer = EventTimer()
        _capi.set_timer(timer)
        for _ in range(reps):
            timer.new_step()
            fn()
        _capi.set_timer(None)
        return sum(v for (name, _), v in timer.averages().items() if name == entry)

    b = ex[0].bytes_moved
    pack()
    per_pack = ex[0].bytes_moved - b
    ms["replica_exchange_pack"] = kernel_ms(pack, "pmx_replica_exchange_pack")
    b = ex[0].bytes_moved
    finish(recv0)
    per_finish = ex[0].bytes_moved - b
    ms["replica_exchange_finish"] = kernel_ms(lambda: finish(recv0), "pmx_replica_exchange_unpack")
    if per_pack:
        gbps["replica_exchange_pack"] = per_pack / (ms["replica_exchange_pack"] * 1e-3) / 1e9
    if per_finish:
        gbps["replica_exchange_finish"] = per_finish / (ms["replica_exchange_finish"] * 1e-3) / 1e9
    return {"replica_exchange": {"ranks": R, "slots_per_rank": nl, "pairwise": pairwise,
                                 "groups_on_rank0": sum(1 for x in sched[0].groups if x.local_slots),
                                 "remote_peers_rank0": sorted(next(iter(recv0.values()), {}).keys()),
                                 "pack_bytes": per_pack, "finish_bytes": per_finish}}


def vendor_gemms(wl, dev, reps: int = 5):
    """The layer's six GEMMs on the same per-copy row groups through the
    vendor library (hipBLASLt via torch.matmul, one call per non-empty copy),
    timed with HIP events: a library reference for the grouped kernel."""
    from placemoe_amd import kernels

    H, I = wl.H, wl.I
    r = kernels.route(wl.selected, wl.C, mapping=wl.mapping, sources=wl.sources)
    counts = [int(c) for c in r.counts.cpu().tolist()]
    g = torch.Generator(device=dev).manual_seed(5)
    bf = dict(dtype=torch.bfloat16, device=dev)
    A = sum(counts)
    x = torch.randn((A, H), generator=g, device=dev).to(torch.bfloat16)
    act = torch.randn((A, I), generator=g, device=dev).to(torch.bfloat16)
    dy = torch.randn((A, H), generator=g, device=dev).to(torch.bfloat16)
    dg1 = torch.randn((A, 2 * I), generator=g, device=dev).to(torch.bfloat16)
    w1, w2 = wl.fc1.detach(), wl.fc2.detach()
    rows, o = [], 0
    for c, n in enumerate(counts):
        if n:
            rows.append((c, slice(o, o + n)))
        o += n
    outs = {"fc1_fwd": torch.empty((A, 2 * I), **bf), "fc2_fwd": torch.empty((A, H), **bf),
            "fc2_dgrad": torch.empty((A, I), **bf), "fc1_dgrad": torch.empty((A, H), **bf),
            "fc2_wgrad": torch.empty((wl.C, H, I), **bf), "fc1_wgrad": torch.empty((wl.C, 2 * I, H), **bf)}
    calls = {
        "fc1_fwd": lambda c, s: torch.matmul(x[s], w1[c].t(), out=outs["fc1_fwd"][s]),
        "fc2_fwd": lambda c, s: torch.matmul(act[s], w2[c].t(), out=outs["fc2_fwd"][s]),
        "fc2_dgrad": lambda c, s: torch.matmul(dy[s], w2[c], out=outs["fc2_dgrad"][s]),
        "fc2_wgrad": lambda c, s: torch.matmul(dy[s].t(), act[s], out=outs["fc2_wgrad"][c]),
        "fc1_wgrad": lambda c, s: torch.matmul(dg1[s].t(), x[s], out=outs["fc1_wgrad"][c]),
        "fc1_dgrad": lambda c, s: torch.matmul(dg1[s], w1[c], out=outs["fc1_dgrad"][s]),
    }
    flops = {"fc1_fwd": 2 * A * H * 2 * I, "fc2_fwd": 2 * A * I * H, "fc2_dgrad": 2 * A * H * I,
             "fc2_wgrad": 2 * A * H * I, "fc1_wgrad": 2 * A * 2 * I * H, "fc1_dgrad": 2 * A * 2 * I * H}
    ms = {}
    for name, fn in calls.items():
        for c, s in rows:
            fn(c, s)
        torch.cuda.synchronize()
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s0.record()
        for _ in range(reps):
            for c, s in rows:
                fn(c, s)
        s1.record()
        torch.cuda.synchronize()
        ms[name] = s0.elapsed_time(s1) / reps
    total = sum(ms.values())
    return {"library": "hipBLASLt (torch.matmul), one call per non-empty copy",
            "kernel_ms": {k: round(v, 4) for k, v in ms.items()},
            "tflops": {k: round(flops[k] / (ms[k] * 1e-3) / 1e12, 1) for k in ms},
            "gemm_tflops": round(sum(flops.values()) / (total * 1e-3) / 1e12, 1)}


def main():
    args = parse()
    if args.gpus != 1:
        print(
            json.dumps({"error": f"bench.py measures one GPU's share; --gpus {args.gpus} is not supported "
                                 "(the multi-GPU exchange is outside this build)"}),
            flush=True,
        )
        return 2
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import placemoe_amd  # noqa: F401
    from placemoe_amd import _capi, experts
    from placemoe_amd.workloads import algorithmic_work, make_workload

    if args.no_top1_fusion:
        experts.set_top1_fusion(False)
    if args.no_backward_overlap:
        experts.set_backward_overlap(False)

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.calibrate_copy:
        # 2^29 bf16 = 1 GiB read + 1 GiB written by one elementwise copy kernel
        src = torch.ones(1 << 29, dtype=torch.bfloat16, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    wl = make_workload(args.config, device=dev)
    dt = torch.float16 if args.dtype == "fp16" else torch.bfloat16
    if dt != torch.bfloat16:
        for f in ("hidden", "routing_weights", "fc1", "fc2"):
            setattr(wl, f, getattr(wl, f).to(dt))
    backward = not wl.meta.get("forward_only", False)
    T, K, H, I, C = wl.T, wl.K, wl.H, wl.I, wl.C
    work = algorithmic_work(T, K, H, I, C)
    x = wl.hidden.requires_grad_(backward)
    w = wl.routing_weights.requires_grad_(backward)
    fc1 = wl.fc1.requires_grad_(backward)
    fc2 = wl.fc2.requires_grad_(backward)
    dout = torch.randn((T, H), device=dev, generator=torch.Generator(device=dev).manual_seed(1)).to(dt)

    fold = args.config == "fold"
    if args.layers > 1:
        ms = layer_stack(wl, dev, args.layers, args.steps, args.warmup, fold)
        print(json.dumps({"metric": "MoE layer fwd+bwd ms", "value": round(ms, 4), "unit": "ms", "n_gpus": 1,
                          "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
                          "higher_is_better": False, "dtype": args.dtype, "data": "synthetic",
                          "config": {"workload": args.config, "layers": args.layers,
                                     "replica_fold": "overlapped per layer" if fold else None}}), flush=True)
        return 0
    if fold:
        from placemoe_amd import kernels
        from placemoe_amd.placement import copy_table

        off_np, slots_np = copy_table(wl.slot_to_logical, wl.num_experts)
        copy_off = torch.as_tensor(off_np, dtype=torch.int32, device=dev)
        copy_slots = torch.as_tensor(slots_np, dtype=torch.int32, device=dev)

    def step():
        for p in (x, w, fc1, fc2):
            p.grad = None
        out = experts.expert_layer(x, w, wl.selected, fc2, fc1_1_2_weight=fc1, mapping=wl.mapping,
                                   sources=wl.sources)
        if backward:
            out.backward(dout)
        if fold:
            for g in (fc1.grad, fc2.grad):
                kernels.replica_fold(g, copy_off, copy_slots, wl.num_experts, writeback=True)
        return out

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / args.steps

    # Per-kernel durations: the backward's independent GEMM pairs, which the
    # timed steps may run on two streams, are serialized here so that each
    # kernel's events bracket it alone.
    timed_overlap = experts.uses_backward_overlap(T * K, H, I)
    timer = EventTimer()
    overlap = experts.set_backward_overlap(False)
    _capi.set_timer(timer)
    for _ in range(args.profile_steps):
        timer.new_step()
        step()
    _capi.set_timer(None)
    experts.set_backward_overlap(overlap)
    avg = timer.averages()
    kernels_ms = {label: avg.get((name, idx)) for name, idx, label in STAGES if (name, idx) in avg}
    if not kernels_ms:
        print(json.dumps({"metric": "MoE layer fwd+bwd ms", "value": round(ms_per_step, 4), "unit": "ms",
                          "note": "no per-kernel timing (--profile-steps 0)"}), flush=True)
        return 0

    flops = {"fc1_fwd": work["fc1_fwd_flops"], "fc2_fwd": work["fc2_fwd_flops"],
             "fc2_dgrad": work["fc2_dgrad_flops"], "fc2_wgrad": work["fc2_wgrad_flops"],
             "fc1_wgrad": work["fc1_wgrad_flops"], "fc1_dgrad": work["fc1_dgrad_flops"]}
    gemm_ms = sum(kernels_ms[k] for k in flops if k in kernels_ms)
    gemm_flops = sum(v for k, v in flops.items() if k in kernels_ms)
    gemm_tflops = gemm_flops / (gemm_ms * 1e-3) / 1e12
    dominant = max((k for k in flops if k in kernels_ms), key=lambda k: kernels_ms[k])
    dom_tflops = flops[dominant] / (kernels_ms[dominant] * 1e-3) / 1e12
    permute_gbps = work["permute_bytes"] / (kernels_ms["permute"] * 1e-3) / 1e9
    bw = {"permute": work["permute_bytes"], "combine_fwd": work["combine_fwd_bytes"],
          "combine_bwd": work["combine_bwd_bytes"], "unpermute_grad": work["unpermute_grad_bytes"],
          "route": work["route_bytes"]}
    if fold:
        # bf16 copy gradients read, fp32 logical sums written, totals written back to every copy
        for label, per_copy in (("fold_gate_up", 2 * I * H), ("fold_down", H * I)):
            bw[label] = C * per_copy * 2 + wl.num_experts * per_copy * 4 + C * per_copy * 2
    bandwidth = {k: round(v / (kernels_ms[k] * 1e-3) / 1e9, 1) for k, v in bw.items() if k in kernels_ms}
    # Top-1 layers run the combine in fc2's epilogue and the unpermute gradient
    # in the fc1 dgrad's: those two kernels' times are inside the GEMMs'.
    fused = {}
    if ("pmx_group_gemm_nt_combine_top1", 0) in avg:
        fused["fc2_fwd"] = "combine_fwd"
    if ("pmx_group_gemm_nn_unpermute_top1", 0) in avg:
        fused["fc1_dgrad"] = "unpermute_grad"

    result = {
        "metric": "MoE layer fwd+bwd ms; grouped-GEMM TFLOP/s (%MFMA peak); permute GB/s",
        "value": round(ms_per_step, 4),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.dtype,
        "data": "synthetic",
        "config": {"workload": f"config{['toy', 'qwen3', 'dsv3', 'skew', 'fold'].index(args.config) + 1}-"
                               f"{args.config}", "tokens": T, "top_k": K, "hidden": H, "moe_intermediate": I,
                   "physical_copies": C, "logical_experts": wl.num_experts, "seed": wl.seed,
                   "pass": "fwd+bwd" if backward else "fwd"},
        "gemm_tflops": round(gemm_tflops, 1),
        "gemm_frac_mfma_peak": round(gemm_tflops / PEAK_BF16_TFLOPS, 4),
        "permute_gbps": round(permute_gbps, 1),
        "permute_frac_hbm_peak": round(permute_gbps / PEAK_HBM_GBPS, 4),
        "kernel_ms": {k: round(v, 4) for k, v in kernels_ms.items()},
        "kernel_timing": "HIP events per kernel over --profile-steps extra steps, backward GEMM pairs serialized",
        "backward_streams": 2 if timed_overlap else 1,
        "bandwidth_gbps": bandwidth,
        "fused": fused,
        "roofline": {"kernel": dominant, "bound": "mfma", "achieved": round(dom_tflops, 1),
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s", "frac": round(dom_tflops / PEAK_BF16_TFLOPS, 4),
                     "traffic": MEASURED_TRAFFIC_BYTES.get((args.config, dominant))},
        "cpu_baseline": None,
    }
    aux_ms, aux_bw, aux_cfg = aux_measurements(wl, dev)
    result["aux_kernel_ms"] = aux_ms
    result["aux_bandwidth_gbps"] = aux_bw
    result["aux_config"] = aux_cfg
    result["device_copy_gbps"] = device_copy_gbps(dev)
    result["dense_vendor_gemm_tflops"] = dense_gemm_tflops(dev)
    result["roofline"]["frac_of_dense_vendor_gemm"] = round(dom_tflops / result["dense_vendor_gemm_tflops"], 4)
    if args.vendor_gemm:
        result["vendor_gemm"] = vendor_gemms(wl, dev)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(wl, args.cpu_sample_tokens, backward)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
