"""The allocation-free routing entry point (pmx_route_noalloc) against
pmx_route through the C ABI: bit-exact on two calls in a row (the second
smaller, so stale scratch from the first must not leak into it), the status
word on a bad id, and refusal of a chunk table larger than the static
scratch."""

import pytest
import torch

from placemoe_amd import _capi
from placemoe_amd.workloads import make_workload
from tests.helpers import assert_exact

pytestmark = pytest.mark.gpu


def _stream(dev):
    return torch.cuda.current_stream(dev).cuda_stream


def _route_both(dev, sel, M, src, C):
    T, K = sel.shape
    S, E = (M.shape if M is not None else (1, C))
    i32 = dict(dtype=torch.int32, device=dev)
    lib = _capi.load()
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    outs = []
    for noalloc in (False, True):
        phys, pos = torch.full((T, K), -7, **i32), torch.full((T, K), -7, **i32)
        counts, offsets = torch.full((C,), -7, **i32), torch.full((C + 1,), -7, **i32)
        if noalloc:
            status = torch.full((1,), -7, **i32)
            _capi.call("pmx_route_noalloc", ptr(sel), ptr(M), ptr(src), 0, S, E, T, K, C, ptr(phys), ptr(counts),
                       ptr(offsets), ptr(pos), ptr(status), _stream(dev))
            st = int(status.item())
        else:
            ws_bytes = lib.pmx_route_workspace_bytes(T * K, C)
            ws = torch.full((ws_bytes,), 0x5A, dtype=torch.uint8, device=dev)
            _capi.call("pmx_route", ptr(sel), ptr(M), ptr(src), 0, S, E, T, K, C, ptr(phys), ptr(counts),
                       ptr(offsets), ptr(pos), ptr(ws), ws_bytes, _stream(dev))
            st = int(ws[:4].view(torch.int32).item())
        outs.append((phys, counts, offsets, pos, st))
    return outs


def _assert_same(outs, label):
    (p0, c0, o0, q0, s0), (p1, c1, o1, q1, s1) = outs
    assert_exact(p1, p0, f"{label} phys")
    assert_exact(c1, c0, f"{label} counts")
    assert_exact(o1, o0, f"{label} offsets")
    assert_exact(q1, q0, f"{label} pos")
    assert s1 == s0, f"{label}: status {s1} != {s0}"


def test_noalloc_route_matches_route_on_consecutive_calls(cuda):
    big = make_workload("qwen3", device=cuda, weights=False)  # 131072 assignments over 160 copies
    small = make_workload("skew", device=cuda, tokens=5000, weights=False)  # 20000 over 96
    for label, wl in (("qwen3 full", big), ("skew 5000", small)):
        print(f"noalloc {label}: T={wl.T} K={wl.K} C={wl.C}", flush=True)
        outs = _route_both(cuda, wl.selected, wl.mapping, wl.sources, wl.C)
        _assert_same(outs, label)
        assert outs[1][4] == 0
    # a bad expert id: both entry points clamp it and report it
    sel = small.selected.clone()
    sel[3, 2] = 999
    outs = _route_both(cuda, sel, small.mapping, small.sources, small.C)
    _assert_same(outs, "bad id")
    assert outs[1][4] == 1
    # and the next good call reports 0 again
    outs = _route_both(cuda, small.selected[:100].contiguous(), small.mapping, small.sources[:100].contiguous(),
                       small.C)
    _assert_same(outs, "after bad id")
    assert outs[1][4] == 0


def test_noalloc_route_identity_and_empty(cuda):
    g = torch.Generator(device=cuda).manual_seed(4)
    sel = torch.randint(0, 33, (777, 3), generator=g, device=cuda)
    _assert_same(_route_both(cuda, sel, None, None, 33), "identity")
    empty = torch.empty((0, 3), dtype=torch.int64, device=cuda)
    outs = _route_both(cuda, empty, None, None, 33)
    _assert_same(outs, "empty")
    assert outs[1][1].cpu().tolist() == [0] * 33


def test_noalloc_route_refuses_tables_beyond_scratch(cuda):
    # 8000 copies x 1024 chunks of int32 is 32 MB, far beyond the 8 MiB scratch.
    lib = _capi.load()
    T, K, C = 600_000, 1, 8000
    assert lib.pmx_route_workspace_bytes(T * K, C) > 8 << 20
    sel = torch.zeros((T, K), dtype=torch.int64, device=cuda)
    i32 = dict(dtype=torch.int32, device=cuda)
    phys, pos = torch.empty((T, K), **i32), torch.empty((T, K), **i32)
    counts, offsets, status = torch.empty(C, **i32), torch.empty(C + 1, **i32), torch.zeros(1, **i32)
    rc = lib.pmx_route_noalloc(sel.data_ptr(), None, None, 0, 1, C, T, K, C, phys.data_ptr(), counts.data_ptr(),
                               offsets.data_ptr(), pos.data_ptr(), status.data_ptr(), _stream(cuda))
    assert rc == _capi.PMX_ERR_SHAPE
