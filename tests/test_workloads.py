"""The synthetic configurations have the properties BASELINE states."""

import numpy as np

from oracle import moe_oracle as O
from placemoe_amd.workloads import algorithmic_work, make_workload, zipf_copy_counts


def _counts(wl):
    src = wl.sources.numpy() if wl.sources is not None else np.zeros(wl.T, dtype=np.int64)
    return O.histogram(O.map_logical_to_physical(wl.mapping.numpy(), src, wl.selected.numpy()), wl.C)


def test_skew_has_tiny_copies_and_a_dominant_copy():
    wl = make_workload("skew", weights=False)
    counts = _counts(wl)
    assert wl.C == 96 and wl.K == 4 and wl.T == 32768
    assert 0.17 <= (counts <= 16).mean() <= 0.23
    assert counts.max() / counts.sum() > 0.10
    assert (counts == 0).any()


def test_qwen3_replicates_the_32_most_routed_experts():
    wl = make_workload("qwen3", weights=False)
    L = wl.slot_to_logical
    assert wl.C == 160 and np.array_equal(L[:128], np.arange(128))
    demand = np.bincount(wl.selected.numpy().reshape(-1), minlength=128)
    assert set(L[128:]) == set(np.argsort(-demand, kind="stable")[:32])
    M = wl.mapping.numpy()
    assert np.array_equal(L[M], np.tile(np.arange(128), (8, 1)))


def test_fold_copy_allocation():
    wl = make_workload("fold", weights=False)
    copies = np.bincount(wl.slot_to_logical, minlength=128)
    assert wl.C == 256 and copies.min() >= 1 and copies.max() <= 4
    assert copies[0] >= copies[-1]
    c = zipf_copy_counts(np.ones(4), 6)
    assert c.sum() == 6 and c.min() >= 1


def test_dsv3_rows_are_zipf_over_16_slots():
    wl = make_workload("dsv3", weights=False)
    counts = _counts(wl)
    assert wl.T == 65536 and wl.K == 1 and wl.C == 16
    assert counts[0] > counts[-1] and counts.sum() == 65536


def test_toy_layout():
    wl = make_workload("toy", weights=False)
    assert wl.slot_to_logical.tolist() == list(range(8)) + [0, 1, 2, 3]
    w = wl.routing_weights.float()
    assert np.allclose(w.sum(1).numpy(), 1.0, atol=1e-2)


def test_algorithmic_work_formulas():
    w = algorithmic_work(T=16384, K=8, H=2048, I=768, C=160)
    assert w["gemm_fwd_flops"] + w["gemm_bwd_flops"] == 18 * 131072 * 2048 * 768
    assert abs(w["permute_bytes"] / 1e9 - 0.605) < 1e-3


def test_backward_overlap_follows_gemm_size():
    """The two-stream backward is chosen for the short-GEMM shapes (Qwen3,
    fold) and not for the long ones (DeepSeek-V3 share, skew), unless set."""
    from placemoe_amd import experts

    prev = experts.set_backward_overlap(None)
    try:
        sizes = {}
        for name in ("qwen3", "fold", "dsv3", "skew"):
            wl = make_workload(name, weights=False)
            sizes[name] = experts.uses_backward_overlap(wl.T * wl.K, wl.H, wl.I)
        assert sizes == {"qwen3": True, "fold": True, "dsv3": False, "skew": False}
        experts.set_backward_overlap(True)
        assert experts.uses_backward_overlap(65536, 7168, 2048)
        experts.set_backward_overlap(False)
        assert not experts.uses_backward_overlap(1024, 2048, 768)
    finally:
        experts.set_backward_overlap(prev)
