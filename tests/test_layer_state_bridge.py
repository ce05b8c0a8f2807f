"""LayerStatePlacement reads L and M from the reference's layer state on every
call (no copy), so a hot update made by the reference's controller reaches the
next forward.  Host-side checks; the device routing is in test_gpu_placement."""

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from placemoe_amd.placement import LayerPlacement, LayerStatePlacement, copy_table
from tests.layer_state_standin import StandInLayerState

CPU = torch.device("cpu")


def _state(seed=0, S=4, E=6, extra=5):
    rng = np.random.default_rng(seed)
    L = np.concatenate([np.arange(E), rng.integers(0, E, extra)])
    rng.shuffle(L)
    owners = np.array([np.nonzero(L == e)[0][0] for e in range(E)])
    M = np.array([[rng.choice(np.nonzero(L == e)[0]) for e in range(E)] for _ in range(S)])
    return StandInLayerState(key="layers.1.mlp.experts", num_experts=E,
                             logical_to_physical=torch.as_tensor(owners), slot_to_logical=torch.as_tensor(L),
                             source_logical_to_physical=torch.as_tensor(M)), L, M, rng


def _other_mapping(L, M, rng):
    """Every (source, expert) moved to the next copy of its expert."""
    out = M.copy()
    for s in range(M.shape[0]):
        for e in range(M.shape[1]):
            copies = np.nonzero(L == e)[0]
            out[s, e] = copies[(int(np.nonzero(copies == M[s, e])[0][0]) + 1) % len(copies)]
    return out


def test_reads_the_source_row_and_follows_hot_updates():
    state, L, M, rng = _state()
    p = LayerPlacement.from_layer_state(state, source_rank=2)
    assert isinstance(p, LayerStatePlacement)
    assert p.key == state.key and p.num_experts == 6 and p.num_slots == len(L) and p.source == 0
    np.testing.assert_array_equal(p.slot_to_logical, L)
    got = p.mapping_for_device(CPU)
    assert got.shape == (1, 6) and got.dtype == torch.int64
    np.testing.assert_array_equal(got[0].numpy(), M[2])
    # the state's own device cache is what the op reads
    assert got.data_ptr() == state._device_source_mapping_cache[(CPU, 2)].data_ptr()
    sel = rng.integers(0, 6, (50, 2))
    np.testing.assert_array_equal(O.map_logical_to_physical(got.numpy(), np.zeros(50), sel), M[2][sel])
    M1 = _other_mapping(L, M, rng)
    assert not np.array_equal(M1[2], M[2])
    assert state.hot_update(M1) == 1
    np.testing.assert_array_equal(p.mapping_for_device(CPU)[0].numpy(), M1[2])
    assert p.placement_version == state.placement_version


def test_per_token_sources_use_the_whole_table():
    state, L, M, rng = _state(seed=1)
    p = LayerPlacement.from_layer_state(state, source_rank=0)
    p.token_sources = torch.as_tensor(rng.integers(0, 4, 40))
    np.testing.assert_array_equal(p.mapping_for_device(CPU).numpy(), M)
    M1 = _other_mapping(L, M, rng)
    state.hot_update(M1)
    np.testing.assert_array_equal(p.mapping_for_device(CPU).numpy(), M1)


def test_state_without_source_lut_routes_by_owner():
    state, L, M, _ = _state(seed=2)
    state.source_logical_to_physical = None
    p = LayerPlacement.from_layer_state(state, source_rank=1)
    np.testing.assert_array_equal(p.mapping_for_device(CPU)[0].numpy(), state.logical_to_physical.numpy())
    p.token_sources = torch.zeros(3, dtype=torch.int64)
    with pytest.raises(RuntimeError, match="no source-rank route LUT"):
        p.mapping_for_device(CPU)


def test_install_mapping_writes_the_state_like_the_reference():
    state, L, M, rng = _state(seed=3)
    p = LayerPlacement.from_layer_state(state, source_rank=0)
    p.mapping_for_device(CPU)
    assert state._device_source_mapping_cache
    M1 = _other_mapping(L, M, rng)
    assert not np.array_equal(M, M1)
    assert p.install_mapping(M1) == 1
    assert not state._device_source_mapping_cache
    np.testing.assert_array_equal(state.source_logical_to_physical.numpy(), M1)
    assert p.install_mapping(M1) == 0
    bad = M1.copy()
    bad[0, 0] = int(np.nonzero(L == 1)[0][0])  # a copy of expert 1 for expert 0
    with pytest.raises(RuntimeError, match="wrong expert"):
        p.install_mapping(bad)
    with pytest.raises(RuntimeError, match="shape"):
        p.install_mapping(M1[:, :-1])
    with pytest.raises(RuntimeError, match="invalid slot"):
        p.install_mapping(np.full_like(M1, len(L)))


def test_copy_tables_follow_the_state_layout():
    state, L, _, _ = _state(seed=4)
    p = LayerPlacement.from_layer_state(state, source_rank=0)
    off, slots = p.copy_tables_for_device(CPU)
    ref_off, ref_slots = copy_table(L, 6)
    np.testing.assert_array_equal(off.numpy(), ref_off)
    np.testing.assert_array_equal(slots.numpy(), ref_slots)
    counts = torch.tensor([1, 2, 3], dtype=torch.int32)
    p.record_slot_tokens(counts)
    p.record_slot_tokens(counts)
    assert p.accumulated_slot_tokens.tolist() == [2, 4, 6]
    p.clear_slot_tokens()
    assert p.accumulated_slot_tokens is None
