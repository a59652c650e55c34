"""The native slot table (libpmoe pmoe_slab_*, host-only) against the
oracle's restatement of the reference's ExpertCache policy.  CPU only."""

import ctypes

import numpy as np
import pytest

from oracle import pmoe_oracle as O
from pagedmoe_amd import _lib
from tests.golden.make_golden import zipf_trace


class NativeSlab:
    def __init__(self, slots, layers, experts, reserve_frac=0.1, lfru=True, scan=8):
        self.lib = _lib.lib()
        self.h = ctypes.c_void_p()
        _lib.check(self.lib.pmoe_slab_create(ctypes.byref(self.h), slots, layers, experts,
                                             reserve_frac, int(lfru), scan), "slab_create")
        self.experts = experts

    def request(self, layer, ids):
        arr = (ctypes.c_int32 * max(1, len(ids)))(*ids)
        mid = (ctypes.c_int32 * max(1, len(ids)))()
        msl = (ctypes.c_int32 * max(1, len(ids)))()
        nm = ctypes.c_int()
        _lib.check(self.lib.pmoe_slab_request(self.h, layer, arr, len(ids), mid, msl,
                                              ctypes.byref(nm)), "slab_request")
        return [(mid[i], msl[i]) for i in range(nm.value)]

    def table(self, layer):
        out = (ctypes.c_int32 * self.experts)()
        _lib.check(self.lib.pmoe_slab_host_table(self.h, layer, out), "host_table")
        return np.array(out[:], np.int32)

    def stats(self):
        st = _lib.SlabStats()
        _lib.check(self.lib.pmoe_slab_stats_get(self.h, ctypes.byref(st)), "stats")
        return st

    def stitch(self):
        return self.lib.pmoe_slab_stitch(self.h)

    def __del__(self):
        self.lib.pmoe_slab_destroy(self.h)


def test_zipf_trace_matches_oracle_config4():
    """96 slots, 384 experts, Zipf(1.1): every table, miss placement and
    counter equal to the oracle's, step by step."""
    trace = zipf_trace(seed=0, steps=400, n_experts=384, k=8)
    nat = NativeSlab(96, 1, 384)
    pol = O.SlotPolicy(96)
    for ids in trace:
        _, placed = pol.step(0, ids)
        got = nat.request(0, ids)
        assert got == placed
        assert np.array_equal(nat.table(0), pol.table(0, 384))
    st = nat.stats()
    assert (st.hits, st.misses, st.evictions) == (pol.hits, pol.misses, pol.evictions)
    assert st.reserve == 9 and st.budget == 87 and st.resident == len(pol.lru)


@pytest.mark.parametrize("lfru", [True, False])
def test_multi_layer_random_requests_match(lfru):
    rng = np.random.default_rng(3)
    nat = NativeSlab(64, 4, 50, lfru=lfru)
    pol = O.SlotPolicy(64, lfru=lfru)
    for _ in range(500):
        layer = int(rng.integers(0, 4))
        ids = rng.integers(0, 50, int(rng.integers(1, 12))).tolist()   # duplicates allowed
        _, placed = pol.step(layer, ids)
        assert nat.request(layer, ids) == placed
        for lyr in range(4):
            assert np.array_equal(nat.table(lyr), pol.table(lyr, 50))


def test_stitch_closed_form_and_unevictable():
    nat = NativeSlab(200, 3, 64)
    assert nat.stitch() == 1
    for lyr in range(3):
        assert nat.table(lyr).tolist() == list(range(lyr * 64, lyr * 64 + 64))
    assert nat.request(1, [5, 6]) == []           # all hits
    st = nat.stats()
    assert st.stitched == 1 and st.hits == 2 and st.evictions == 0


def test_stitch_declines_when_too_small():
    nat = NativeSlab(100, 2, 64)
    assert nat.stitch() == 0


def test_bad_ids_rejected():
    nat = NativeSlab(40, 1, 10)
    with pytest.raises(_lib.PmoeError):
        nat.request(0, [3, 10])
