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

    def set_stage(self, first, n):
        _lib.check(self.lib.pmoe_slab_set_stage(self.h, first, n), "set_stage")

    def prefill(self, layer, ids):
        arr = (ctypes.c_int32 * max(1, len(ids)))(*ids)
        mid = (ctypes.c_int32 * max(1, len(ids)))()
        msl = (ctypes.c_int32 * max(1, len(ids)))()
        nm, nu, t = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        _lib.check(self.lib.pmoe_slab_prefill_request(self.h, layer, arr, len(ids), mid, msl,
                                                      ctypes.byref(nm), ctypes.byref(nu),
                                                      ctypes.byref(t)), "prefill_request")
        return t.value, [(mid[i], msl[i]) for i in range(nm.value)], nu.value

    def done(self, ticket):
        _lib.check(self.lib.pmoe_slab_prefill_done(self.h, ticket), "prefill_done")

    def admit(self, layer, ids, clear_pins=True):
        arr = (ctypes.c_int32 * max(1, len(ids)))(*ids)
        mid = (ctypes.c_int32 * max(1, len(ids)))()
        msl = (ctypes.c_int32 * max(1, len(ids)))()
        nm = ctypes.c_int()
        _lib.check(self.lib.pmoe_slab_admit(self.h, layer, arr, len(ids), mid, msl,
                                            ctypes.byref(nm), int(clear_pins)), "admit")
        return [(mid[i], msl[i]) for i in range(nm.value)]

    def install(self, layer, ids):
        arr = (ctypes.c_int32 * max(1, len(ids)))(*ids)
        _lib.check(self.lib.pmoe_slab_install(self.h, layer, arr, len(ids)), "install")

    def dirty(self, layer):
        return self.lib.pmoe_slab_dirty(self.h, layer)

    def capacity(self):
        f, st, room = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        _lib.check(self.lib.pmoe_slab_capacity(self.h, ctypes.byref(f), ctypes.byref(st),
                                               ctypes.byref(room)), "capacity")
        return f.value, st.value, room.value


class _NativeKat:
    """slot_kats adapter over the native policy (layer 0, 64 experts)."""

    def __init__(self, slots, lfru=True, stage=None):
        self.nat = NativeSlab(slots, 1, 64, lfru=lfru)
        if stage is not None:
            self.nat.set_stage(*stage)
        self.rows = {}

    def step(self, ids):
        return self.nat.request(0, ids)

    def prefill(self, ids):
        t, placed, unplaced = self.nat.prefill(0, ids)
        row = {e: int(s) for e, s in enumerate(self.nat.table(0)) if s >= 0}
        row.update(dict(placed))
        self.rows[t] = row
        return t, placed, unplaced

    def compute_row(self, ticket):
        return self.rows[ticket]

    def done(self, ticket):
        self.nat.done(ticket)

    def table(self):
        return {e: int(s) for e, s in enumerate(self.nat.table(0)) if s >= 0}

    @property
    def evictions(self):
        return self.nat.stats().evictions

    @property
    def hits(self):
        return self.nat.stats().hits

    @property
    def misses(self):
        return self.nat.stats().misses

    def admit(self, ids):
        return self.nat.admit(0, ids)

    def install(self, ids):
        self.nat.install(0, ids)


def test_native_flow_admit_known_answer():
    from tests import slot_kats
    slot_kats.run_flow_kat(_NativeKat(8), slot_kats.FLOW_ADMIT)


@pytest.mark.parametrize("seed", [0, 1])
def test_flow_admission_matches_oracle(seed):
    """Flow tokens: admit every layer's routing (pins cleared once per token),
    then install a random subset of the pending reads (copies land in any
    order); placements, tables and counters equal to the oracle's.  A
    pending expert cannot be fetched by the decode or prefill policy."""
    rng = np.random.default_rng(10 + seed)
    slots, layers, experts = 40, 3, 50
    nat = NativeSlab(slots, layers, experts)
    pol = O.SlotPolicy(slots)
    pending = []
    for _ in range(300):
        for layer in range(layers):
            ids = rng.choice(experts, 6, replace=False).tolist()
            placed = nat.admit(layer, ids, clear_pins=layer == 0)
            assert placed == pol.admit(layer, ids, clear_pins=layer == 0)
            pending += [(layer, e) for e, _ in placed]
        rng.shuffle(pending)
        land, pending = pending[:len(pending) // 2], pending[len(pending) // 2:]
        for layer in range(layers):
            ids = [e for lyr, e in land if lyr == layer]
            if ids:
                nat.install(layer, ids)
                pol.install(layer, ids)
        for layer in range(layers):
            assert np.array_equal(nat.table(layer), pol.table(layer, experts))
        st = nat.stats()
        assert (st.hits, st.misses, st.evictions) == (pol.hits, pol.misses, pol.evictions)
    if pending:
        layer, e = pending[0]
        with pytest.raises(_lib.PmoeError, match="not installed"):
            nat.request(layer, [e])


@pytest.mark.parametrize("name", ["LFRU_SECOND_CHANCE", "PINNED_OVER_BUDGET"])
def test_native_lfru_known_answer(name):
    from tests import slot_kats
    kat = getattr(slot_kats, name)
    slot_kats.run_decode_kat(_NativeKat(kat["slots"]), kat)


def test_native_plain_lru_known_answer():
    from tests import slot_kats
    kat = slot_kats.PLAIN_LRU
    slot_kats.run_decode_kat(_NativeKat(kat["slots"], lfru=False), kat)


@pytest.mark.parametrize("name", ["PREFILL_AFTER_DECODE", "PREFILL_COLD"])
def test_native_prefill_known_answer(name):
    from tests import slot_kats
    kat = getattr(slot_kats, name)
    slot_kats.run_prefill_kat(_NativeKat(kat["slots"], stage=kat["stage"]), kat)


@pytest.mark.parametrize("seed", [0, 1])
def test_prefill_and_decode_interleaved_match_oracle(seed):
    """Random interleavings of decode steps and prefill groups (two groups
    open at once, as the overlapped fetch keeps them) on 3 layers: every
    placement, table and counter equal to the oracle's."""
    rng = np.random.default_rng(seed)
    slots, layers, experts, stage = 48, 3, 40, 24
    nat = NativeSlab(slots, layers, experts)
    nat.set_stage(slots + layers, stage)
    pol = O.SlotPolicy(slots)
    pol.set_stage(slots + layers, stage)
    open_groups = []
    for _ in range(400):
        layer = int(rng.integers(0, layers))
        r = rng.random()
        if r < 0.5 or len(open_groups) >= 2:
            for t_n, t_o in open_groups:
                nat.done(t_n)
                pol.prefill_done(t_o)
            open_groups = []
            ids = rng.choice(experts, int(rng.integers(1, 9)), replace=False).tolist()
            assert nat.request(layer, ids) == pol.step(layer, ids)[1]
        else:
            ids = rng.choice(experts, int(rng.integers(1, 30)), replace=False).tolist()
            t_n, placed_n, un_n = nat.prefill(layer, ids)
            t_o, placed_o, un_o = pol.step_prefill(layer, ids)
            assert placed_n == placed_o and un_n == un_o
            open_groups.append((t_n, t_o))
        for lyr in range(layers):
            assert np.array_equal(nat.table(lyr), pol.table(lyr, experts))
        st = nat.stats()
        assert (st.hits, st.misses, st.evictions) == (pol.hits, pol.misses, pol.evictions)
        free, stage_free, _ = nat.capacity()
        assert free == len(pol.free) and stage_free == len(pol.stage_free)


def test_eviction_by_another_layer_marks_its_row_dirty():
    """A fetch of layer 0 that evicts layer 1's expert leaves layer 1's
    device row stale until it is republished (cache.py:821-831, :843-859).
    Host-only: the dirty flag is what pmoe_slab_sync_table acts on."""
    nat = NativeSlab(8, 2, 16)          # budget 4
    nat.request(1, [3])
    nat.request(0, [0, 1, 2])
    assert nat.dirty(0) == 1 and nat.dirty(1) == 1   # nothing published yet
    t1 = nat.table(1)
    assert t1[3] >= 0
    nat.request(0, [4])                 # 5 resident > budget 4: layer 1's 3 is the LRU head
    assert nat.table(1)[3] == -1
    assert nat.dirty(1) == 1
    assert nat.stats().evictions == 1


def test_prefill_request_reports_unplaced_past_stage():
    nat = NativeSlab(8, 1, 64)          # 8 free slots, budget 4, no stage
    t, placed, unplaced = nat.prefill(0, list(range(10)))
    assert [s for _, s in placed] == list(range(8)) and unplaced == 2
    assert nat.stats().prefill_installs == 4 and nat.stats().prefill_starved == 2
    nat.done(t)
    assert nat.capacity()[0] == 4       # the four held slots came back

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
