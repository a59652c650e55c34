"""The slot-safety ledger (pagedmoe_amd/verify.py), on the CPU.

1. The checker on hand-written event sequences: each violation it names
   is flagged, and the orderings that make a write safe are not.
2. The schedules the streaming code produces -- prefill fetch groups whose
   copies run under the previous group's compute, decode with speculative
   reads and no synchronisation between layers, flow decode -- driven
   through a CPU twin of the cache (tests/cache_twin.py) whose copies land
   a few stream positions after they are issued: no conflicts.
3. Planted mistakes in the twin (a fence left out, a join left out, a row
   not republished) are caught, so the clean runs above mean something.

Reference behaviour: PAGED_MOE_SLAB_VERIFY's WRITE-WHILE-COMPUTE and
OWNER-MISMATCH checks (cache.py:554-556, :1171-1206).
"""

import numpy as np
import pytest
import torch

from pagedmoe_amd import config, kernels as K, verify as V
from pagedmoe_amd.ring import PrefetchRing
from pagedmoe_amd.streaming import StreamedSwitchGLU
from tests.cache_twin import DEMAND, SLAB, SPEC, TwinCache

E = 32


# ---------------------------------------------------------------- the checker

def ledger():
    return V.SlotLedger(SLAB, [DEMAND, SPEC], lambda d, s, n: (d, divmod(s, E)),
                        print_conflicts=False)


def copy(eng, slot, layer, e, batch=-1):
    return [(V.SUBMIT, eng, slot, layer * E + e, 1), (V.ISSUE, eng, batch, 0, 0)]


def row(layer, mapping):
    return [(V.PUBLISH, SLAB, layer, 0, 0)] + [(V.ROW, SLAB, layer, e, s)
                                               for e, s in mapping.items()]


def compute(layer):
    return [(V.COMPUTE, SLAB, layer, 0, 0)]


def kinds(led):
    return [c.split()[1] for c in led.conflicts]


def test_fenced_joined_copy_is_clean():
    led = ledger()
    led.feed(row(0, {3: 5}) + compute(0)                       # slot 5 read
             + [(V.FENCE, DEMAND, 0, 0, 0)] + copy(DEMAND, 5, 1, 7)   # overwritten after a fence
             + [(V.JOIN, DEMAND, 0, 0, 0)] + row(1, {7: 5}) + compute(1))
    assert led.conflicts == []


def test_copy_without_a_fence_after_a_read_is_write_while_compute():
    led = ledger()
    led.feed(row(0, {3: 5}) + compute(0) + copy(DEMAND, 5, 1, 7))
    assert kinds(led) == ["WRITE-WHILE-COMPUTE"]
    led = ledger()                                              # a fence older than the read
    led.feed([(V.FENCE, DEMAND, 0, 0, 0)] + row(0, {3: 5}) + compute(0) + copy(DEMAND, 5, 1, 7))
    assert kinds(led) == ["WRITE-WHILE-COMPUTE"]


def test_compute_before_the_join_is_read_before_landed():
    led = ledger()
    led.feed(copy(DEMAND, 2, 0, 4) + row(0, {4: 2}) + compute(0))
    assert kinds(led) == ["READ-BEFORE-LANDED"]
    for done in ([(V.JOIN, DEMAND, 0, 0, 0)], [(V.HOST_SYNC, DEMAND, 0, 0, 0)]):
        led = ledger()
        led.feed(copy(DEMAND, 2, 0, 4) + done + row(0, {4: 2}) + compute(0))
        assert led.conflicts == []
    led = ledger()                                              # a batch join covers its batch only
    led.feed(copy(SPEC, 2, 0, 4, batch=1) + copy(SPEC, 3, 0, 5, batch=2)
             + [(V.BATCH_JOIN, SPEC, 1, 0, 0)] + row(0, {4: 2, 5: 3}) + compute(0))
    assert kinds(led) == ["READ-BEFORE-LANDED"] and "slot=3" in led.conflicts[0]


def test_stale_row_is_owner_mismatch():
    led = ledger()
    led.feed(row(0, {3: 5}) + compute(0) + [(V.FENCE, DEMAND, 0, 0, 0)]
             + copy(DEMAND, 5, 1, 7) + [(V.JOIN, DEMAND, 0, 0, 0)] + compute(0))
    assert kinds(led) == ["OWNER-MISMATCH"]


def test_unordered_copies_into_one_slot_are_write_over_write():
    led = ledger()
    led.feed(copy(SPEC, 6, 0, 1, batch=0) + copy(DEMAND, 6, 0, 2))
    assert kinds(led) == ["WRITE-OVER-WRITE"]
    led = ledger()                                              # host waited for the first
    led.feed(copy(SPEC, 6, 0, 1, batch=0) + [(V.HOST_DONE, SPEC, 0, 0, 0)] + copy(DEMAND, 6, 0, 2))
    assert led.conflicts == []
    led = ledger()                                              # joined, then fenced
    led.feed(copy(SPEC, 6, 0, 1, batch=0) + [(V.BATCH_JOIN, SPEC, 0, 0, 0),
                                             (V.FENCE, DEMAND, 0, 0, 0)] + copy(DEMAND, 6, 0, 2))
    assert led.conflicts == []


def test_events_of_other_slabs_are_ignored():
    led = ledger()
    led.feed([(V.COMPUTE, 999, 0, 0, 0), (V.SUBMIT, 998, 1, 1, 1), (V.ISSUE, 998, -1, 0, 0)])
    assert led.conflicts == [] and led.pos == 0


# ---------------------------------------------------------------- schedules

@pytest.fixture
def cpu_seam(monkeypatch):
    monkeypatch.setattr(K, "note_workspace_errors", lambda: None)
    monkeypatch.setattr(K, "raise_workspace_errors", lambda: None)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)


class _NoFence:
    def record(self):
        pass

    def synchronize(self):
        pass


def build(n_layers, slots, stage=0, lag=3):
    keys = [f"layers.{i}.mlp.switch_mlp" for i in range(n_layers)]
    twin = TwinCache(slots, keys, E, stage_slots=stage, lag=lag)
    layers = [StreamedSwitchGLU(k, None, twin) for k in keys]
    ring = PrefetchRing(layers, twin)
    ring._fence = _NoFence()
    return twin, layers, ring


def fake_compute(hidden):
    def run(ids, table):
        return torch.zeros(ids.shape + (hidden,))
    return run


def routing(rng, n, k=4):
    return torch.from_numpy(np.stack([rng.choice(E, k, replace=False) for _ in range(n)])
                            .astype(np.int32))


def test_prefill_groups_schedule_is_race_free(cpu_seam):
    """96-token prefill of 3 layers through 16 routed + 8 stage slots: each
    layer's misses come in several groups, group i+1's copies issued under
    group i's compute."""
    twin, layers, _ = build(3, 16, stage=8)
    rng = np.random.default_rng(0)
    overlapped = 0
    for s in layers:
        ind2 = routing(rng, 96)
        before = twin.ledger.counts["COMPUTE"]
        s.call(torch.zeros(96, 8), ind2, fake_compute(8))       # the seam's own dispatch
        assert twin.ledger.counts["COMPUTE"] - before >= 3       # several groups
        groups = s.last_groups
        overlapped += sum(1 for g in groups[1:] if g[0] == "open")
    assert overlapped > 0                                        # copies under compute happened
    assert twin.ledger.conflicts == [], twin.ledger.conflicts[:3]
    assert twin.ledger.counts["ISSUE"] > 0


def test_planted_missing_fence_is_caught(cpu_seam, monkeypatch):
    twin, layers, _ = build(3, 16, stage=8)
    monkeypatch.setattr(twin, "fence", lambda: None)
    rng = np.random.default_rng(0)
    for s in layers:
        s.run_passes(routing(rng, 96), fake_compute(8))
    assert "WRITE-WHILE-COMPUTE" in kinds(twin.ledger)


def test_planted_missing_join_is_caught(cpu_seam, monkeypatch):
    twin, layers, _ = build(3, 16, stage=8)
    monkeypatch.setattr(twin, "join", lambda: None)
    rng = np.random.default_rng(0)
    for s in layers:
        s.run_passes(routing(rng, 96), fake_compute(8))
    assert "READ-BEFORE-LANDED" in kinds(twin.ledger)


class _Guess:
    """Route prediction stand-in: the target layer's true next routing
    (from the test's schedule) plus one wrong id."""

    def __init__(self, schedule, layer, clock):
        self.schedule, self.layer, self.clock = schedule, layer, clock

    def predict_ids(self, x, slack):
        ids = list(self.schedule[self.clock[0]][self.layer][0].tolist())
        wrong = next(e for e in range(E) if e not in ids)
        return torch.tensor([ids + [wrong]], dtype=torch.int32)


def test_decode_speculation_schedule_without_synchronisation(cpu_seam):
    """6 decode layers, 24 routed slots, prediction on: guesses read into
    free slots under later layers' compute and claimed by their targets,
    with nothing waited for between layers (copies land `lag` positions
    after issue)."""
    twin, layers, ring = build(6, 24, lag=4)
    ring.governor.set_mode("on")
    rng = np.random.default_rng(1)
    schedule = [[routing(rng, 1) for _ in layers] for _ in range(12)]
    clock = [0]
    for i, s in enumerate(layers):
        s.pred = _Guess(schedule, i, clock)
    x2 = torch.zeros(1, 8)
    for t in range(12):
        clock[0] = t
        for i, s in enumerate(layers):
            s.call(x2, schedule[t][i], fake_compute(8))
    st = twin.pol
    assert twin.ledger.counts["SUBMIT"] > 0
    assert ring.stats()["pred_issued"] > 0 and ring.spec_reads > 0
    assert twin.ledger.conflicts == [], twin.ledger.conflicts[:3]
    assert st.hits > 0


def test_flow_schedule_is_race_free(cpu_seam, monkeypatch):
    """Flow decode: residency once per token (admit behind a fence at the
    stream's tail, install once landed, rows republished), layers with no
    host round trip."""
    monkeypatch.setattr(config, "FLOW_WARMUP", 1)
    monkeypatch.setattr(config, "FLOW_WARM_HIT", 0.0)
    monkeypatch.setattr(config, "FLOW_MAX_CRIT", 0.0)      # no miss-rate exit here
    twin, layers, ring = build(3, 16, lag=2)
    ring.flow = True
    rng = np.random.default_rng(2)
    x2 = torch.zeros(1, 8)
    hot = [routing(rng, 1) for _ in layers]
    for t in range(16):
        for i, s in enumerate(layers):
            ind2 = hot[i] if t % 3 else routing(rng, 1)
            s.call(x2, ind2, fake_compute(8))
    assert ring.flow_tokens > 10
    assert twin.ledger.counts["BATCH_JOIN"] > 0
    assert twin.ledger.conflicts == [], twin.ledger.conflicts[:3]


def test_planted_stale_flow_rows_are_caught(cpu_seam, monkeypatch):
    """The same flow run with begin_token's row republish left out: a layer
    computes through a row that still maps an evicted expert to a slot now
    holding another."""
    monkeypatch.setattr(config, "FLOW_WARMUP", 1)
    monkeypatch.setattr(config, "FLOW_WARM_HIT", 0.0)
    monkeypatch.setattr(config, "FLOW_MAX_CRIT", 0.0)
    twin, layers, ring = build(3, 16, lag=2)
    ring.flow = True
    rng = np.random.default_rng(2)
    x2 = torch.zeros(1, 8)
    for t in range(4):                                  # warm up with rows in sync
        for s in layers:
            s.call(x2, routing(rng, 1), fake_compute(8))
    monkeypatch.setattr(twin, "sync_table", lambda layer_key: False)
    for t in range(16):
        for s in layers:
            s.call(x2, routing(rng, 1), fake_compute(8))
    assert {"OWNER-MISMATCH", "READ-BEFORE-LANDED"} & set(kinds(twin.ledger))


def test_flow_leaves_when_tokens_keep_missing_and_returns_when_warm(cpu_seam, monkeypatch):
    """Flow's exit (streaming.py:1585-1613 behaviour): tokens whose routing
    keeps missing push the missing-experts EMA over FLOW_MAX_CRIT, flow ends
    (its admitted copies installed, flow_drop), per-layer tokens follow; a
    hot routing brings the misses under half the bar and flow resumes.  The
    ledger stays clean throughout."""
    monkeypatch.setattr(config, "FLOW_WARMUP", 1)
    monkeypatch.setattr(config, "FLOW_WARM_HIT", 0.0)
    monkeypatch.setattr(config, "FLOW_MAX_CRIT", 5.0)
    twin, layers, ring = build(3, 16, lag=2)
    ring.flow = True
    rng = np.random.default_rng(3)
    x2 = torch.zeros(1, 8)
    hot = [routing(rng, 1) for _ in layers]
    modes = []
    for t in range(40):
        cold = 4 <= t < 16
        for i, s in enumerate(layers):
            s.call(x2, routing(rng, 1) if cold else hot[i], fake_compute(8))
        modes.append(ring.token_flow)
    assert any(modes[:4]) and not all(modes[4:20])          # flow on, then off under misses
    assert modes[-1] and ring._flow_backoff                  # and back once hot again
    assert twin.ledger.conflicts == [], twin.ledger.conflicts[:3]
