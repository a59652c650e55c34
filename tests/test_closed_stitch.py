"""Closed stitch (pagedmoe_amd/closed.py) on the CPU: arming after warm
per-layer tokens, a kept attempt, a replay with the KV cache rewound by one
token, cooldown, disarming on a prompt -- driven through the cache twin
(tests/cache_twin.py) with the device miss counter stood in by a host count
over the twin's tables (reference behaviour: streaming.py:2691-2870)."""

import numpy as np
import pytest
import torch
from torch import nn

from pagedmoe_amd import closed as C, config, kernels as K
from pagedmoe_amd.ring import PrefetchRing
from pagedmoe_amd.streaming import StreamedSwitchGLU
from tests.cache_twin import TwinCache

E = 32


class KV:
    """A layer cache holding one float per token; trim(n) drops n."""

    def __init__(self):
        self.vals = []

    @property
    def offset(self):
        return len(self.vals)

    def trim(self, n):
        n = min(n, len(self.vals))
        del self.vals[len(self.vals) - n:]
        return n


class Model(nn.Module):
    """Layers of the seam only; the routing of each call comes from the
    test's schedule, and each layer appends its input's first value to its
    cache (so a rewind shows)."""

    def __init__(self, layers, schedule):
        super().__init__()
        self.seams = layers
        self.schedule = schedule
        self.calls = []

    def forward(self, x, cache=None):
        t = int(x[0, 0, 0].item())
        self.calls.append(t)
        for i, s in enumerate(self.seams):
            cache[i].vals.append(t)
            s.call(x.reshape(-1, 8), self.schedule[t][i], lambda ids, table: torch.zeros(
                ids.shape + (8,)))
        return x


@pytest.fixture
def closed_twin(monkeypatch):
    monkeypatch.setattr(K, "note_workspace_errors", lambda: None)
    monkeypatch.setattr(K, "raise_workspace_errors", lambda: None)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    monkeypatch.setattr(config, "STITCH_PARTIAL", True)
    keys = [f"layers.{i}.mlp.switch_mlp" for i in range(2)]
    twin = TwinCache(24, keys, E)
    seams = [StreamedSwitchGLU(k, None, twin) for k in keys]
    ring = PrefetchRing(seams, twin)
    ring.governor.set_mode("off")
    miss = {"n": 0}

    def begin():
        for s in seams:
            twin.sync_table(s.layer_key)
        miss["n"] = 0
        ring.closed_active = True

    def count(table, ids):                  # table is the twin's layer index
        row = twin.pol.table(int(table), E)
        miss["n"] += int(sum(1 for e in ids.reshape(-1).tolist() if row[e] < 0))

    def end():
        ring.closed_active = False
        return miss["n"]

    monkeypatch.setattr(ring, "begin_closed", begin)
    monkeypatch.setattr(ring, "count_missing", count)
    monkeypatch.setattr(ring, "end_closed", end)
    return twin, seams, ring


def ids(*e):
    return torch.tensor([list(e)], dtype=torch.int32)


def test_arm_keep_replay_cooldown(closed_twin, monkeypatch):
    twin, seams, ring = closed_twin
    hot = [ids(0, 1, 2, 3), ids(4, 5, 6, 7)]
    cold = [ids(20, 21, 22, 23), ids(24, 25, 26, 27)]
    schedule = {0: hot, 1: cold}
    model = Model(seams, schedule)
    model._pagedmoe_ring, model._pagedmoe_cache = ring, twin
    assert C.install(model) and C.install(model)
    kv = [KV(), KV()]
    tok = lambda t: torch.full((1, 1, 8), float(t))
    syncs = {"n": 0}
    orig = StreamedSwitchGLU.routed_ids

    def counted(self, indices):
        syncs["n"] += 1
        return orig(self, indices)

    monkeypatch.setattr(StreamedSwitchGLU, "routed_ids", counted)
    # token 0 misses (cold slab), then 4 warm tokens arm it
    for _ in range(1 + C.WARM_TOKENS):
        model(tok(0), cache=kv)
    assert ring.closed_armed and ring.closed_ok == 0
    n_sync = syncs["n"]
    model(tok(0), cache=kv)                          # a kept closed token: no per-layer sync
    assert ring.closed_ok == 1 and syncs["n"] == n_sync
    assert model.calls[-1] == 0 and kv[0].offset == 6
    model(tok(1), cache=kv)                          # cold experts: attempt, rewind, replay
    assert ring.closed_replay == 1 and model.calls[-2:] == [1, 1]
    assert kv[0].vals == [0] * 6 + [1] and kv[1].vals == [0] * 6 + [1]
    assert syncs["n"] == n_sync + 2                  # the replay ran per layer
    assert not ring.closed_armed and ring.closed_cooldown == C.COOLDOWN
    for _ in range(C.COOLDOWN):                      # cooldown: per-layer tokens only
        model(tok(0), cache=kv)
    assert ring.closed_ok == 1 and not ring.closed_armed
    for _ in range(C.WARM_TOKENS):
        model(tok(0), cache=kv)
    assert ring.closed_armed
    model(torch.zeros(1, 5, 8), cache=kv)            # a prompt disarms
    assert not ring.closed_armed
    C.uninstall(model)
    assert "forward" not in model.__dict__


def test_not_installed_when_off_or_stitched(closed_twin, monkeypatch):
    twin, seams, ring = closed_twin
    model = Model(seams, {})
    model._pagedmoe_ring, model._pagedmoe_cache = ring, twin
    monkeypatch.setattr(config, "STITCH_PARTIAL", False)
    assert not C.install(model)
    monkeypatch.setattr(config, "STITCH_PARTIAL", True)
    twin.stitched = True
    assert not C.install(model)


def test_caches_that_cannot_rewind_are_never_attempted(closed_twin):
    twin, seams, ring = closed_twin
    model = Model(seams, {0: [ids(0, 1, 2, 3), ids(4, 5, 6, 7)]})
    model._pagedmoe_ring, model._pagedmoe_cache = ring, twin
    assert C.install(model)

    class NoTrim(KV):
        trim = None

    kv = [NoTrim(), NoTrim()]
    for _ in range(10):
        model(torch.zeros(1, 1, 8), cache=kv)
    assert ring.closed_armed and ring.closed_ok == 0 and ring.closed_replay == 0
