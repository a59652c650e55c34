"""A CPU stand-in for ExpertCache that emits the slot ledger's events.

Test infrastructure only.  Residency decisions come from the oracle's slot
policy (oracle.pmoe_oracle.SlotPolicy); each method emits the ledger events
of the native call it stands in for, in the order that call makes them
(pagedmoe_amd/csrc/slab.hip and copy_engine.cpp):

* fetch (pmoe_slab_fetch): settle handed-back guesses, the policy step
  (a guess whose slot is taken back is waited for), claimed guesses
  (completion query, batch join), copies queued, row upload, flush
  (fence, issue, join);
* fetch_prefill (pmoe_slab_fetch_prefill): policy step, copies queued and
  issued behind the latest fence;
* speculate (pmoe_slab_speculate): one copy and one batch per guess;
* flow_admit / flow_install_ready (ExpertCache): copies queued per layer,
  one fence and one batched issue; a batch joined once it has landed.

Copies are asynchronous: a copy completes ``lag`` compute-stream positions
after it was issued, and only a completion query (or a host wait) tells the
host so.  The StreamedSwitchGLU / PrefetchRing code under test drives this
twin exactly as it drives the real cache, so the ledger checks the
schedule that code produces.
"""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np

from oracle import pmoe_oracle as O
from pagedmoe_amd import verify as V
from pagedmoe_amd.cache import FlowBatch, PrefillGroup

DEMAND, SPEC, SLAB = 101, 102, 103


class TwinCache:
    def __init__(self, slots, layer_keys, n_experts, *, stage_slots=0, hidden=8,
                 reserve_frac=0.1, lag=3, expert_bytes=64 << 20):
        self.layer_keys = list(layer_keys)
        self._li = {k: i for i, k in enumerate(self.layer_keys)}
        self.n_experts = int(n_experts)
        self.routed_slots = int(slots)
        # expert_bytes only sizes the prefill fetch groups (64 MiB: groups of 8)
        self.geom = SimpleNamespace(hidden=hidden, inter=hidden, bits=4,
                                    expert_bytes=expert_bytes)
        self.pol = O.SlotPolicy(slots, reserve_frac)
        self.pol.set_stage(slots, stage_slots)
        self.pol.settle = self._settle_spec        # completion-aware hand-back
        self.reserve = self.pol.reserve
        self.stitched = False
        self.group_passes = 0
        self.spec_log = None
        self.lag = int(lag)
        self.ledger = V.SlotLedger(SLAB, [DEMAND, SPEC],
                                   lambda dst, src, n: (dst, divmod(src, self.n_experts)),
                                   print_conflicts=False)
        self._issued = {}          # (engine, batch) -> ledger position at issue
        self._done = set()         # (engine, batch) the host knows complete
        self._next_batch = {DEMAND: 0, SPEC: 0}
        self._queued = {DEMAND: 0, SPEC: 0}
        self.spec_batch = {}       # slot -> batch of the guess read into it
        self._published = {}       # layer -> row as last uploaded

    # ------------------------------------------------------------ events

    def emit(self, kind, who, a=0, b=0, c=0):
        self.ledger.feed([(kind, who, a, b, c)])

    def _submit(self, engine, slot, li, e):
        self.emit(V.SUBMIT, engine, slot, li * self.n_experts + e, 1)
        self._queued[engine] += 1

    def _issue(self, engine, batched):
        b = -1
        if batched:
            b = self._next_batch[engine]
            self._next_batch[engine] += 1
        if self._queued[engine]:
            self.emit(V.ISSUE, engine, b)
            self._queued[engine] = 0
        self._issued[(engine, b)] = self.ledger.pos
        return b

    def _batch_done(self, engine, b):
        key = (engine, b)
        done = key in self._done or self.ledger.pos - self._issued.get(key, -10 ** 9) >= self.lag
        if done:
            self._done.add(key)
            self.emit(V.HOST_DONE, engine, b)
        return done

    def _upload(self, li, row):
        self.emit(V.PUBLISH, SLAB, li)
        for e in np.nonzero(row >= 0)[0]:
            self.emit(V.ROW, SLAB, li, int(e), int(row[e]))
        self._published[li] = row.copy()

    def _settle_spec(self):
        keep = []
        for slot in self.pol.__dict__.setdefault("draining", []):
            b = self.spec_batch.get(slot)
            if b is None or self._batch_done(SPEC, b):
                self.pol.free.append(slot)
                self.spec_batch.pop(slot, None)
            else:
                keep.append(slot)
        self.pol.draining[:] = keep

    # ------------------------------------------------------------ tables

    def layer_index(self, layer_key):
        return self._li[layer_key]

    def host_table(self, layer_key):
        return self.pol.table(self._li[layer_key], self.n_experts)

    def table_ptr(self, layer_key):
        return self._li[layer_key]

    def sync_table(self, layer_key):
        li = self._li[layer_key]
        row = self.pol.table(li, self.n_experts)
        if li in self._published and np.array_equal(self._published[li], row):
            return False
        self._upload(li, row)
        return True

    def shared_slot(self, layer_key):
        return -1

    def raw_stats(self):
        return SimpleNamespace(hits=self.pol.hits, misses=self.pol.misses)

    def note_compute(self, layer_key):
        self.emit(V.COMPUTE, SLAB, self._li[layer_key])

    # ------------------------------------------------------------ decode

    def fetch(self, layer_key, expert_ids):
        li = self._li[layer_key]
        ids = sorted({int(e) for e in expert_ids})
        if self.spec_log is not None:
            self.spec_log.append(("fetch", layer_key, list(ids)))
        self._settle_spec()
        staged = dict(self.pol.__dict__.setdefault("staged", {}))
        hits, placed = self.pol.step(li, ids)
        for key, slot in staged.items():
            b = self.spec_batch.get(slot)
            if key[0] == li and key[1] in ids:           # claimed: the stream waits for it
                self._batch_done(SPEC, b)
                self.emit(V.BATCH_JOIN, SPEC, b)
                self.spec_batch.pop(slot, None)
            elif key not in self.pol.staged and slot not in self.pol.draining:
                self.emit(V.HOST_DONE, SPEC, b)           # taken back: the host waits for it
                self._done.add((SPEC, b))
                self.spec_batch.pop(slot, None)
        for e, slot in placed:
            self._submit(DEMAND, slot, li, e)
        self._upload(li, self.pol.table(li, self.n_experts))
        if placed:
            self.emit(V.FENCE, DEMAND)
            self._issue(DEMAND, False)
            self.emit(V.JOIN, DEMAND)
        return len(placed)

    # ------------------------------------------------------------ prefill

    def capacity(self):
        return (len(self.pol.free), len(self.pol.stage_free),
                max(0, self.pol.budget - len(self.pol.lru)))

    def fence(self):
        self.emit(V.FENCE, DEMAND)

    def join(self):
        self.emit(V.JOIN, DEMAND)

    def fetch_prefill(self, layer_key, expert_ids):
        li = self._li[layer_key]
        ids = sorted({int(e) for e in expert_ids})
        t, placed, nu = self.pol.step_prefill(li, ids)
        for e, slot in placed:
            self._submit(DEMAND, slot, li, e)
        self._issue(DEMAND, False)
        return PrefillGroup(t, ids, len(placed), nu)

    def publish_group(self, group):
        li = self.pol.groups[group.ticket]["layer"]
        self._upload(li, self.pol.compute_row(group.ticket, self.n_experts))

    def prefill_done(self, group):
        self.pol.prefill_done(group.ticket)

    # ------------------------------------------------------------ speculation

    def spec_fence(self):
        self.emit(V.FENCE, SPEC)

    def speculate(self, layer_key, expert_ids, max_staged=None):
        li = self._li[layer_key]
        cap = self.reserve if max_staged is None else int(max_staged)
        if self.spec_log is not None:
            self.spec_log.append(("speculate", layer_key, [int(e) for e in expert_ids], cap))
        got = self.pol.speculate(li, [int(e) for e in expert_ids], cap)
        for e, slot in got:
            self._submit(SPEC, slot, li, e)
            self.spec_batch[slot] = self._issue(SPEC, True)
        return len(got)

    def drop_staged(self):
        self.pol.drop_all_staged()

    def sync_spec(self):
        self.emit(V.HOST_SYNC, SPEC)
        for key in self._issued:
            if key[0] == SPEC:
                self._done.add(key)

    # ------------------------------------------------------------ flow

    def flow_admit(self, batch):
        items = []
        for i, (layer_key, ids) in enumerate(batch):
            li = self._li[layer_key]
            placed = self.pol.admit(li, ids, clear_pins=(i == 0))
            for e, slot in placed:
                self._submit(DEMAND, slot, li, e)
            if placed:
                items.append((layer_key, [e for e, _ in placed]))
        if not items:
            return None
        self.fence()
        return FlowBatch(self._issue(DEMAND, True), items)

    def flow_install_ready(self, batches, wait=False):
        left = []
        for fb in batches:
            if not wait and not self._batch_done(DEMAND, fb.batch):
                left.append(fb)
                continue
            self.emit(V.BATCH_JOIN, DEMAND, fb.batch)
            for layer_key, ids in fb.items:
                self.pol.install(self._li[layer_key], ids)
        return left
