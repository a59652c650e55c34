"""Expert residency over one HBM slab: slot table, pinned host store, paging.

Counterpart of the reference's ``ExpertCache`` slab path (cache.py:410).  The
policy itself is native (libpmoe ``pmoe_slab_*``): LRU with the LFRU second
chance, a reserve of free slots, pins for the experts of the current layer
step, and a full "stitch" when every expert fits (cache.py:717-787).  Misses
are copied from a pinned host expert store into their slots by the native copy
engine on side streams; the compute stream waits on events, never the host.
The reference's misses come from SSD preads; the host store stands in for the
page cache and is filled from a quantized safetensors checkpoint
(checkpoint.py) or from resident modules.
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import config
from ._lib import Geom, PmoeError, SlabStats, check, lib
from .slab import SlabStore


class HostExpertStore:
    """Pinned host memory holding every (layer, expert) in slot layout:
    expert e of layer l at ``((l * n_experts) + e) * expert_bytes``."""

    def __init__(self, g: Geom, n_layers: int, n_experts: int):
        self.geom = g
        self.n_layers = n_layers
        self.n_experts = n_experts
        self.expert_bytes = int(g.expert_bytes)
        self.nbytes = n_layers * n_experts * self.expert_bytes
        self._ptr = ctypes.c_void_p()
        check(lib().pmoe_host_alloc(ctypes.byref(self._ptr), self.nbytes), "pmoe_host_alloc")
        buf = (ctypes.c_uint8 * self.nbytes).from_address(self._ptr.value)
        self.bytes = np.frombuffer(buf, dtype=np.uint8)

    @classmethod
    def from_checkpoint(cls, model_dir, layers=None, group: int = 64) -> "HostExpertStore":
        """A store holding every expert of the MoE layers of a quantized
        safetensors checkpoint (stacked or per-expert layout), read straight
        from the files into slot layout (checkpoint.py).  ``layers`` keeps
        only those layer numbers; ``layer_numbers`` lists the store's layers
        in order."""
        from . import checkpoint as ck
        from ._lib import geom

        index = ck.read_headers(model_dir)
        found = ck.find_moe_layers(index)
        if layers is not None:
            keep = set(int(n) for n in layers)
            found = [f for f in found if f[0] in keep]
        if not found:
            raise PmoeError(f"{model_dir}: no quantized MoE expert tensors found")
        layouts = [ck.layer_layout(path, index) for _, path in found]
        hidden, inter, bits = layouts[0].geometry(group)
        g = geom(hidden, inter, bits, group)
        store = cls(g, len(layouts), layouts[0].n_experts)
        ck.fill_host_store(store, layouts, g)
        store.layer_numbers = [n for n, _ in found]
        return store

    @property
    def address(self) -> int:
        return self._ptr.value

    def expert_view(self, layer: int, e: int) -> np.ndarray:
        off = (layer * self.n_experts + e) * self.expert_bytes
        return self.bytes[off:off + self.expert_bytes]

    def write_from_slot(self, layer: int, e: int, slab: SlabStore, slot: int) -> None:
        """Copy one slot's bytes (device) into the store entry (host)."""
        host = torch.from_numpy(self.expert_view(layer, e))
        host.copy_(slab.slot_bytes(slot), non_blocking=False)

    def close(self) -> None:
        if self._ptr.value:
            self.bytes = None
            lib().pmoe_host_free(self._ptr)
            self._ptr = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# prefill-ahead stands down while the share of its reads the next layer
# routed stays under AHEAD_MIN_PRECISION (cache.py:237-243)
AHEAD_MIN_PRECISION = 0.5
AHEAD_MIN_SAMPLE = 512
AHEAD_DECAY = 0.98


def default_stage_slots(g: Geom, n_experts: int) -> int:
    """The prefill stage's size: four groups of PREFILL_STAGE_GROUP_MB (at
    least 8 experts a group) and at least 32 slots, as ensure_stage sizes it
    (cache.py:1358-1372), but never more than two layers' worth of experts:
    a group holds at most one layer's distinct experts and at most two groups
    are in flight (one computing, the next one's copies under it)."""
    if not config.PREFILL_STAGE:
        return 0
    per = max(1, int(g.expert_bytes))
    group = max(config.PREFILL_STAGE_GROUP_MB << 20, 8 * per)
    return min(max(32, (4 * group) // per), 2 * int(n_experts))


class PrefillGroup:
    """One prefill fetch group's held slots (a native ticket) and its copy
    counts."""

    __slots__ = ("ticket", "ids", "n_miss", "n_unplaced")

    def __init__(self, ticket: int, ids, n_miss: int, n_unplaced: int):
        self.ticket = ticket
        self.ids = list(ids)
        self.n_miss = n_miss
        self.n_unplaced = n_unplaced


class FlowBatch:
    """One token's admitted misses (flow decode): the copy batch that brings
    them in and the (layer key, expert ids) to install once it has landed."""

    __slots__ = ("batch", "items")

    def __init__(self, batch: int, items):
        self.batch = batch
        self.items = items


class ExpertCache:
    """Slot residency of the routed experts of ``layer_keys`` (E experts each)
    in a slab of ``slots`` routed slots, plus one pinned slot per layer for a
    shared expert when ``n_shared`` is 1, plus ``stage_slots`` prefill stage
    slots (default: ``default_stage_slots``) that never hold resident experts.

    Slab slot order: routed [0, slots), shared [slots, slots + layers),
    stage after those."""

    def __init__(self, g: Geom, slots: int, layer_keys, n_experts: int, *,
                 host_store: HostExpertStore | None = None, n_shared: int = 0,
                 reserve_frac: float | None = None, lfru: bool | None = None,
                 lfru_scan: int | None = None, stage_slots: int | None = None, device="cuda"):
        self.geom = g
        self.layer_keys = list(layer_keys)
        self._layer = {k: i for i, k in enumerate(self.layer_keys)}
        self.n_experts = int(n_experts)
        self.routed_slots = int(slots)
        self.n_shared = int(n_shared)
        self.stage_slots = (default_stage_slots(g, self.n_experts) if stage_slots is None
                            else int(stage_slots))
        self.stage_first = self.routed_slots + self.n_shared * len(self.layer_keys)
        self.slab = SlabStore(g, self.stage_first + self.stage_slots, device)
        self.host_store = host_store
        self._h = ctypes.c_void_p()
        check(lib().pmoe_slab_create(
            ctypes.byref(self._h), self.routed_slots, len(self.layer_keys), self.n_experts,
            config.SLAB_RESERVE_FRAC if reserve_frac is None else reserve_frac,
            int(config.LFRU if lfru is None else lfru),
            config.LFRU_SCAN if lfru_scan is None else lfru_scan), "pmoe_slab_create")
        check(lib().pmoe_slab_set_stage(self._h, self.stage_first, self.stage_slots),
              "pmoe_slab_set_stage")
        self._ce = ctypes.c_void_p()
        self._ce_spec = ctypes.c_void_p()
        if host_store is not None:
            check(lib().pmoe_copy_engine_create(ctypes.byref(self._ce), config.COPY_SPLIT_BYTES,
                                                config.COPY_STREAMS), "pmoe_copy_engine_create")
            # speculative reads get an engine (and stream) of their own, so a
            # demand copy never queues behind a guess on one stream
            check(lib().pmoe_copy_engine_create(ctypes.byref(self._ce_spec),
                                                config.COPY_SPLIT_BYTES, 1),
                  "pmoe_copy_engine_create")
            check(lib().pmoe_slab_set_spec_engine(self._h, self._ce_spec),
                  "pmoe_slab_set_spec_engine")
        self.reserve = max(4, int(self.routed_slots * (config.SLAB_RESERVE_FRAC
                                                       if reserve_frac is None else reserve_frac)))
        self.stitched = False
        self.group_passes = 0
        self.spec_log = None     # a list records fetch / speculate calls (tests replay them)
        self.ledger = None       # slot-safety ledger (config.SLAB_VERIFY)
        self._ahead_n = 0.0      # prefill-ahead reads started / used, decayed
        self._ahead_u = 0.0
        self.ahead_skipped = 0
        if config.SLAB_VERIFY:
            self.verify_slots(True)

    # ------------------------------------------------------------- slot safety

    def _locate(self, dst: int, src: int, nbytes: int):
        """(slot, (layer index, expert)) of a whole-expert copy into this
        slab, or None for other copies."""
        eb = int(self.geom.expert_bytes)
        off = dst - self.slab.data_ptr
        if nbytes != eb or off < 0 or off % eb or off // eb >= self.slab.slots:
            return None
        owner = None
        if self.host_store is not None:
            key, rem = divmod(src - self.host_store.address, eb)
            if rem == 0 and 0 <= key < self.host_store.n_layers * self.n_experts:
                owner = divmod(key, self.n_experts)
        return off // eb, owner

    def verify_slots(self, on: bool = True):
        """Start (or stop) replaying this cache's copy and compute ordering
        through a ``verify.SlotLedger`` (the reference's
        PAGED_MOE_SLAB_VERIFY).  Returns the ledger."""
        from . import verify

        if on and self.ledger is None:
            engines = [e.value for e in (self._ce, self._ce_spec) if e.value]
            self.ledger = verify.SlotLedger(self._h.value, engines, self._locate)
            verify.attach(self.ledger)
        elif not on and self.ledger is not None:
            verify.detach(self.ledger)
        return self.ledger

    def note_compute(self, layer_key) -> None:
        """A compute reading the layer's uploaded row has just been
        enqueued (a no-op unless the slot ledger is on)."""
        if self.ledger is None:
            return
        from . import verify

        check(lib().pmoe_ledger_note(verify.COMPUTE, self._h, self.layer_index(layer_key), 0, 0),
              "pmoe_ledger_note")
        verify.drain()

    @classmethod
    def from_budget(cls, budget_bytes: int, g: Geom, layer_keys, n_experts: int, **kw):
        """Size the slab from a byte budget, as the reference's
        ``ExpertCache(budget_bytes)`` + ``enable_slabs`` do (cache.py:421,
        :914-1006): slots = budget // expert_bytes."""
        slots = int(budget_bytes) // int(g.expert_bytes)
        if slots < 1:
            raise ValueError(f"budget {budget_bytes} B holds no {int(g.expert_bytes)} B expert")
        return cls(g, slots, layer_keys, n_experts, **kw)

    # ------------------------------------------------------------- tables

    def layer_index(self, layer_key) -> int:
        return self._layer[layer_key]

    def table_ptr(self, layer_key) -> int:
        """Device address of the layer's expert->slot row (int32 [E])."""
        p = lib().pmoe_slab_device_table(self._h, self.layer_index(layer_key))
        if not p:
            raise PmoeError(lib().pmoe_last_error().decode())
        return p

    def host_table(self, layer_key) -> np.ndarray:
        out = (ctypes.c_int32 * self.n_experts)()
        check(lib().pmoe_slab_host_table(self._h, self.layer_index(layer_key), out),
              "pmoe_slab_host_table")
        return np.array(out[:], np.int32)

    def flow_table(self, layer_key):
        """Device pointer of the layer's expert->slot row (-1 = not
        resident), republished first if its residency changed since the
        last upload -- e.g. another layer's fetch evicted one of its experts
        (the reference's flow_table, cache.py:843-859).  The upload is
        enqueued on the current stream."""
        self.sync_table(layer_key)
        return self.table_ptr(layer_key)

    def sync_table(self, layer_key) -> bool:
        """Republish the layer's device row if it is stale; True if it was."""
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        r = lib().pmoe_slab_sync_table(self._h, self.layer_index(layer_key), stream)
        if r < 0:
            check(r, "pmoe_slab_sync_table")
        return r == 1

    def device_table(self, layer_key) -> np.ndarray:
        """The layer's device row as the kernels see it (synchronises)."""
        out = (ctypes.c_int32 * self.n_experts)()
        check(lib().pmoe_slab_read_device_row(self._h, self.layer_index(layer_key), out),
              "pmoe_slab_read_device_row")
        return np.array(out[:], np.int32)

    def table_dirty(self, layer_key) -> bool:
        r = lib().pmoe_slab_dirty(self._h, self.layer_index(layer_key))
        if r < 0:
            check(r, "pmoe_slab_dirty")
        return r == 1

    def stitch_table(self, layer_key):
        return self.table_ptr(layer_key) if self.stitched else None

    def shared_slot(self, layer_key) -> int:
        if not self.n_shared:
            return -1
        return self.routed_slots + self.layer_index(layer_key)

    def publish(self, layer_key) -> None:
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        check(lib().pmoe_slab_publish(self._h, self.layer_index(layer_key), stream),
              "pmoe_slab_publish")

    # ------------------------------------------------------------- fetch

    def request(self, layer_key, expert_ids):
        """Policy step only: [(expert, slot)] of the misses that got a slot."""
        ids = [int(e) for e in expert_ids]
        arr = (ctypes.c_int32 * max(1, len(ids)))(*ids)
        mid = (ctypes.c_int32 * max(1, len(ids)))()
        msl = (ctypes.c_int32 * max(1, len(ids)))()
        nm = ctypes.c_int()
        check(lib().pmoe_slab_request(self._h, self.layer_index(layer_key), arr, len(ids), mid, msl,
                                      ctypes.byref(nm)), "pmoe_slab_request")
        return [(mid[i], msl[i]) for i in range(nm.value)]

    def fetch(self, layer_key, expert_ids) -> int:
        """One decode-layer fetch (cache.py:2525 on the slab path): classify,
        copy the misses from the host store into their slots, publish the
        table, and make the current stream wait for the copies.  Returns the
        number of misses copied."""
        if self.host_store is None:
            raise PmoeError("fetch needs a host expert store")
        ids = [int(e) for e in expert_ids]
        if self.spec_log is not None:
            self.spec_log.append(("fetch", layer_key, list(ids)))
        arr = (ctypes.c_int32 * max(1, len(ids)))(*ids)
        nm = ctypes.c_int()
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        check(lib().pmoe_slab_fetch(self._h, self._ce, ctypes.byref(self.geom),
                                    ctypes.c_void_p(self.slab.data_ptr),
                                    ctypes.c_void_p(self.host_store.address),
                                    self.layer_index(layer_key), arr, len(ids),
                                    ctypes.byref(nm), stream), "pmoe_slab_fetch")
        return nm.value

    # ------------------------------------------------------------- prefill

    def capacity(self):
        """(free routed slots, free stage slots, budget room)."""
        f, st, room = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        check(lib().pmoe_slab_capacity(self._h, ctypes.byref(f), ctypes.byref(st),
                                       ctypes.byref(room)), "pmoe_slab_capacity")
        return f.value, st.value, room.value

    def request_prefill(self, layer_key, expert_ids):
        """Policy step only (no copies): (ticket, [(miss id, slot)], unplaced)."""
        ids = [int(e) for e in expert_ids]
        arr = (ctypes.c_int32 * max(1, len(ids)))(*ids)
        mid = (ctypes.c_int32 * max(1, len(ids)))()
        msl = (ctypes.c_int32 * max(1, len(ids)))()
        nm, nu, t = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        check(lib().pmoe_slab_prefill_request(self._h, self.layer_index(layer_key), arr, len(ids),
                                              mid, msl, ctypes.byref(nm), ctypes.byref(nu),
                                              ctypes.byref(t)), "pmoe_slab_prefill_request")
        return t.value, [(mid[i], msl[i]) for i in range(nm.value)], nu.value

    def fence(self) -> None:
        """Copies issued from now on wait for everything queued so far on
        the current stream."""
        check(lib().pmoe_copy_fence(self._ce, self._stream()), "pmoe_copy_fence")

    def join(self) -> None:
        """The current stream waits for every copy issued so far."""
        check(lib().pmoe_copy_join(self._ce, self._stream()), "pmoe_copy_join")

    def fetch_prefill(self, layer_key, expert_ids) -> PrefillGroup:
        """One prefill fetch group (cache.py:2535-2578, _begin(prefill=True)):
        policy step, then its misses copied behind the latest fence; nothing
        waits for them yet.  Before the group computes: ``publish_group`` and
        ``join``; after its compute is enqueued: ``prefill_done``."""
        if self.host_store is None:
            raise PmoeError("fetch_prefill needs a host expert store")
        ids = sorted({int(e) for e in expert_ids})
        arr = (ctypes.c_int32 * max(1, len(ids)))(*ids)
        nm, nu, t = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        check(lib().pmoe_slab_fetch_prefill(self._h, self._ce, ctypes.byref(self.geom),
                                            ctypes.c_void_p(self.slab.data_ptr),
                                            ctypes.c_void_p(self.host_store.address),
                                            self.layer_index(layer_key), arr, len(ids),
                                            ctypes.byref(nm), ctypes.byref(nu), ctypes.byref(t)),
              "pmoe_slab_fetch_prefill")
        return PrefillGroup(t.value, ids, nm.value, nu.value)

    def publish_group(self, group: PrefillGroup) -> None:
        """Upload the group's compute row (resident + its held slots) on the
        current stream."""
        check(lib().pmoe_slab_prefill_publish(self._h, group.ticket, self._stream()),
              "pmoe_slab_prefill_publish")

    def prefill_done(self, group: PrefillGroup) -> None:
        check(lib().pmoe_slab_prefill_done(self._h, group.ticket), "pmoe_slab_prefill_done")

    # ------------------------------------------------------------- speculation

    def spec_fence(self) -> None:
        """Speculative reads issued from now on wait for everything queued
        so far on the current stream (recorded before a layer's compute, so
        the guesses it issues afterwards run under that compute)."""
        if self._ce_spec.value:
            check(lib().pmoe_copy_fence(self._ce_spec, self._stream()), "pmoe_copy_fence")

    def speculate(self, layer_key, expert_ids, max_staged: int | None = None) -> int:
        """Start speculative reads (prediction-driven prefetch,
        cache.py:2853) of expert_ids, in priority order, into free slots
        only; a guess is claimed by the layer's next fetch.  At most
        ``max_staged`` (default: the reserve) guesses are outstanding.
        Returns the reads started."""
        if not self._ce_spec.value:
            return 0
        ids = [int(e) for e in expert_ids]
        cap = self.reserve if max_staged is None else int(max_staged)
        if self.spec_log is not None:
            self.spec_log.append(("speculate", layer_key, list(ids), cap))
        arr = (ctypes.c_int32 * max(1, len(ids)))(*ids)
        n = ctypes.c_int()
        check(lib().pmoe_slab_speculate(self._h, ctypes.byref(self.geom),
                                        ctypes.c_void_p(self.slab.data_ptr),
                                        ctypes.c_void_p(self.host_store.address),
                                        self.layer_index(layer_key), arr, len(ids), cap,
                                        ctypes.byref(n)), "pmoe_slab_speculate")
        return n.value

    def prefill_group_experts(self) -> int:
        """Experts in one prefill fetch group (the stage's group size, at
        least 8 experts, at most GROUP_BYTES)."""
        per = int(self.geom.expert_bytes)
        return max(1, min(config.GROUP_BYTES,
                          max(config.PREFILL_STAGE_GROUP_MB << 20, 8 * per)) // per)

    def prefill_ahead(self, layer_key, expert_ids, free_floor: int | None = None,
                      stage_floor: int | None = None) -> int:
        """Start a later prefill layer's predicted reads (cache.py:2580-2650):
        ids in priority order into free routed slots while more than
        ``free_floor`` (default max(8, slots // 50)) stay free, then into
        prefill stage slots while more than ``stage_floor`` stay free for
        that layer's unpredicted misses (default one fetch group's worth, at
        most a quarter of the stage: the reference's stage holds four groups
        and keeps one back); never an eviction.  The reads run on the speculation engine behind its latest
        fence; that layer's prefill groups claim the ids they route and hand
        back the rest.  Stands down while fewer than half of the recent
        guesses were used (after AHEAD_MIN_SAMPLE of them).  Returns the reads
        started."""
        if not self._ce_spec.value or self.stitched:
            return 0
        if self._ahead_n >= AHEAD_MIN_SAMPLE and self._ahead_u < AHEAD_MIN_PRECISION * self._ahead_n:
            self.ahead_skipped += 1
            self._ahead_n *= AHEAD_DECAY
            self._ahead_u *= AHEAD_DECAY
            return 0
        if free_floor is None:
            free_floor = max(8, self.routed_slots // 50)
        if stage_floor is None:
            stage_floor = min(self.stage_slots // 4, self.prefill_group_experts())
        ids = [int(e) for e in expert_ids]
        arr = (ctypes.c_int32 * max(1, len(ids)))(*ids)
        n = ctypes.c_int()
        check(lib().pmoe_slab_prefill_ahead(self._h, ctypes.byref(self.geom),
                                            ctypes.c_void_p(self.slab.data_ptr),
                                            ctypes.c_void_p(self.host_store.address),
                                            self.layer_index(layer_key), arr, len(ids),
                                            int(free_floor), int(stage_floor), ctypes.byref(n)),
              "pmoe_slab_prefill_ahead")
        return n.value

    def note_ahead(self, started: int, used: int) -> None:
        """Precision bookkeeping of one prefill-ahead set (cache.py:2694-2696)."""
        self._ahead_n = self._ahead_n * AHEAD_DECAY + started
        self._ahead_u = self._ahead_u * AHEAD_DECAY + used

    def drop_staged(self) -> None:
        """Hand back every outstanding guess (flow decode, prefill)."""
        check(lib().pmoe_slab_drop_staged(self._h), "pmoe_slab_drop_staged")

    def sync_spec(self) -> None:
        """Block until every speculative read has landed."""
        if self._ce_spec.value:
            check(lib().pmoe_copy_sync(self._ce_spec), "pmoe_copy_sync")

    # ------------------------------------------------------------- flow

    def flow_admit(self, batch) -> FlowBatch | None:
        """Flow decode's residency update for one token (flow_admit,
        cache.py:861-910): ``batch`` = [(layer key, ids)] of the last token's
        routing.  Hits get recency and reuse credit; misses take slots
        (evicting) and are copied in from the host store as one copy batch
        behind a fence at the current stream's tail, with nothing waiting for
        it.  The caller must have waited for every kernel queued before (an
        evicted slot is overwritten) and installs the batch once it has
        landed (``flow_install_ready``).  None when nothing was admitted."""
        if self.host_store is None:
            raise PmoeError("flow_admit needs a host expert store")
        items = []
        eb = int(self.geom.expert_bytes)
        for i, (layer_key, ids) in enumerate(batch):
            ids = sorted({int(e) for e in ids})
            li = self.layer_index(layer_key)
            arr = (ctypes.c_int32 * max(1, len(ids)))(*ids)
            mid = (ctypes.c_int32 * max(1, len(ids)))()
            msl = (ctypes.c_int32 * max(1, len(ids)))()
            nm = ctypes.c_int()
            check(lib().pmoe_slab_admit(self._h, li, arr, len(ids), mid, msl, ctypes.byref(nm),
                                        int(i == 0)), "pmoe_slab_admit")
            placed = [(mid[j], msl[j]) for j in range(nm.value)]
            for e, slot in placed:
                check(lib().pmoe_copy_submit(
                    self._ce, ctypes.c_void_p(self.slab.data_ptr + slot * eb),
                    ctypes.c_void_p(self.host_store.address + (li * self.n_experts + e) * eb),
                    eb, 1), "pmoe_copy_submit")
            if placed:
                items.append((layer_key, [e for e, _ in placed]))
        if not items:
            return None
        self.fence()
        b = ctypes.c_int()
        check(lib().pmoe_copy_issue(self._ce, ctypes.byref(b)), "pmoe_copy_issue")
        return FlowBatch(b.value, items)

    def flow_install_ready(self, batches, wait: bool = False) -> list:
        """Install every admitted batch whose copies have landed (all of them
        with ``wait``): the current stream waits on the batch's copy events,
        then its experts become resident (table rows dirty, republished by
        ``sync_table``).  Returns the batches still in flight."""
        left = []
        stream = self._stream()
        for fb in batches:
            if not wait:
                r = lib().pmoe_copy_batch_done(self._ce, fb.batch)
                if r < 0:
                    check(r, "pmoe_copy_batch_done")
                if r == 0:
                    left.append(fb)
                    continue
            check(lib().pmoe_copy_batch_join(self._ce, fb.batch, stream), "pmoe_copy_batch_join")
            for layer_key, ids in fb.items:
                arr = (ctypes.c_int32 * len(ids))(*ids)
                check(lib().pmoe_slab_install(self._h, self.layer_index(layer_key), arr, len(ids)),
                      "pmoe_slab_install")
            check(lib().pmoe_copy_batch_release(self._ce, fb.batch), "pmoe_copy_batch_release")
        return left

    @staticmethod
    def _stream():
        return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def sync_copies(self) -> None:
        if self._ce.value:
            check(lib().pmoe_copy_sync(self._ce), "pmoe_copy_sync")

    def load_stitch(self) -> bool:
        """Pin every expert of every layer in slot layer*E + e when they all
        fit (cache.py:717-787); copies them from the host store."""
        if not config.STITCH:
            return False
        r = lib().pmoe_slab_stitch(self._h)
        if r < 0:
            check(r, "pmoe_slab_stitch")
        if r == 0:
            return False
        if self.host_store is not None:
            for layer_key in self.layer_keys:
                li = self.layer_index(layer_key)
                table = self.host_table(layer_key)
                for e in range(self.n_experts):
                    src = torch.from_numpy(self.host_store.expert_view(li, e))
                    self.slab.slot_bytes(int(table[e])).copy_(src, non_blocking=False)
        for layer_key in self.layer_keys:
            self.publish(layer_key)
        torch.cuda.current_stream().synchronize()
        self.stitched = True
        return True

    # ------------------------------------------------------------- stats

    def raw_stats(self) -> SlabStats:
        st = SlabStats()
        check(lib().pmoe_slab_stats_get(self._h, ctypes.byref(st)), "pmoe_slab_stats_get")
        return st

    @property
    def hits(self) -> int:
        return self.raw_stats().hits

    @property
    def misses(self) -> int:
        return self.raw_stats().misses

    @property
    def evictions(self) -> int:
        return self.raw_stats().evictions

    def stats(self) -> dict:
        """Residency counters in the reference's names (cache.py:2967-3061)."""
        st = self.raw_stats()
        total = st.hits + st.misses
        h2d = lib().pmoe_copy_bytes(self._ce) if self._ce.value else 0
        return {
            "hits": st.hits, "misses": st.misses, "hit_rate": st.hits / total if total else 0.0,
            "evictions": st.evictions, "slot_starved": st.starved, "slab_slots": st.slots,
            "slab_free": st.slots - st.resident, "resident": st.resident, "budget": st.budget,
            "reserve": st.reserve, "stitched": bool(st.stitched),
            "read_gb": st.bytes_copied / 1e9, "h2d_gb": h2d / 1e9,
            "group_passes": self.group_passes,
            "prefill_slot_reads": st.prefill_slot_reads, "prefill_installs": st.prefill_installs,
            "stage_reads": st.stage_reads, "prefill_slot_starved": st.prefill_starved,
            "stage_slots": st.stage_slots, "flow_admits": st.flow_admits,
            "spec_started": st.spec_started, "spec_claims": st.spec_claims,
            "spec_claims_late": st.spec_claims_late, "spec_dropped": st.spec_dropped,
            "prefill_ahead_reads": st.ahead_started, "prefill_ahead_used": st.ahead_claims,
            "prefill_ahead_skipped": self.ahead_skipped,
            "slab_conflicts": None if self.ledger is None else len(self.ledger.conflicts),
        }

    def close(self) -> None:
        if self.ledger is not None:
            self.verify_slots(False)
        if self._ce_spec.value:
            lib().pmoe_copy_sync(self._ce_spec)
            lib().pmoe_slab_drop_staged(self._h)
            lib().pmoe_slab_set_spec_engine(self._h, None)
            lib().pmoe_copy_engine_destroy(self._ce_spec)
            self._ce_spec = ctypes.c_void_p()
        if self._ce.value:
            lib().pmoe_copy_engine_destroy(self._ce)
            self._ce = ctypes.c_void_p()
        if self._h.value:
            lib().pmoe_slab_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
