"""Slot-safety ledger: does any slot write race a compute that reads it?

Counterpart of the reference's PAGED_MOE_SLAB_VERIFY (config.py:1467):
per-slot write-in-flight counters and ``check_slots`` (cache.py:554-556,
:1171-1206), which flag WRITE-WHILE-COMPUTE and OWNER-MISMATCH.  The
reference's writes are host preads into unified memory, so a counter of
writes in flight is the whole story there.  Here a write is an H2D copy on a
copy stream and a read is a kernel on the compute stream, ordered only by
events, so the check is a replay of the ordering events instead:

* the compute stream is a sequence of positions: each fence, join, row
  upload (PUBLISH) and compute advances it;
* a copy waits for its engine's latest fence (a position) and is waited for
  by the compute stream from the position of the first join that covers it,
  or is known complete once the host has seen it finish;
* a compute at position p reads every slot of its layer's uploaded row.

Violations:

* ``WRITE-WHILE-COMPUTE``: a copy into slot s issued while a compute queued
  at or after its fence may still read s;
* ``WRITE-OVER-WRITE``: a copy into s not ordered after the previous copy
  into s (neither joined before its fence nor seen complete);
* ``READ-BEFORE-LANDED``: a compute reads s before the stream has waited for
  the last copy into s;
* ``OWNER-MISMATCH``: a row maps expert e of layer l to slot s, but the last
  copy into s brought another (layer, expert).

Events come from libpmoe's ledger (``pmoe_ledger_*``; the copy engines and
the slab record theirs, ``ExpertCache.note_compute`` the computes) in call
order, on one compute stream.  ``SlotLedger.feed`` takes them as
(kind, who, a, b, c) tuples, so any event source can be checked.
"""

from __future__ import annotations

import ctypes
import weakref

FENCE, SUBMIT, ISSUE, JOIN, BATCH_JOIN, HOST_DONE, HOST_SYNC, PUBLISH, ROW, COMPUTE = range(1, 11)
KIND_NAMES = {FENCE: "FENCE", SUBMIT: "SUBMIT", ISSUE: "ISSUE", JOIN: "JOIN",
              BATCH_JOIN: "BATCH_JOIN", HOST_DONE: "HOST_DONE", HOST_SYNC: "HOST_SYNC",
              PUBLISH: "PUBLISH", ROW: "ROW", COMPUTE: "COMPUTE"}


class _Copy:
    __slots__ = ("slot", "owner", "fence", "joined", "done")

    def __init__(self, slot, owner):
        self.slot, self.owner = slot, owner
        self.fence = None      # compute-stream position the copy waits for
        self.joined = None     # first position at which the stream waits for it
        self.done = False      # the host saw it complete


class _Engine:
    __slots__ = ("fence", "queued", "open", "batches")

    def __init__(self):
        self.fence = None
        self.queued: list = []
        self.open: list = []       # issued, not yet joined or seen complete
        self.batches: dict = {}    # batch id -> copies of its latest issue


class SlotLedger:
    """Replays ledger events of one slab and the engines that fill it.

    ``locate(dst, src, nbytes)`` maps a copy to (slot, owner) -- owner being
    (layer index, expert) -- or None for a copy this ledger does not track.
    """

    def __init__(self, slab, engines, locate, print_conflicts: bool = True):
        self.slab = slab
        self.engines = {e: _Engine() for e in engines}
        self.locate = locate
        self.print_conflicts = print_conflicts
        self.pos = 0
        self.rows: dict = {}          # layer -> {expert: slot} as uploaded
        self.last_copy: dict = {}     # slot -> _Copy
        self.last_read: dict = {}     # slot -> position of the last compute reading it
        self.conflicts: list = []
        self.counts = {name: 0 for name in KIND_NAMES.values()}

    def owns(self, who) -> bool:
        return who == self.slab or who in self.engines

    def _flag(self, what: str, **kw) -> None:
        line = f"[slab] {what} " + " ".join(f"{k}={v}" for k, v in kw.items())
        self.conflicts.append(line)
        if self.print_conflicts:
            print(line, flush=True)

    def feed(self, events) -> None:
        for kind, who, a, b, c in events:
            if not self.owns(who):
                continue
            self.counts[KIND_NAMES.get(kind, str(kind))] += 1
            if who == self.slab:
                self._slab_event(kind, a, b, c)
            else:
                self._engine_event(self.engines[who], kind, a, b, c)

    # ------------------------------------------------------------ events

    def _slab_event(self, kind, layer, expert, slot) -> None:
        if kind == PUBLISH:
            self.pos += 1
            self.rows[layer] = {}
        elif kind == ROW:
            self.rows.setdefault(layer, {})[expert] = slot
        elif kind == COMPUTE:
            self.pos += 1
            for e, s in self.rows.get(layer, {}).items():
                cp = self.last_copy.get(s)
                if cp is not None:
                    if not cp.done and (cp.joined is None or cp.joined >= self.pos):
                        self._flag("READ-BEFORE-LANDED", layer=layer, expert=e, slot=s,
                                   at=self.pos)
                    if cp.owner is not None and cp.owner != (layer, e):
                        self._flag("OWNER-MISMATCH", layer=layer, expert=e, slot=s,
                                   holds=cp.owner, at=self.pos)
                self.last_read[s] = self.pos

    def _engine_event(self, eng: _Engine, kind, a, b, c) -> None:
        if kind == FENCE:
            self.pos += 1
            eng.fence = self.pos
        elif kind == SUBMIT:
            where = self.locate(a, b, c)
            if where is not None:
                eng.queued.append(_Copy(*where))
        elif kind == ISSUE:
            for cp in eng.queued:
                cp.fence = eng.fence
                s = cp.slot
                r = self.last_read.get(s)
                if r is not None and (cp.fence is None or r >= cp.fence):
                    self._flag("WRITE-WHILE-COMPUTE", slot=s, owner=cp.owner, fence=cp.fence,
                               read_at=r)
                prev = self.last_copy.get(s)
                if prev is not None and not prev.done and not (
                        prev.joined is not None and cp.fence is not None
                        and prev.joined < cp.fence):
                    self._flag("WRITE-OVER-WRITE", slot=s, owner=cp.owner, prev=prev.owner)
                self.last_copy[s] = cp
            eng.open.extend(eng.queued)
            if a >= 0:
                eng.batches[a] = list(eng.queued)
            eng.queued = []
        elif kind == JOIN:
            self.pos += 1
            for cp in eng.open:
                if cp.joined is None:
                    cp.joined = self.pos
            eng.open = []
        elif kind == BATCH_JOIN:
            self.pos += 1
            for cp in eng.batches.get(a, ()):
                if cp.joined is None:
                    cp.joined = self.pos
        elif kind == HOST_DONE:
            for cp in eng.batches.get(a, ()):
                cp.done = True
        elif kind == HOST_SYNC:
            for cp in eng.open:
                cp.done = True
            for cps in eng.batches.values():
                for cp in cps:
                    cp.done = True
            eng.open = []

    def report(self) -> dict:
        return {"conflicts": len(self.conflicts), "first": self.conflicts[:5],
                "events": dict(self.counts)}


# ---------------------------------------------------------------- native log

_ledgers: "weakref.WeakSet" = weakref.WeakSet()


def attach(ledger: SlotLedger) -> None:
    """Route native ledger events to ``ledger`` (recording starts with the
    first attached ledger)."""
    from ._lib import check, lib

    if not len(_ledgers):
        check(lib().pmoe_ledger_enable(1), "pmoe_ledger_enable")
    _ledgers.add(ledger)


def detach(ledger: SlotLedger) -> None:
    from ._lib import lib

    drain()
    _ledgers.discard(ledger)
    if not len(_ledgers):
        lib().pmoe_ledger_enable(0)


def drain() -> int:
    """Move every recorded event to the attached ledgers that own it."""
    from ._lib import LedgerRec, PmoeError, lib

    cap = 1 << 15
    buf = (LedgerRec * cap)()
    n = ctypes.c_int()
    total = 0
    ledgers = list(_ledgers)
    while True:
        dropped = lib().pmoe_ledger_drain(buf, cap, ctypes.byref(n))
        if dropped < 0:
            raise PmoeError(lib().pmoe_last_error().decode())
        if dropped > 0:
            raise PmoeError(f"slot ledger overflowed: {dropped} events lost")
        events = [(r.kind, r.who, r.a, r.b, r.c) for r in buf[:n.value]]
        for led in ledgers:
            led.feed(events)
        total += n.value
        if n.value < cap:
            return total
